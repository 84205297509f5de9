"""Build step: compiles the HIP sources into ``recir_amd/librecir_hstu.so`` for gfx950."""
from __future__ import annotations

import os
import shutil
import subprocess

_PKG = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_PKG)
LIB_PATH = os.path.join(_PKG, "librecir_hstu.so")
# the same sources with the forward kernel's phase stamps compiled in (bench.py --phase-trace); never
# loaded by the operators
TRACE_LIB_PATH = os.path.join(_PKG, "librecir_hstu_trace.so")
SOURCES = [os.path.join(_PKG, "csrc", n) for n in ("hstu_attn.hip", "hstu_mfma_any.hip", "hstu_mfma_any_rab.hip", "hstu_mfma_any_elems.hip", "hstu_mfma_any_elems_rab.hip")]


def hipcc_path() -> str:
    return shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _common_flags(trace: bool, defines) -> list:
    return [
        "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
        # no compiler-generated packed fp32 arithmetic
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
        "-I", os.path.join(_ROOT, "include"),
        *(["-DHSTU_TRACE=1"] if trace else []), *defines,
    ]


def compile_commands(out: str = LIB_PATH, trace: bool = False, defines=(), obj_dir: str = "") -> list:
    """One compile command per source (they run side by side) and the link command, last."""
    objs = [os.path.join(obj_dir, os.path.splitext(os.path.basename(s))[0] + ".o") for s in SOURCES]
    flags = _common_flags(trace, defines)
    cmds = [[hipcc_path(), *flags, "-c", src, "-o", obj] for src, obj in zip(SOURCES, objs)]
    cmds.append([hipcc_path(), "--offload-arch=gfx950", "-fPIC", "-shared", *objs, "-o", out])
    return cmds


def build_library(verbose: bool = False, trace: bool = False, defines=()) -> str:
    """Always recompiles (a minute or two); returns the path of the shared library.  ``trace=True``
    builds the phase-trace variant instead."""
    import tempfile
    from concurrent.futures import ThreadPoolExecutor

    out = TRACE_LIB_PATH if trace else LIB_PATH
    noise = "is not a recognized feature for this target"

    def run(cmd):
        res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        log = "\n".join(l for l in res.stdout.splitlines() if noise not in l)
        if res.returncode != 0:
            raise RuntimeError("hipcc failed:\n" + log)
        return log

    with tempfile.TemporaryDirectory(prefix="recir_hstu_build_") as obj_dir:
        *compiles, link = compile_commands(out, trace, defines, obj_dir)
        with ThreadPoolExecutor(max_workers=len(compiles)) as pool:
            logs = list(pool.map(run, compiles))
        logs.append(run(link))
    if verbose and any(l.strip() for l in logs):
        print("\n".join(l for l in logs if l.strip()))
    return out


if __name__ == "__main__":
    import sys

    # usage: python -m recir_amd.build [--trace] [-DNAME=VALUE ...]   (measurement builds of the kernels' switches)
    print(build_library(verbose=True, trace="--trace" in sys.argv[1:], defines=[a for a in sys.argv[1:] if a.startswith("-D")]))
