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


def _obj(obj_dir: str, src: str, suffix: str = "") -> str:
    return os.path.join(obj_dir, os.path.splitext(os.path.basename(src))[0] + suffix + ".o")


def compile_commands(out: str = LIB_PATH, trace: bool = False, defines=(), obj_dir: str = "") -> list:
    """One compile command per source (they run side by side) and the link command, last."""
    objs = [_obj(obj_dir, s) for s in SOURCES]
    flags = _common_flags(trace, defines)
    cmds = [[hipcc_path(), *flags, "-c", src, "-o", obj] for src, obj in zip(SOURCES, objs)]
    cmds.append([hipcc_path(), "--offload-arch=gfx950", "-fPIC", "-shared", *objs, "-o", out])
    return cmds


def _run_all(compiles, links, verbose: bool) -> None:
    from concurrent.futures import ThreadPoolExecutor

    noise = "is not a recognized feature for this target"

    def run(cmd):
        res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        log = "\n".join(l for l in res.stdout.splitlines() if noise not in l)
        if res.returncode != 0:
            raise RuntimeError("hipcc failed:\n" + log)
        return log

    with ThreadPoolExecutor(max_workers=min(len(compiles), os.cpu_count() or 4)) as pool:
        logs = list(pool.map(run, compiles))
    logs += [run(link) for link in links]
    if verbose and any(l.strip() for l in logs):
        print("\n".join(l for l in logs if l.strip()))


def build_library(verbose: bool = False, trace: bool = False, defines=()) -> str:
    """Always recompiles (a minute or two); returns the path of the shared library.  ``trace=True``
    builds the phase-trace variant instead."""
    import tempfile

    out = TRACE_LIB_PATH if trace else LIB_PATH
    with tempfile.TemporaryDirectory(prefix="recir_hstu_build_") as obj_dir:
        *compiles, link = compile_commands(out, trace, defines, obj_dir)
        _run_all(compiles, [link], verbose)
    return out


def build_both(verbose: bool = False) -> tuple:
    """The library and its phase-trace variant in one go.  Only the first source reads HSTU_TRACE (the
    head-dim-128 forward kernel's phase stamps and the entry points that hand it the trace buffer): it is
    compiled twice, the translation units of the general MFMA kernels once, and their objects go into both
    libraries.  Returns the two paths."""
    import tempfile

    traced, shared = SOURCES[:1], SOURCES[1:]
    with tempfile.TemporaryDirectory(prefix="recir_hstu_build_") as obj_dir:
        compiles, links = [], []
        shared_objs = [_obj(obj_dir, s) for s in shared]
        compiles += [[hipcc_path(), *_common_flags(False, ()), "-c", src, "-o", obj] for src, obj in zip(shared, shared_objs)]
        for trace, out in ((False, LIB_PATH), (True, TRACE_LIB_PATH)):
            objs = [_obj(obj_dir, s, "_trace" if trace else "") for s in traced]
            compiles += [[hipcc_path(), *_common_flags(trace, ()), "-c", src, "-o", obj] for src, obj in zip(traced, objs)]
            links.append([hipcc_path(), "--offload-arch=gfx950", "-fPIC", "-shared", *objs, *shared_objs, "-o", out])
        # the longest compilations first
        compiles.sort(key=lambda c: 0 if "elems" in c[-3] else 1)
        _run_all(compiles, links, verbose)
    return LIB_PATH, TRACE_LIB_PATH


if __name__ == "__main__":
    import sys

    # usage: python -m recir_amd.build [--trace | --both] [-DNAME=VALUE ...]   (measurement builds of the kernels' switches)
    if "--both" in sys.argv[1:]:
        print(*build_both(verbose=True))
    else:
        print(build_library(verbose=True, trace="--trace" in sys.argv[1:], defines=[a for a in sys.argv[1:] if a.startswith("-D")]))
