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
SOURCES = [os.path.join(_PKG, "csrc", "hstu_attn.hip")]


def hipcc_path() -> str:
    return shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def compile_command(out: str = LIB_PATH, trace: bool = False, defines=()) -> list:
    return [
        hipcc_path(), "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
        # no compiler-generated packed fp32 arithmetic
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
        "-I", os.path.join(_ROOT, "include"),
        *(["-DHSTU_TRACE=1"] if trace else []), *defines,
        *SOURCES, "-o", out,
    ]


def build_library(verbose: bool = False, trace: bool = False, defines=()) -> str:
    """Always recompiles (a minute); returns the path of the shared library.  ``trace=True`` builds
    the phase-trace variant instead."""
    out = TRACE_LIB_PATH if trace else LIB_PATH
    cmd = compile_command(out, trace, defines)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    noise = "is not a recognized feature for this target"
    log = "\n".join(l for l in res.stdout.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + log)
    if verbose and log.strip():
        print(log)
    return out


if __name__ == "__main__":
    import sys

    # usage: python -m recir_amd.build [--trace] [-DNAME=VALUE ...]   (measurement builds of the kernels' switches)
    print(build_library(verbose=True, trace="--trace" in sys.argv[1:], defines=[a for a in sys.argv[1:] if a.startswith("-D")]))
