"""Invariants of the compiled kernels that the source relies on but cannot state in C++.

The backward key-tile kernel keeps its dK and dV accumulators in fixed accumulation registers
a[0:127]; every instruction that touches them is written out by hand (recir_amd/csrc/hstu_bwd_acc_regs.h).
That is only correct while the compiler itself places no AGPR instruction in that kernel (no MFMA of its
own, no VGPR spilled to an AGPR).  The device assembly is generated here and checked for it; needs
hipcc, no GPU.
"""
import os
import re
import shutil
import subprocess

import pytest

from recir_amd import build


@pytest.fixture(scope="module")
def device_asm(tmp_path_factory):
    if not (shutil.which("hipcc") or os.path.exists("/opt/rocm/bin/hipcc")):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "hstu_attn.s"
    cmd = [a for a in build.compile_command(str(out)) if a not in ("-fPIC", "-shared")] + ["-S", "--cuda-device-only"]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert res.returncode == 0, res.stdout[-2000:]
    return out.read_text()


def _kernels(asm, name_part):
    """(mangled name, body lines) of every kernel whose name contains name_part."""
    found = []
    lines = asm.splitlines()
    i = 0
    while i < len(lines):
        m = re.match(r"^(_Z\w*" + name_part + r"\w*):", lines[i])
        if m:
            j = i + 1
            while j < len(lines) and not lines[j].startswith(".Lfunc_end"):  # (a kernel may end in several places)
                j += 1
            found.append((m.group(1), lines[i:j + 1]))
            i = j
        i += 1
    return found


def test_key_tile_kernel_accumulators_are_untouched_by_the_compiler(device_asm):
    kernels = _kernels(device_asm, "hstu_bwd_dkv_d128")
    assert len(kernels) == 8  # semi-local x bias x per-token scale
    for name, body in kernels:
        in_asm = False
        hand_mfma = hand_acc = 0
        for line in body:
            if "#ASMSTART" in line:
                in_asm = True
            elif "#ASMEND" in line:
                in_asm = False
            text = line.split(";")[0]
            touches_agpr = "v_accvgpr" in text or re.search(r"\ba\[?\d", text) is not None
            if touches_agpr:
                assert in_asm, f"{name}: the compiler placed an AGPR instruction: {line.strip()}"
                hand_acc += 1
            if "v_mfma" in text:
                assert in_asm, f"{name}: an MFMA the compiler placed: {line.strip()}"
                hand_mfma += 1
        # tile bodies of 64 products each: two LDS stages x (unmasked, masked), and for the semi-local
        # instantiations a third mask form
        bodies = 6 if "hstu_bwd_dkv_d128ILb1E" in name else 4
        assert hand_mfma == 64 * bodies, (name, hand_mfma)
        assert hand_acc >= 128 + 128 + 128, (name, hand_acc)  # clear, accumulate, read back


def test_key_tile_kernel_register_budget(device_asm):
    """128 accumulation registers are declared for it, nothing spills, one wave per SIMD fits."""
    meta = re.findall(r"\.agpr_count:\s+(\d+).*?\.name:\s+(\S+).*?\.vgpr_count:\s+(\d+)\s+\.vgpr_spill_count:\s+(\d+)",
                      device_asm, flags=re.S)
    rows = [(n, int(a), int(v), int(sp)) for a, n, v, sp in meta if "hstu_bwd_dkv_d128" in n]
    assert len(rows) == 8
    for name, agprs, total, spills in rows:
        assert agprs == 128, (name, agprs)
        assert spills == 0, (name, spills)
        assert total <= 512, (name, total)
