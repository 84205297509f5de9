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
    return _device_asm_of(tmp_path_factory, "hstu_attn")


def _device_asm_of(tmp_path_factory, unit):
    """Device assembly of one translation unit of the library, with the library's own compile flags."""
    out = tmp_path_factory.mktemp("asm") / (unit + ".s")
    compiles = build.compile_commands(obj_dir=str(out.parent))[:-1]
    (cmd,) = [c for c in compiles if os.path.basename(c[c.index("-c") + 1]) == unit + ".hip"]
    cmd = [a for a in cmd[:cmd.index("-o")] if a not in ("-fPIC", "-c")] + ["-S", "--cuda-device-only", "-o", str(out)]
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


def _vgprs(text):
    """Indices of the VGPRs an instruction's operands name (v7, v[12:27]); AGPRs are not meant."""
    regs = set()
    for a, b in re.findall(r"(?<![\w\]])v\[(\d+):(\d+)\]", text):
        regs.update(range(int(a), int(b) + 1))
    for a in re.findall(r"(?<![\w\[])v(\d+)\b", text):
        regs.add(int(a))
    return regs


def test_nothing_the_compiler_placed_touches_a_hand_written_score_product_before_its_wait(device_asm):
    """The score products of the key-tile kernel are MFMAs written as assembly with VGPR results; the
    compiler's hazard recogniser does not see them, so the wait an MFMA result needs before another
    instruction may read it is written by hand too (an ``s_nop 15`` behind each chain).  That only
    holds while the compiler places no instruction of its own that names those result registers
    between the chain's first MFMA and that wait -- a copy, a spill -- which is checked here."""
    kernels = _kernels(device_asm, "hstu_bwd_dkv_d128")
    assert len(kernels) == 8
    for name, body in kernels:
        in_asm = False
        pending = set()   # result VGPRs of hand MFMAs whose wait has not been seen yet
        chains = waits = 0
        for line in body:
            if "#ASMSTART" in line:
                in_asm = True
                continue
            if "#ASMEND" in line:
                in_asm = False
                continue
            text = line.split(";")[0].strip()
            if not text or text.startswith("."):
                continue
            if in_asm:
                m = re.match(r"v_mfma_f32_32x32x16_bf16\s+v\[(\d+):(\d+)\]", text)
                if m:
                    if not pending:
                        chains += 1
                    pending.update(range(int(m.group(1)), int(m.group(2)) + 1))
                elif text.startswith("s_nop 15"):
                    waits += 1
                    pending.clear()
                continue
            if pending:
                operands = text.split(None, 1)[1] if " " in text else ""
                hit = _vgprs(operands) & pending
                assert not hit, f"{name}: `{text}` names v{sorted(hit)[:4]} while a hand-written MFMA into them has no wait yet"
        assert chains >= 4 and waits >= chains, (name, chains, waits)
        assert not pending, f"{name}: a chain of score products without its wait"
