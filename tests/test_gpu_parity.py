"""GPU parity tests: the HIP kernels, called through the C ABI (via the operator), against the CPU
oracle on identical seeded inputs, against the reference's golden vectors, and through
size-independent properties at the benchmark's full sizes.

Tolerances: fp32 kernel rtol 2e-4 / atol 2e-6 (the reference's own kernel-test range, 1e-5..2e-4);
bf16 max-abs 1e-2 and 2e-2 relative (to the largest reference magnitude and in Frobenius norm);
mask, offsets and tail rows bit-exact.
"""
import os

import numpy as np
import pytest
import torch

from tests.golden.cases import SMALL_CASES, build_inputs, fixture_file
from tests.parity_util import (BF16_REL, FP8_MAX_ABS, expected_kernel, FP32_ATOL, FP32_RTOL, assert_bf16_close, assert_same_zero_structure,
                               error_stats, run_hip, run_oracle, to_device)

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu_and_library():
    from recir_amd import _lib

    assert torch.cuda.is_available(), "these tests need the MI355X"
    _lib.load()  # raises if the HIP library is missing: nothing else can compute the operator


def _case_scale(scale):
    return scale


@pytest.mark.parametrize("name", sorted(SMALL_CASES))
def test_small_cases_match_reference_golden(oracle, name):
    import recir_amd
    from recir_amd import ops

    case = SMALL_CASES[name]
    golden = np.load(os.path.join(GOLDEN, fixture_file(case)))[name]
    wl, scale, nt = build_inputs(case)
    ntd = None if nt is None else nt.cuda()
    # goldens with ctx > 0 pin the reference's contextual rule
    with ops.reference_contextual_rule():
        out = run_hip(wl, attn_scale=scale, num_targets=ntd, dtype="fp32")
    end = int(wl.seq_offsets[-1])
    np.testing.assert_allclose(out[:end].cpu().numpy(), golden, rtol=FP32_RTOL, atol=FP32_ATOL)
    assert not out[end:].cpu().numpy().any()
    assert out.shape == (wl.T, wl.H, wl.v.shape[2]) and out.dtype == torch.float32
    if case["bf16_inputs"]:
        with ops.reference_contextual_rule():
            outb = run_hip(wl, attn_scale=scale, num_targets=ntd, dtype="bf16")
        assert outb.dtype == torch.bfloat16
        assert_bf16_close(outb[:end], golden, name)
        assert not outb[end:].float().cpu().numpy().any()
        from recir_amd import _lib
        # a mask type other than the causal one, or a head dim other than 128, runs on the general MFMA kernel
        assert _lib.last_kernel() == expected_kernel(case["Dqk"], case["Dv"], causal=case["mask_type"] == "lower_triangular")


def test_config1_smoke_shape_fp32(oracle):
    from recir_amd.workloads import make_config

    wl = make_config(1)
    out = run_hip(wl)
    ref = run_oracle(oracle, wl)
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=FP32_RTOL, atol=FP32_ATOL)


@pytest.mark.parametrize("config", [2, 3, 4])
def test_full_size_configs_match_oracle(oracle, config):
    from recir_amd import _lib
    from recir_amd.workloads import make_config

    wl = make_config(config)
    out = run_hip(wl)
    assert _lib.last_kernel().startswith("tiled_d128")
    ref = run_oracle(oracle, wl)
    st = assert_bf16_close(out, ref, f"config{config}")
    print(f"config{config}: {st}")
    assert_same_zero_structure(out, ref, int(wl.seq_offsets[-1]))
    if config in (2, 4):  # the reference operator's own numbers at this size
        fx = np.load(os.path.join(GOLDEN, f"config{config}.npz"))
        assert_bf16_close(out[torch.from_numpy(fx["rows"]).cuda()], fx["row_values"], "golden rows")


@pytest.mark.parametrize("config", [2, 3])
def test_tiled_and_generic_kernels_agree(oracle, config):
    """Tiling invariance (the idea of recir/ops/pallas/tests/test_hstu_attention.py:76-89): the
    one-wave-per-row kernel and the tiled MFMA kernel see the same mask and agree in value."""
    from recir_amd import _lib, ops
    from recir_amd.workloads import make_jagged

    wl = make_jagged([300, 129, 64, 1, 0, 517], [40, 129, 0, 0, 0, 6], 2, 128, 128, max_seq_len=600,
                     alpha=1.0 / 128, dtype="bf16", seed=config, with_rab=(config == 3),
                     contextual_seq_len=8 if config == 3 else 0, tail_rows=7)
    with ops.force_kernel(ops.KERNEL_TILED_DIRECT):
        a = run_hip(wl)
        assert _lib.last_kernel().startswith("tiled_d128")
    with ops.force_kernel(ops.KERNEL_MFMA_GENERAL):
        a2 = run_hip(wl)
        assert _lib.last_kernel() == "mfma_bf16_d128"
    # two tilings with their own order of the elementwise arithmetic: equal to bf16 rounding of P
    assert error_stats(a2, a.float().cpu().numpy())["rel_to_max"] <= 2 ** -7
    with ops.force_kernel(ops.KERNEL_GENERIC):
        b = run_hip(wl)
        assert _lib.last_kernel() == "generic_bf16"
    ref = run_oracle(oracle, wl)
    assert_bf16_close(a, ref, "tiled")
    assert_bf16_close(b, ref, "generic")
    za = ~a.float().cpu().numpy().reshape(wl.T, -1).any(axis=1)
    zb = ~b.float().cpu().numpy().reshape(wl.T, -1).any(axis=1)
    np.testing.assert_array_equal(za, zb)


@pytest.mark.parametrize("kernel", ["tiled", "mfma_general", "generic"])
@pytest.mark.parametrize("ctx", [0, 5, 200])
def test_mask_is_bit_exact(oracle, kernel, ctx):
    """Positive constant scores and one-hot values make out[m, c] non-zero exactly when row m keeps a
    key j with j % 128 == c: the zero pattern of the output is the mask, compared exactly."""
    from recir_amd import ops
    from recir_amd.workloads import make_jagged

    lengths = [330, 128, 65, 1, 0, 191, 127]
    targets = [70, 128, 1, 0, 0, 64, 200]
    wl = make_jagged(lengths, targets, 1, 128, 128, max_seq_len=400, alpha=1.0 / 128, dtype="bf16",
                     contextual_seq_len=ctx, tail_rows=9)
    wl.q.fill_(0.5)
    wl.k.fill_(0.25)
    wl.v.zero_()
    off = wl.seq_offsets.numpy()
    for b, n in enumerate(lengths):
        for j in range(n):
            wl.v[off[b] + j, 0, j % 128] = 1.0
    variant = {"tiled": ops.KERNEL_TILED_DIRECT, "mfma_general": ops.KERNEL_MFMA_GENERAL, "generic": ops.KERNEL_GENERIC}[kernel]
    with ops.force_kernel(variant):
        out = run_hip(wl).float().cpu().numpy()
    want = np.zeros((wl.T, 128), dtype=bool)
    for b, (n, t) in enumerate(zip(lengths, targets)):
        for m in range(n):
            for j in range(n):
                if oracle.keep(m, j, n, t, ctx):
                    want[off[b] + m, j % 128] = True
    np.testing.assert_array_equal(out[:, 0, :] != 0, want)


def test_kept_key_count_per_row_is_exact(oracle):
    """Constant scores and v = 1: out[m] = unit * (#kept keys of row m); counts up to 2048 are
    recovered exactly by rounding, at the benchmark's sequence lengths."""
    from recir_amd.workloads import make_config

    wl = make_config(2)
    wl.q.fill_(0.5)
    wl.k.fill_(0.25)
    wl.v.fill_(1.0)
    out = run_hip(wl, dtype="bf16").float().cpu().numpy()
    c = wl.alpha * 128 * 0.5 * 0.25
    # P' = S sigmoid(alpha S) is rounded to bf16 once; use the kernel's own first-row value as unit
    off = wl.seq_offsets.numpy()
    unit = out[off[0], 0, 0]
    assert abs(unit - c / (1 + np.exp(-c)) / wl.max_seq_len) <= 1e-2 * unit
    for b in range(wl.B):
        n, t = int(wl.lengths[b]), int(wl.num_targets[b])
        cap = n - t
        want = np.array([m + 1 if m < cap else cap + 1 for m in range(n)], dtype=np.float64)
        got = out[off[b]:off[b] + n, :, :].astype(np.float64) / unit
        # bf16 output rounding: 8 significant bits => relative 2^-8
        assert np.all(np.abs(got - want[:, None, None]) <= want[:, None, None] * 2.0 ** -7 + 1e-3)


def test_properties_at_full_size(oracle):
    from recir_amd.workloads import make_config

    wl = make_config(2)
    q, k, v, off, nt = to_device(wl)
    import recir_amd

    kw = dict(max_seq_len=wl.max_seq_len, alpha=wl.alpha)
    base = recir_amd.jagged_hstu_attention(q, k, v, off, nt, **kw).float()
    # q = 0 or k = 0 => exact zeros (silu(0) = 0); the reference's own known-answer test
    assert not recir_amd.jagged_hstu_attention(torch.zeros_like(q), k, v, off, nt, **kw).any()
    assert not recir_amd.jagged_hstu_attention(q, torch.zeros_like(k), v, off, nt, **kw).any()
    # linear in v: doubling v doubles the output exactly (power of two)
    dbl = recir_amd.jagged_hstu_attention(q, k, v * 2, off, nt, **kw).float()
    assert torch.equal(dbl, base * 2)
    # deterministic
    again = recir_amd.jagged_hstu_attention(q, k, v, off, nt, **kw).float()
    assert torch.equal(again, base)
    # attn_scale = 1/N given explicitly is the default
    sc = torch.tensor(1.0 / wl.max_seq_len, device=q.device)
    expl = recir_amd.jagged_hstu_attention(q, k, v, off, nt, attn_scale=sc, **kw).float()
    assert torch.equal(expl, base)
    # sequences are independent: permuting whole sequences permutes the output rows
    lengths = wl.lengths
    perm = np.random.default_rng(0).permutation(wl.B)
    offs = wl.seq_offsets.numpy()
    idx = np.concatenate([np.arange(offs[b], offs[b + 1]) for b in perm])
    idx_t = torch.from_numpy(idx).cuda()
    off2 = torch.from_numpy(np.concatenate([[0], np.cumsum(lengths[perm])])).cuda()
    out2 = recir_amd.jagged_hstu_attention(q[idx_t], k[idx_t], v[idx_t], off2, nt[torch.from_numpy(perm).cuda()], **kw).float()
    assert torch.equal(out2, base[idx_t])


def test_int32_offsets_and_absent_targets(oracle):
    from recir_amd.workloads import make_jagged

    wl = make_jagged([200, 77, 0, 130], [0, 0, 0, 0], 2, 128, 128, max_seq_len=256, alpha=1 / 128,
                     dtype="bf16", seed=4)
    a = run_hip(wl)
    b = run_hip(wl, offsets_dtype=torch.int32)
    c = run_hip(wl, num_targets=None)
    assert torch.equal(a, b) and torch.equal(a, c)
    assert_bf16_close(a, run_oracle(oracle, wl), "int32/none")


def test_scalar_and_per_token_scale_tiled(oracle):
    from recir_amd.workloads import make_jagged

    wl = make_jagged([200, 77, 130], [10, 0, 130], 2, 128, 128, max_seq_len=256, alpha=1 / 128,
                     dtype="bf16", seed=6)
    s0 = torch.tensor(0.013)
    assert_bf16_close(run_hip(wl, attn_scale=s0), run_oracle(oracle, wl, attn_scale=s0), "0-d scale")
    st = torch.rand(wl.T, generator=torch.Generator().manual_seed(1)) * 0.02
    assert_bf16_close(run_hip(wl, attn_scale=st), run_oracle(oracle, wl, attn_scale=st), "[T] scale")
    assert_bf16_close(run_hip(wl, attn_scale=0.5), run_oracle(oracle, wl, attn_scale=0.5), "float scale")


@pytest.mark.parametrize("generic", [False, True], ids=["default_kernel", "generic_kernel"])
@pytest.mark.parametrize("shape", [(2, 8, 6), (3, 64, 64), (1, 128, 32), (2, 40, 200)])
def test_other_head_dims(oracle, shape, generic):
    """Head dims other than 128, fp32 and bf16, on the kernel the library picks (the general MFMA kernels) and
    on the generic one."""
    import contextlib

    from recir_amd import _lib, ops
    from recir_amd.workloads import make_jagged

    H, Dqk, Dv = shape
    wl = make_jagged([70, 0, 5, 129], [9, 0, 5, 1], H, Dqk, Dv, max_seq_len=130, alpha=0.11, seed=8,
                     with_rab=True, rab_std=0.3, contextual_seq_len=2, tail_rows=2)
    ref = run_oracle(oracle, wl)
    with (ops.force_kernel(ops.KERNEL_GENERIC) if generic else contextlib.nullcontext()):
        out = run_hip(wl)
        k32 = _lib.last_kernel()
        outb = run_hip(wl, dtype="bf16")
        k16 = _lib.last_kernel()
    if generic:
        assert (k32, k16) == ("generic_fp32", "generic_bf16")
    else:
        # (fp32 tiles stop at head dim 128: 40 / 200 is the generic kernel's)
        assert k32 == expected_kernel(Dqk, Dv, "fp32", rab=True) and k16 == expected_kernel(Dqk, Dv, "bf16", rab=True)
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=FP32_RTOL, atol=FP32_ATOL)
    wlb_ref = run_oracle(oracle, wl, q=wl.q.bfloat16().float(), k=wl.k.bfloat16().float())
    st = error_stats(outb, wlb_ref)
    assert st["rel_to_max"] <= 3e-2, st  # v is also rounded to bf16 here


@pytest.mark.parametrize("D,dtype", [(128, "bf16"), (8, "fp32")])
def test_alpha_default_is_inverse_sqrt_of_head_dim(oracle, D, dtype):
    """``alpha=None`` means ``1/sqrt(Dqk)`` (recir/ops/pallas/jagged_hstu_attention.py:1550-1555),
    on the tiled kernel (head dim 128) and on the generic one (head dim 8)."""
    import math

    import recir_amd
    from recir_amd import _lib
    from recir_amd.workloads import make_jagged

    wl = make_jagged([150, 3, 70], [20, 0, 70], 2, D, D, max_seq_len=160, alpha=1.0 / math.sqrt(D), dtype=dtype, seed=21,
                     tail_rows=3)
    q, k, v, off, nt = to_device(wl)
    out = recir_amd.jagged_hstu_attention(q, k, v, off, nt, max_seq_len=wl.max_seq_len)  # alpha, attn_scale left out
    torch.cuda.synchronize()
    assert _lib.last_kernel() == expected_kernel(D, D, dtype)
    ref = run_oracle(oracle, wl)  # the oracle gets 1/sqrt(D) explicitly
    if dtype == "bf16":
        assert_bf16_close(out, ref, f"alpha=None D={D}")
    else:
        np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=FP32_RTOL, atol=FP32_ATOL)
    # and it is not what another alpha would give (the scores here are O(1), so alpha matters)
    other = run_oracle(oracle, make_jagged([150, 3, 70], [20, 0, 70], 2, D, D, max_seq_len=160, alpha=1.0 / D, dtype=dtype,
                                           seed=21, tail_rows=3))
    assert np.abs(other - ref).max() > 10 * (BF16_REL if dtype == "bf16" else FP32_RTOL) * np.abs(ref).max()


@pytest.mark.parametrize("D", [128, 64])
def test_many_short_sequences_use_the_general_work_list(oracle, D):
    """More sequences than the single-block work-list builder tabulates (1024): both MFMA kernel
    families, forward and backward."""
    from recir_amd import _lib
    from recir_amd.workloads import make_jagged
    from tests.test_gpu_bwd import assert_grads_close, run_hip_bwd

    rng = np.random.default_rng(5)
    lengths = rng.integers(0, 40, size=1300)
    lengths[7] = 300
    targets = np.minimum(rng.integers(0, 4, size=1300), lengths)
    wl = make_jagged(lengths, targets, 2, D, D, max_seq_len=320, alpha=1 / D, dtype="bf16", seed=11)
    out = run_hip(wl)
    assert _lib.last_kernel() == expected_kernel(D, D)
    assert_bf16_close(out, run_oracle(oracle, wl), f"B=1300 D={D}")
    dout = torch.randn(wl.T, wl.H, D, generator=torch.Generator().manual_seed(6)).bfloat16().float()
    got = run_hip_bwd(wl, dout)
    assert _lib.last_kernel() == expected_kernel(D, D, bwd=True)
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha)
    assert_grads_close(got, want[:3], int(wl.seq_offsets[-1]), BF16_REL, f"B=1300 D={D} backward")


@pytest.mark.parametrize("lengths", [[1500] + [70] * 30, [300] * 16, [700]], ids=["one_long", "even", "single"])
def test_work_list_dealing_by_tiles_and_by_pairs(oracle, lengths):
    """One sequence far longer than the rest, or fewer (sequence, head) pairs than XCDs, makes the
    work-list builder deal single tiles to the XCD lists; an even batch deals whole pairs."""
    from recir_amd.workloads import make_jagged

    wl = make_jagged(lengths, [3] * len(lengths), 2, 128, 128, max_seq_len=max(lengths), alpha=1 / 128,
                     dtype="bf16", seed=21)
    assert_bf16_close(run_hip(wl), run_oracle(oracle, wl), f"lengths {lengths[:2]}...")


@pytest.mark.parametrize("D,with_rab", [(128, False), (128, True), (64, False), (64, True)])
def test_sequences_longer_than_max_seq_len_do_not_break_the_work_list(oracle, D, with_rab):
    """Out of contract (n > max_seq_len), but the launch must stay in bounds: the work lists are
    then longer than the grid assumes and the workgroups loop over them; a pair whose diagonal lies
    outside the bias table has no bias, as in the oracle.  Head dim 128 and the general MFMA kernels,
    forward and backward."""
    from recir_amd import _lib
    from recir_amd.workloads import make_jagged
    from tests.test_gpu_bwd import _scale_np, assert_grads_close, run_hip_bwd

    wl = make_jagged([3000, 40, 1500], [10, 0, 0], 1, D, D, max_seq_len=256, alpha=1 / D, dtype="bf16", seed=12,
                     with_rab=with_rab, rab_std=0.5)
    out = run_hip(wl)
    assert _lib.last_kernel() == expected_kernel(D, D, rab=with_rab)
    assert_bf16_close(out, run_oracle(oracle, wl), "n > N")
    dout = torch.randn(wl.T, wl.H, D, generator=torch.Generator().manual_seed(4)).bfloat16().float()
    got = run_hip_bwd(wl, dout, rab=wl.rab)
    assert _lib.last_kernel() == expected_kernel(D, D, bwd=True, rab=with_rab)
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                           rab=None if wl.rab is None else wl.rab.numpy())
    assert_grads_close(got, want[:3], int(wl.seq_offsets[-1]), BF16_REL, "n > N backward")


def test_work_lists_are_reused_for_the_same_offset_tensors_and_rebuilt_when_they_change(oracle):
    """The operator keeps the work lists of a layout and reuses them while the caller passes the
    very same offset tensors unchanged (the layers of one step); an in-place change of the offsets
    (version counter) or other tensors build new lists."""
    import recir_amd
    from recir_amd import ops
    from recir_amd.workloads import make_jagged

    recir_amd.set_plan_cache(True)  # also empties it
    wl = make_jagged([300, 129, 64, 1, 0, 517], [40, 129, 0, 0, 0, 6], 2, 128, 128, max_seq_len=600,
                     alpha=1.0 / 128, dtype="bf16", seed=31)
    q, k, v, off, nt = to_device(wl)
    kw = dict(max_seq_len=wl.max_seq_len, alpha=wl.alpha)
    before = dict(ops.plan_cache_stats)
    a = recir_amd.jagged_hstu_attention(q, k, v, off, nt, **kw)
    b = recir_amd.jagged_hstu_attention(q, k, v, off, nt, **kw)      # same tensors: lists reused
    c = recir_amd.jagged_hstu_attention(v, q, k, off, nt, **kw)      # another layer's q, k, v
    assert ops.plan_cache_stats["misses"] - before["misses"] == 1
    assert ops.plan_cache_stats["hits"] - before["hits"] == 2
    assert torch.equal(a, b)
    assert_bf16_close(a, run_oracle(oracle, wl), "first call")
    assert_bf16_close(c, oracle.attn_fwd(wl.v.numpy(), wl.q.numpy(), wl.k.numpy(), wl.seq_offsets.numpy(),
                                         wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha), "reused")
    # the same tensor objects with another layout written into them
    wl2 = make_jagged([100, 400, 3, 250, 200, 58], [0, 10, 3, 0, 100, 1], 2, 128, 128, max_seq_len=600,
                      alpha=1.0 / 128, dtype="bf16", seed=31)
    assert wl2.T == wl.T
    off.copy_(wl2.seq_offsets.to(off.device))
    nt.copy_(wl2.num_targets.to(nt.device))
    d = recir_amd.jagged_hstu_attention(q, k, v, off, nt, **kw)
    assert ops.plan_cache_stats["misses"] - before["misses"] == 2
    assert_bf16_close(d, oracle.attn_fwd(wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl2.seq_offsets.numpy(),
                                         wl2.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha),
                      "after an in-place change of the offsets")
    # tensors made under inference mode have no version counter: never cached, still right
    with torch.inference_mode():
        off_i, nt_i = off.clone(), nt.clone()
        f1 = recir_amd.jagged_hstu_attention(q, k, v, off_i, nt_i, **kw)
        f2 = recir_amd.jagged_hstu_attention(q, k, v, off_i, nt_i, **kw)
    assert torch.equal(f1, d) and torch.equal(f2, d)
    assert ops.plan_cache_stats["misses"] - before["misses"] == 2 and ops.plan_cache_stats["hits"] - before["hits"] == 2
    # switched off: every call builds its lists
    recir_amd.set_plan_cache(False)
    e = recir_amd.jagged_hstu_attention(q, k, v, off, nt, **kw)
    assert torch.equal(d, e)
    assert ops.plan_cache_stats["misses"] - before["misses"] == 2 and ops.plan_cache_stats["hits"] - before["hits"] == 2
    # a step scope: reuse inside, nothing kept afterwards; offsets that arrive on the host are moved
    # to the device and still reused (the entry is keyed on the caller's tensors)
    off_h, nt_h = off.cpu(), nt.cpu()
    with recir_amd.plan_cache_scope():
        g1 = recir_amd.jagged_hstu_attention(q, k, v, off_h, nt_h, **kw)
        g2 = recir_amd.jagged_hstu_attention(q, k, v, off_h, nt_h, **kw)
    assert torch.equal(g1, d) and torch.equal(g2, d)
    assert ops.plan_cache_stats["misses"] - before["misses"] == 3 and ops.plan_cache_stats["hits"] - before["hits"] == 3
    assert not ops._plan_cache and not ops._plan_cache_enabled  # off again, as before the scope


def test_rab_zero_is_identical_to_no_rab():
    from recir_amd.workloads import make_jagged

    wl = make_jagged([300, 64], [30, 0], 2, 128, 128, max_seq_len=320, alpha=1 / 128, dtype="bf16", seed=2)
    a = run_hip(wl)
    b = run_hip(wl, rab=torch.zeros(2, 2 * 320 - 1))
    st = error_stats(b, a.float().cpu().numpy())
    # a zero bias goes through the biased code path (alpha applied before silu instead of after):
    # equal up to one bf16 rounding of P
    assert st["rel_to_max"] <= 2 ** -7, st


def test_empty_batch_and_all_empty_sequences():
    import recir_amd

    dev = torch.device("cuda:0")
    q = torch.randn(6, 2, 128, device=dev).bfloat16()
    out = recir_amd.jagged_hstu_attention(q, q, q, torch.zeros(4, dtype=torch.int64, device=dev), max_seq_len=8)
    assert not out.any()
    out = recir_amd.jagged_hstu_attention(q.float(), q.float(), q.float(), torch.zeros(2, dtype=torch.int64, device=dev), max_seq_len=8)
    assert not out.any()
    e = torch.empty(0, 2, 128, device=dev, dtype=torch.bfloat16)
    out = recir_amd.jagged_hstu_attention(e, e, e, torch.zeros(2, dtype=torch.int64, device=dev), max_seq_len=8)
    assert out.shape == (0, 2, 128)


def test_runs_on_the_callers_stream():
    import recir_amd
    from recir_amd.workloads import make_config

    wl = make_config(2)
    q, k, v, off, nt = to_device(wl)
    base = recir_amd.jagged_hstu_attention(q, k, v, off, nt, max_seq_len=2048, alpha=wl.alpha)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out = recir_amd.jagged_hstu_attention(q, k, v, off, nt, max_seq_len=2048, alpha=wl.alpha)
    s.synchronize()
    assert torch.equal(out, base)


def test_fp8_quantiser_is_bit_exact(oracle):
    """Per-head scales and e4m3 codes against the C restatement of the reference recipe
    (kjt_split_per_feature.cpp:493-502), which is itself pinned to torch's float8_e4m3fn cast."""
    import recir_amd

    g = torch.Generator().manual_seed(3)
    x = (torch.randn(301, 3, 128, generator=g) * torch.tensor([0.05, 1.0, 40.0]).view(1, 3, 1)).bfloat16()
    x[5, 1, 7] = 0.0
    codes, scale = recir_amd.quantize_e4m3_per_head(x.cuda())
    want_codes, want_scale = oracle.quant_e4m3_per_head(x.float().numpy())
    np.testing.assert_array_equal(scale.cpu().numpy(), want_scale)
    np.testing.assert_array_equal(codes.view(torch.uint8).cpu().numpy(), want_codes)
    assert codes.dtype == torch.float8_e4m3fn


def _fp8_reference(oracle, wl):
    """fp32 oracle on the dequantised q, k: S = alpha * sq[h] * sk[h] * (Q8 . K8^T)."""
    q8, qs = oracle.quant_e4m3_per_head(wl.q.numpy())
    k8, ks = oracle.quant_e4m3_per_head(wl.k.numpy())
    qd = torch.from_numpy(oracle.e4m3_decode(q8) * qs.reshape(1, -1, 1))
    kd = torch.from_numpy(oracle.e4m3_decode(k8) * ks.reshape(1, -1, 1))
    return run_oracle(oracle, wl, q=qd, k=kd)


@pytest.mark.parametrize("with_rab", [False, True])
def test_fp8_small_case(oracle, with_rab):
    from recir_amd import _lib
    from recir_amd.workloads import make_jagged

    wl = make_jagged([300, 129, 64, 1, 0, 517], [40, 129, 0, 0, 0, 6], 2, 128, 128, max_seq_len=600,
                     alpha=1.0 / 128, dtype="fp8", seed=21, with_rab=with_rab, rab_std=0.3,
                     contextual_seq_len=8 if with_rab else 0, tail_rows=5)
    out = run_hip(wl, fp8=True)
    assert _lib.last_kernel().startswith("tiled_d128_fp8qk")
    # against the same quantised operands: only bf16-level differences remain
    assert_bf16_close(out, _fp8_reference(oracle, wl), "fp8 vs dequantised oracle")
    # against the unquantised fp32 reference: the stated fp8 tolerance
    st = error_stats(out, run_oracle(oracle, wl))
    assert st["max_abs"] <= FP8_MAX_ABS, st
    assert not out[int(wl.seq_offsets[-1]):].any()


@pytest.mark.parametrize("seed", range(10))
def test_fp8_randomized_cases(oracle, seed):
    """The fp8 q/k kernel on seeded random cases (tile-boundary lengths, targets, prefix, window,
    bias), against the oracle on the same quantised operands."""
    from recir_amd import _lib
    from recir_amd.workloads import make_jagged

    rng = np.random.default_rng(2000 + seed)
    B = int(rng.integers(1, 6))
    edges = np.array([0, 1, 31, 32, 33, 63, 64, 65, 127, 128, 129, 191, 192, 255, 256, 257])
    lengths = [int(rng.choice(edges)) if rng.random() < 0.5 else int(rng.integers(0, 420)) for _ in range(B)]
    targets = [int(rng.integers(0, n + 1)) if rng.random() < 0.6 else 0 for n in lengths]
    A = int(rng.choice([0, 0, 33, 128]))
    wl = make_jagged(lengths, targets, int(rng.integers(1, 4)), 128, 128, max_seq_len=max(max(lengths), 1) + 3,
                     alpha=1.0 / 128, dtype="fp8", seed=seed, contextual_seq_len=int(rng.choice([0, 0, 3, 70])),
                     tail_rows=int(rng.integers(0, 4)), max_attn_len=A, full_attn_size=int(rng.choice([0, 40])) if A else 0,
                     with_rab=bool(rng.random() < 0.4), rab_std=0.3)
    what = (f"seed {seed}: lengths {lengths} targets {targets} H {wl.H} ctx {wl.contextual_seq_len} "
            f"A {wl.max_attn_len} F {wl.full_attn_size} rab {wl.rab is not None}")
    out = run_hip(wl, fp8=True)
    if wl.T:
        assert _lib.last_kernel().startswith("tiled_d128_fp8qk"), what
    assert_bf16_close(out, _fp8_reference(oracle, wl), what)
    assert not out[int(wl.seq_offsets[-1]):].any(), what


def test_config5_fp8_matches_oracle(oracle):
    from recir_amd.workloads import make_config

    wl = make_config(5)
    out = run_hip(wl, fp8=True)
    st_q = assert_bf16_close(out, _fp8_reference(oracle, wl), "config5 vs dequantised oracle")
    st = error_stats(out, run_oracle(oracle, wl))
    print("config5 vs dequantised:", st_q, " vs fp32 reference:", st)
    assert st["max_abs"] <= FP8_MAX_ABS, st
    assert st["rel_fro"] <= 5e-2, st  # relative form of the same bound (outputs are O(1e-3))
    assert_same_zero_structure(out, run_oracle(oracle, wl), int(wl.seq_offsets[-1]))


def test_fp8_region_swap_in_a_traced_graph(oracle):
    """The training-to-inference hook end to end: trace a function that calls the bf16 operator,
    cut out the matched node as a region, let the factory build its replacement, splice it back and
    run both graphs.  The swapped graph must equal the fp8 entry point bit for bit and stay within
    the fp8 tolerance of the fp32 oracle."""
    import torch.fx as fx
    from torch.fx.experimental.proxy_tensor import make_fx

    import recir_amd
    from recir_amd import _lib
    from recir_amd.workloads import make_jagged

    wl = make_jagged([200, 70, 0, 131], [16, 70, 0, 3], 2, 128, 128, max_seq_len=256, alpha=1.0 / 128,
                     dtype="bf16", seed=31, tail_rows=3)
    q, k, v, off, nt = to_device(wl)
    op = recir_amd.hstu_jagged_attention_fwd.default

    def f(q, k, v, off, nt):
        out, _aux = op(wl.max_seq_len, wl.alpha, q, k, v, off, "lower_triangular", nt, None, 0, 0, 0)
        return out.float() * 2.0

    gm = make_fx(f, tracing_mode="fake")(q, k, v, off, nt)
    node = next(n for n in gm.graph.nodes if recir_amd.hstu_attention_matcher(n))
    region = fx.Graph()
    env = {a: region.placeholder(a.name) for a in node.args if isinstance(a, fx.Node)}
    region.output(region.node_copy(node, lambda n: env[n]))
    run = recir_amd.fp8_attention_region(fx.GraphModule(torch.nn.Module(), region))
    ref_bf16 = gm(q, k, v, off, nt)
    assert _lib.last_kernel() == "tiled_d128_bf16"
    with gm.graph.inserting_before(node):
        repl = gm.graph.call_function(run, tuple(a for a in node.args if isinstance(a, fx.Node)))
    node.replace_all_uses_with(repl)
    gm.graph.erase_node(node)
    gm.recompile()
    got = gm(q, k, v, off, nt)
    torch.cuda.synchronize()
    assert _lib.last_kernel() == "tiled_d128_fp8qk"
    direct = recir_amd.jagged_hstu_attention_fp8(q, k, v, off, nt, max_seq_len=wl.max_seq_len, alpha=wl.alpha)
    assert torch.equal(got, direct.float() * 2.0)
    want = 2.0 * run_oracle(oracle, wl)
    st = error_stats(got, want)
    assert st["max_abs"] <= 2 * FP8_MAX_ABS and st["rel_fro"] <= 5e-2, st
    assert error_stats(ref_bf16, want)["rel_fro"] <= 2e-2


def test_fp8_region_swap_keeps_the_reference_contextual_rule(oracle):
    """A node that calls the reference's operator with ``contextual_seq_len = 4`` means "keys whose
    target-clamped id is 0" (kjt_split_per_feature.cpp:672-674): key 0, or every key of a sequence
    that is all targets.  The fp8 region built from it must keep that rule, not the prefix rule of
    ``recir::hstu_jagged_attention_fwd`` -- checked against the oracle in the reference's mode on the
    dequantised operands; the same inputs under the prefix rule differ, so the test tells them apart."""
    import torch.fx as fx
    from torch.fx.experimental.proxy_tensor import make_fx

    import recir_amd
    from recir_amd import _lib
    from recir_amd.workloads import make_jagged

    # sequences 1 and 3 are all targets (cap = 0): there the two rules keep different pairs
    wl = make_jagged([200, 70, 5, 131, 9], [16, 70, 0, 131, 2], 2, 128, 128, max_seq_len=256, alpha=1.0 / 128,
                     dtype="bf16", seed=37, tail_rows=2)
    q, k, v, off, nt = to_device(wl)
    ctx = 4
    for op, rule, via in ((recir_amd.triton_ragged_attention_fwd.default, oracle.CTX_REFCPP,
                           recir_amd.attention_via_fp8_reference_rule),
                          (recir_amd.hstu_jagged_attention_fwd.default, oracle.CTX_PREFIX,
                           recir_amd.attention_via_fp8)):
        def f(q, k, v, off, nt):
            out, _aux = op(wl.max_seq_len, wl.alpha, q, k, v, off, "lower_triangular", nt, None, 0, ctx, 0)
            return out

        gm = make_fx(f, tracing_mode="fake")(q, k, v, off, nt)
        node = next(n for n in gm.graph.nodes if recir_amd.hstu_attention_matcher(n))
        region = fx.Graph()
        env = {a: region.placeholder(a.name) for a in node.args if isinstance(a, fx.Node)}
        region.output(region.node_copy(node, lambda n: env[n]))
        run = recir_amd.fp8_attention_region(fx.GraphModule(torch.nn.Module(), region))
        calls = [n for n in run.gm.graph.nodes if n.op == "call_function" and n.target in (
            recir_amd.attention_via_fp8, recir_amd.attention_via_fp8_reference_rule)]
        assert len(calls) == 1 and calls[0].target is via
        got = run(q, k, v, off, nt)[0]
        torch.cuda.synchronize()
        assert _lib.last_kernel().startswith("tiled_d128_fp8qk")
        q8, qs = oracle.quant_e4m3_per_head(wl.q.numpy())
        k8, ks = oracle.quant_e4m3_per_head(wl.k.numpy())
        qd = torch.from_numpy(oracle.e4m3_decode(q8) * qs.reshape(1, -1, 1))
        kd = torch.from_numpy(oracle.e4m3_decode(k8) * ks.reshape(1, -1, 1))
        want = run_oracle(oracle, wl, q=qd, k=kd, ctx=ctx, ctx_mode=rule)
        other = run_oracle(oracle, wl, q=qd, k=kd, ctx=ctx, ctx_mode=1 - rule)
        assert np.abs(want - other).max() > 1e-3  # the two rules differ on these inputs
        assert_bf16_close(got, want, f"fp8 region, contextual rule {rule}")
        assert_same_zero_structure(got, want, int(wl.seq_offsets[-1]))
        # and the unquantised graph it replaced, against the fp32 oracle at the fp8 tolerance
        st = error_stats(got, run_oracle(oracle, wl, ctx=ctx, ctx_mode=rule))
        assert st["max_abs"] <= FP8_MAX_ABS, st


def test_generic_kernel_policy_warns_or_rejects(oracle):
    """A bf16 call that only the slow generic kernels cover (here: head dims 264 / 260) says so once by default,
    is rejected by the C ABI under the 'error' policy (RECIR_HSTU_FLAG_TILED_ONLY), and is silent under
    'silent'; the result is the oracle's in every case that runs.  fp32 calls never warn."""
    import warnings

    import recir_amd
    from recir_amd import _lib, ops
    from recir_amd.workloads import make_jagged

    wl = make_jagged([70, 33, 0, 129], [8, 33, 0, 3], 2, 264, 260, max_seq_len=160, alpha=1.0 / 264, dtype="bf16", seed=41)
    want = run_oracle(oracle, wl)
    ops._generic_warned.clear()
    prev = recir_amd.set_generic_kernel_policy("warn")
    try:
        with warnings.catch_warnings(record=True) as rec:
            warnings.simplefilter("always")
            out = run_hip(wl)
            out2 = run_hip(wl)
        assert _lib.last_kernel() == "generic_bf16"
        msgs = [str(w.message) for w in rec if issubclass(w.category, RuntimeWarning)]
        assert len(msgs) == 1 and "head dims 264 / 260" in msgs[0], msgs  # once per reason
        assert_bf16_close(out, want, "generic kernel, head dims 264 / 260")
        assert torch.equal(out, out2)
        recir_amd.set_generic_kernel_policy("error")
        with pytest.raises(ValueError, match="only the generic kernel"):
            run_hip(wl)
        with ops.force_kernel(ops.KERNEL_GENERIC):  # an explicit choice of the generic kernel is not rejected
            assert torch.equal(run_hip(wl), out)
        # a call the MFMA kernels cover passes under the same policy
        wl128 = make_jagged([70, 33], [8, 33], 2, 128, 128, max_seq_len=160, alpha=1.0 / 128, dtype="bf16", seed=42)
        assert_bf16_close(run_hip(wl128), run_oracle(oracle, wl128), "tiled kernel under the error policy")
        assert _lib.last_kernel() == "tiled_d128_bf16"
        recir_amd.set_generic_kernel_policy("silent")
        ops._generic_warned.clear()
        with warnings.catch_warnings(record=True) as rec:
            warnings.simplefilter("always")
            run_hip(wl)
        assert not [w for w in rec if issubclass(w.category, RuntimeWarning)]
        recir_amd.set_generic_kernel_policy("warn")
        with warnings.catch_warnings(record=True) as rec:  # the fp32 smoke path is the generic kernel by design
            warnings.simplefilter("always")
            wl32 = make_jagged([20, 20], [4, 4], 2, 32, 32, max_seq_len=20, alpha=1.0 / 32, dtype="fp32", seed=43)
            run_hip(wl32)
        assert not [w for w in rec if issubclass(w.category, RuntimeWarning)]
    finally:
        recir_amd.set_generic_kernel_policy(prev)


def test_semilocal_full_size_matches_oracle(oracle):
    """Configuration 2 with the reference's semi-local shape (256 local + 256 full tail): the tiled
    kernel (which skips key tiles below the window) against the oracle."""
    from recir_amd import _lib
    from recir_amd.workloads import make_config

    wl = make_config(6)
    out = run_hip(wl)
    assert _lib.last_kernel() == "tiled_d128_bf16"
    ref = run_oracle(oracle, wl)
    st = assert_bf16_close(out, ref, "config6")
    print(f"config6: {st}")


@pytest.mark.parametrize("A,F,ctx", [(64, 0, 0), (100, 37, 0), (33, 200, 0), (128, 64, 5), (1, 1, 0)])
def test_semilocal_windows_across_tiles(oracle, A, F, ctx):
    from recir_amd import ops
    from recir_amd.workloads import make_jagged

    wl = make_jagged([1, 63, 64, 65, 127, 129, 0, 300, 517, 90], [0, 3, 64, 1, 100, 0, 0, 60, 130, 90], 2, 128, 128,
                     max_seq_len=520, alpha=1.0 / 128, dtype="bf16", seed=50 + A, contextual_seq_len=ctx,
                     tail_rows=3, max_attn_len=A, full_attn_size=F)
    ref = run_oracle(oracle, wl)
    out = run_hip(wl)
    assert_bf16_close(out, ref, f"A{A} F{F}")
    assert not out[int(wl.seq_offsets[-1]):].float().cpu().numpy().any()
    with ops.force_kernel(ops.KERNEL_GENERIC):
        outg = run_hip(wl)
    assert_bf16_close(outg, ref, f"generic A{A} F{F}")
    with ops.force_kernel(ops.KERNEL_MFMA_GENERAL):  # its own walk of the key tiles under the window
        outm = run_hip(wl)
    assert_bf16_close(outm, ref, f"general MFMA kernel A{A} F{F}")
    # fp8 q/k variant shares the tile walk
    out8 = run_hip(wl, fp8=True)
    st = error_stats(out8, ref)
    assert st["max_abs"] <= FP8_MAX_ABS, st


def test_fp8_scales_ignore_padding_rows(oracle):
    """Rows at and after seq_offsets[-1] are padding the caller may have left uninitialised: NaN there
    must not reach a head's scale (it would poison every valid row), and the padding gets zero codes."""
    import recir_amd
    from recir_amd.workloads import make_jagged

    wl = make_jagged([150, 64, 33], [10, 0, 33], 2, 128, 128, max_seq_len=256, alpha=1 / 128, dtype="bf16", seed=71,
                     tail_rows=6)
    end = int(wl.seq_offsets[-1])
    wl.q[end:] = 0  # the oracle's quantiser looks at every row it is given
    wl.k[end:] = 0
    q, k, v, off, nt = to_device(wl)
    q[end:] = float("nan")
    k[end:] = float("inf")
    v[end:] = float("nan")
    codes, scale = recir_amd.quantize_e4m3_per_head(q, off)
    codes_ref, scale_ref = recir_amd.quantize_e4m3_per_head(q[:end].contiguous())
    assert torch.equal(scale, scale_ref) and torch.isfinite(scale).all().item()
    assert torch.equal(codes[:end].view(torch.uint8), codes_ref.view(torch.uint8))
    assert not codes[end:].view(torch.uint8).any().item()
    out = recir_amd.jagged_hstu_attention_fp8(q, k, v, off, nt, max_seq_len=wl.max_seq_len, alpha=wl.alpha)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all().item() and not out[end:].float().abs().any().item()
    assert_bf16_close(out[:end], _fp8_reference(oracle, wl)[:end], "fp8 with NaN padding")


@pytest.mark.parametrize("seed", range(10))
def test_long_sequences_randomized(oracle, seed):
    """Sequences long enough for the leading-tile loop of the direct-to-LDS kernel (eight or more key
    tiles that are unmasked for a whole query tile), with what decides where that loop starts and
    stops drawn at random: lengths off the tile grid, target counts that cut the history short or
    leave query tiles of targets only, contextual prefixes, tail rows, the kind of output scale."""
    from recir_amd import _lib
    from recir_amd.workloads import make_jagged

    rng = np.random.default_rng(7000 + seed)
    B = int(rng.integers(1, 4))
    lengths = [int(rng.integers(600, 2300)) for _ in range(B)]
    if seed % 3 == 0:
        lengths[0] = int(rng.choice([640, 704, 768, 1024, 1279, 1281]))
    targets = []
    for n in lengths:
        kind = rng.random()
        targets.append(0 if kind < 0.3 else int(rng.integers(1, 200)) if kind < 0.7 else int(rng.integers(n // 2, n)))
    H = int(rng.integers(1, 3))
    ctx = int(rng.choice([0, 0, 5, 70, 700]))
    N = max(lengths) + int(rng.integers(0, 70))
    wl = make_jagged(lengths, targets, H, 128, 128, max_seq_len=N, alpha=1.0 / 128, dtype="bf16", seed=300 + seed,
                     contextual_seq_len=ctx, tail_rows=int(rng.integers(0, 4)))
    scale = None
    if seed % 2:
        scale = (0.5 + torch.rand(wl.T, generator=torch.Generator().manual_seed(seed))) / 100
    out = run_hip(wl, attn_scale=scale)
    assert _lib.last_kernel() == "tiled_d128_bf16"
    ref = run_oracle(oracle, wl, attn_scale=scale)
    assert_bf16_close(out, ref, f"long seed {seed}: lengths {lengths} targets {targets} H {H} ctx {ctx}")


def test_grouped_work_lists_give_the_same_output(oracle):
    """RECIR_HSTU_FLAG_GROUPED_LISTS only changes the order in which an XCD's work list is walked
    (groups of eight (sequence, head) pairs): bit-identical output, forward and backward, with more
    pairs per list than one group holds and with lists that tiles are dealt to."""
    import recir_amd
    from recir_amd import _lib, ops
    from recir_amd.workloads import make_jagged

    rng = np.random.default_rng(5)
    for lengths in ([int(x) for x in rng.integers(1, 700, size=40)], [900] + [70] * 20):
        targets = [int(rng.integers(0, n // 3 + 1)) for n in lengths]
        wl = make_jagged(lengths, targets, 4, 128, 128, max_seq_len=max(lengths) + 3, alpha=1.0 / 128, dtype="bf16",
                         seed=77, tail_rows=2)
        out = run_hip(wl)
        assert _lib.last_kernel() == "tiled_d128_bf16"
        assert_bf16_close(out, run_oracle(oracle, wl), f"{len(lengths)} sequences, lists as built")
        q, k, v, off, nt = to_device(wl)
        dout = torch.randn(wl.T, wl.H, 128, generator=torch.Generator().manual_seed(1)).to(q.device, q.dtype)
        grads = recir_amd.jagged_hstu_attention_backward(dout, q, k, v, off, nt, None, max_seq_len=wl.max_seq_len,
                                                         alpha=wl.alpha)
        with ops.extra_flags(_lib.FLAG_GROUPED_LISTS):
            out_g = run_hip(wl)
            grads_g = recir_amd.jagged_hstu_attention_backward(dout, q, k, v, off, nt, None,
                                                               max_seq_len=wl.max_seq_len, alpha=wl.alpha)
        torch.cuda.synchronize()
        assert torch.equal(out, out_g)
        for a, b in zip(grads, grads_g):
            assert torch.equal(a, b)


@pytest.mark.parametrize("kernel", ["mfma_general", "generic"])
@pytest.mark.parametrize("A,F,ctx", [(0, 0, 0), (0, 0, 5), (7, 0, 0), (40, 16, 0), (3, 300, 2)])
def test_noncausal_mask_is_bit_exact(oracle, A, F, ctx, kernel):
    """The mask of a mask type other than "lower_triangular" (kjt_split_per_feature.cpp:650-671), read
    off the zero pattern of the output as in test_mask_is_bit_exact: the general MFMA kernel (which the
    library picks, and which leaves out the key tiles no row of a wave can see) and the generic one."""
    from recir_amd import _lib, ops
    from recir_amd.workloads import make_jagged

    lengths = [130, 64, 65, 1, 0, 97]
    targets = [30, 64, 1, 0, 0, 120]
    wl = make_jagged(lengths, targets, 1, 128, 128, max_seq_len=140, alpha=1.0 / 128, dtype="bf16",
                     contextual_seq_len=ctx, tail_rows=3, max_attn_len=A, full_attn_size=F, mask_type="full")
    wl.q.fill_(0.5)
    wl.k.fill_(0.25)
    wl.v.zero_()
    off = wl.seq_offsets.numpy()
    for b, n in enumerate(lengths):
        for j in range(n):
            wl.v[off[b] + j, 0, j % 128] = 1.0
    with ops.force_kernel(ops.KERNEL_AUTO if kernel == "mfma_general" else ops.KERNEL_GENERIC):
        out = run_hip(wl).float().cpu().numpy()
    assert _lib.last_kernel() == ("mfma_bf16_d128" if kernel == "mfma_general" else "generic_bf16")
    want = np.zeros((wl.T, 128), dtype=bool)
    for b, (n, t) in enumerate(zip(lengths, targets)):
        for m in range(n):
            for j in range(n):
                if oracle.keep_nc(m, j, n, t, ctx, oracle.CTX_PREFIX, A, F):
                    want[off[b] + m, j % 128] = True
    np.testing.assert_array_equal(out[:, 0, :] != 0, want)


def test_noncausal_mask_is_rejected_where_it_does_not_run():
    """fp8 q/k and the head-dim-128 kernel selector cover the causal mask only: an error, never another mask."""
    import recir_amd
    from recir_amd import ops
    from recir_amd.workloads import make_jagged

    wl = make_jagged([70, 30], [5, 0], 2, 128, 128, max_seq_len=80, alpha=1 / 128, dtype="bf16", mask_type="full",
                     max_attn_len=9)
    q, k, v, off, nt = to_device(wl)
    with ops.force_kernel(ops.KERNEL_TILED_DIRECT), pytest.raises(ValueError, match="head-dim-128 kernel needs"):
        run_hip(wl)
    with pytest.raises(ValueError, match="causal"):
        ops.attention_via_fp8(80, 1 / 128, q, k, v, off, "full", nt, None, 9, 0, 0)
    dout = torch.ones_like(v)
    with ops.force_kernel(ops.KERNEL_TILED_DIRECT), pytest.raises(ValueError, match="head-dim-128 backward needs"):
        recir_amd.jagged_hstu_attention_backward(dout, q, k, v, off, nt, max_seq_len=80, alpha=1 / 128,
                                                 max_attn_len=9, invalid_attn_mask_type="full")
