"""GPU parity tests of the backward: the HIP kernels, called through the C ABI (via the operator),
against the backward oracle on identical seeded inputs and against golden gradients taken by
autograd through the reference's compiled forward operator.

Tolerances: fp32 kernels rtol 2e-4 / atol 2e-4 of the largest gradient magnitude (the reference's
own backward test uses rtol = atol = 2e-4, recir/ops/pallas/tests/test_jagged_hstu_attention.py:
263-270); bf16 kernels 2e-2 relative to the largest reference magnitude and in Frobenius norm;
tail rows bit-exact zero.
"""
import os

import numpy as np
import pytest
import torch

from tests.golden.cases import SMALL_CASES, build_inputs, fixture_file, upstream_gradient
from tests.parity_util import BF16_REL, error_stats, expected_kernel, report, to_device

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
BWD_FP32_TOL = 2e-4


@pytest.fixture(scope="module", autouse=True)
def _need_gpu_and_library():
    from recir_amd import _lib

    assert torch.cuda.is_available(), "these tests need the MI355X"
    _lib.load()


def _scale_np(scale):
    if scale is None:
        return None
    return scale.numpy() if scale.dim() else np.float32(scale.item())


def run_hip_bwd(wl, dout, *, attn_scale=None, num_targets="default", rab=None, ctx=None, dtype=None):
    import recir_amd

    q, k, v, off, nt = to_device(wl, dtype)
    if num_targets != "default":
        nt = num_targets
    sc = attn_scale.cuda() if isinstance(attn_scale, torch.Tensor) else attn_scale
    grads = recir_amd.jagged_hstu_attention_backward(
        dout.to(q.device, q.dtype), q, k, v, off, nt, sc, max_seq_len=wl.max_seq_len, alpha=wl.alpha,
        contextual_seq_len=wl.contextual_seq_len if ctx is None else ctx,
        rab=None if rab is None else rab.cuda(), max_attn_len=wl.max_attn_len,
        full_attn_size=wl.full_attn_size, invalid_attn_mask_type=wl.mask_type)
    torch.cuda.synchronize()
    return grads


def assert_grads_close(got, want, end, tol, what):
    for g, w, name in zip(got, want, ("dq", "dk", "dv")):
        st = error_stats(g, w)
        report(f"{what} {name}", st)
        assert st["rel_to_max"] <= tol, (what, name, st)
        assert st["rel_fro"] <= tol, (what, name, st)
        assert st["worst_row_rel"] <= tol, (what, name, st)  # per (token, head) row, relative to that row
        assert not g[end:].float().cpu().numpy().any(), (what, name, "tail rows must be zero")


@pytest.mark.parametrize("name", sorted(SMALL_CASES))
def test_small_cases_match_backward_oracle_and_golden(oracle, name):
    from recir_amd import ops

    case = SMALL_CASES[name]
    wl, scale, nt = build_inputs(case)
    dout = upstream_gradient(case, wl)
    ntd = None if nt is None else nt.cuda()
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           None if nt is None else nt.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                           attn_scale=_scale_np(scale), contextual_seq_len=case["ctx"],
                           ctx_mode=oracle.CTX_REFCPP, max_attn_len=case["max_attn_len"],
                           full_attn_size=case["full_attn_size"], mask_type=case["mask_type"])
    end = int(wl.seq_offsets[-1])
    causal = case["mask_type"] == "lower_triangular"  # the other mask types run on the general MFMA kernels
    with ops.reference_contextual_rule():
        got = run_hip_bwd(wl, dout, attn_scale=scale, num_targets=ntd, dtype="fp32")
    assert all(g.dtype == torch.float32 for g in got)
    assert_grads_close(got, want, end, BWD_FP32_TOL, name)
    if case["Dqk"] < 128:  # golden gradients: autograd through the reference's C++ forward
        fx = np.load(os.path.join(GOLDEN, fixture_file(case, backward=True)))
        assert_grads_close(got, [fx[f"{name}/{k}"] for k in ("dq", "dk", "dv")], end, BWD_FP32_TOL, name + " golden")
    if case["bf16_inputs"]:
        with ops.reference_contextual_rule():
            gotb = run_hip_bwd(wl, dout, attn_scale=scale, num_targets=ntd, dtype="bf16")
        assert all(g.dtype == torch.bfloat16 for g in gotb)
        assert_grads_close(gotb, want, end, BF16_REL, name + " bf16")
        from recir_amd import _lib
        assert _lib.last_kernel() == expected_kernel(case["Dqk"], case["Dv"], causal=causal, bwd=True)
        with ops.reference_contextual_rule(), ops.force_kernel(ops.KERNEL_GENERIC):
            gotg = run_hip_bwd(wl, dout, attn_scale=scale, num_targets=ntd, dtype="bf16")
        assert _lib.last_kernel() == "bwd_generic_bf16"
        assert_grads_close(gotg, want, end, BF16_REL, name + " bf16 generic")


@pytest.mark.parametrize("ctx,with_rab,per_token", [(0, True, False), (5, True, True), (3, False, True)])
def test_bias_prefix_rule_and_per_token_scale(oracle, ctx, with_rab, per_token):
    from recir_amd.workloads import make_jagged

    wl = make_jagged([33, 1, 0, 70, 12], [5, 0, 0, 20, 12], 2, 16, 24, max_seq_len=80, alpha=0.2, dtype="fp32",
                     seed=21 + ctx, contextual_seq_len=ctx, tail_rows=3)
    g = torch.Generator().manual_seed(5)
    dout = torch.randn(wl.T, wl.H, 24, generator=g)
    rab = torch.randn(wl.H, 2 * 80 - 1, generator=g) if with_rab else None
    scale = (torch.rand(wl.T, generator=g) * 0.5 + 0.1) if per_token else torch.tensor(0.07)
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=80, alpha=0.2, attn_scale=_scale_np(scale),
                           rab=None if rab is None else rab.numpy(), contextual_seq_len=ctx)
    got = run_hip_bwd(wl, dout, attn_scale=scale, rab=rab)
    assert_grads_close(got, want, int(wl.seq_offsets[-1]), BWD_FP32_TOL, f"ctx{ctx}")


def test_autograd_through_the_forward_operator(oracle):
    """out.backward(dout) on the forward operator gives the backward operator's gradients."""
    import recir_amd

    case = SMALL_CASES["ref_targets_and_empty"]
    wl, scale, nt = build_inputs(case)
    dout = upstream_gradient(case, wl).cuda()
    q, k, v, off, ntd = to_device(wl, "fp32")
    q.requires_grad_(True), k.requires_grad_(True), v.requires_grad_(True)
    out = recir_amd.jagged_hstu_attention(q, k, v, off, ntd, max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                                          attn_scale=scale.cuda())
    out.backward(dout)
    direct = recir_amd.jagged_hstu_attention_backward(dout, q.detach(), k.detach(), v.detach(), off, ntd,
                                                      scale.cuda(), max_seq_len=wl.max_seq_len, alpha=wl.alpha)
    for a, b in zip((q.grad, k.grad, v.grad), direct):
        assert torch.equal(a, b)
    want = oracle.attn_bwd(dout.cpu().numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           nt.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha, attn_scale=_scale_np(scale))
    assert_grads_close((q.grad, k.grad, v.grad), want, int(wl.seq_offsets[-1]), BWD_FP32_TOL, "autograd")


def test_backward_of_empty_batch_and_zero_gradient():
    import recir_amd

    dev = torch.device("cuda:0")
    q = torch.randn(6, 2, 8, device=dev)
    off0 = torch.zeros(1 + 0 + 1, dtype=torch.int64, device=dev)  # one empty sequence
    dq, dk, dv = recir_amd.jagged_hstu_attention_backward(torch.randn_like(q), q, q, q, off0, max_seq_len=4)
    assert not dq.any() and not dk.any() and not dv.any()
    off = torch.tensor([0, 6], device=dev)
    dq, dk, dv = recir_amd.jagged_hstu_attention_backward(torch.zeros_like(q), q, q, q, off, max_seq_len=8)
    assert not dq.any() and not dk.any() and not dv.any()


def _mid_workload(seed, lengths, targets, ctx=0):
    from recir_amd.workloads import make_jagged

    return make_jagged(lengths, targets, 2, 128, 128, max_seq_len=max(lengths) + 8, alpha=1.0 / 128, dtype="bf16",
                       seed=seed, contextual_seq_len=ctx, tail_rows=5)


@pytest.mark.parametrize("ctx", [0, 70])
def test_tiled_backward_matches_oracle_on_ragged_tiles(oracle, ctx):
    """Lengths around every tile boundary (64, 128), targets straddling tiles, an all-target and an
    empty sequence, contextual keys past one tile."""
    from recir_amd import _lib

    lengths = [1, 63, 64, 65, 127, 128, 129, 0, 191, 257, 330, 90]
    targets = [0, 3, 64, 1, 100, 0, 129, 0, 60, 2, 200, 90]
    wl = _mid_workload(31 + ctx, lengths, targets, ctx)
    g = torch.Generator().manual_seed(9)
    dout = torch.randn(wl.T, wl.H, 128, generator=g).to(torch.bfloat16).float()
    scale = torch.tensor(0.02)
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                           attn_scale=np.float32(0.02), contextual_seq_len=ctx)
    got = run_hip_bwd(wl, dout, attn_scale=scale)
    assert _lib.last_kernel() == "bwd_tiled_d128_bf16"
    assert_grads_close(got, want, int(wl.seq_offsets[-1]), BF16_REL, f"ragged ctx{ctx}")


@pytest.mark.parametrize("A,F,ctx", [(0, 0, 0), (0, 0, 70), (100, 37, 5)])
def test_tiled_backward_with_score_bias(oracle, A, F, ctx):
    """Relative bias rab[h, query - key + N - 1] inside the tiled kernels (plain and semi-local mask),
    a bias large enough that dropping it, or reading it at a shifted index, fails the tolerance."""
    from recir_amd import _lib, ops
    from recir_amd.workloads import make_jagged

    lengths = [1, 63, 64, 65, 127, 128, 129, 0, 191, 257, 330, 90]
    targets = [0, 3, 64, 1, 100, 0, 129, 0, 60, 2, 200, 90]
    wl = make_jagged(lengths, targets, 2, 128, 128, max_seq_len=max(lengths), alpha=1.0 / 128, dtype="bf16",
                     seed=41 + ctx, contextual_seq_len=ctx, tail_rows=5, max_attn_len=A, full_attn_size=F)
    g = torch.Generator().manual_seed(12)
    dout = torch.randn(wl.T, wl.H, 128, generator=g).to(torch.bfloat16).float()
    rab = torch.randn(wl.H, 2 * wl.max_seq_len - 1, generator=g)
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha, rab=rab.numpy(),
                           contextual_seq_len=ctx, max_attn_len=A, full_attn_size=F)
    end = int(wl.seq_offsets[-1])
    got = run_hip_bwd(wl, dout, rab=rab)
    assert _lib.last_kernel() == "bwd_tiled_d128_bf16_rab"
    assert_grads_close(got, want, end, BF16_REL, f"rab A{A} F{F} ctx{ctx}")
    no_bias = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                              wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                              contextual_seq_len=ctx, max_attn_len=A, full_attn_size=F)
    assert error_stats(got[0], no_bias[0])["rel_fro"] > 10 * BF16_REL  # the bias matters at this size
    shifted = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                              wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                              rab=torch.roll(rab, 1, dims=1).numpy(), contextual_seq_len=ctx, max_attn_len=A,
                              full_attn_size=F)
    assert error_stats(got[0], shifted[0])["rel_fro"] > 10 * BF16_REL  # and so does its index
    with ops.force_kernel(ops.KERNEL_GENERIC):
        gotg = run_hip_bwd(wl, dout, rab=rab)
    assert_grads_close(gotg, want, end, BF16_REL, "generic rab")


@pytest.mark.parametrize("with_rab", [False, True])
def test_tiled_backward_with_per_token_scale(oracle, with_rab):
    """attn_scale as a [T] vector (row m of P carries attn_scale[m]) inside the tiled kernels; the
    vector varies by 4x across tokens so that using one value for all rows fails."""
    from recir_amd import _lib

    lengths = [1, 63, 64, 65, 127, 128, 129, 0, 191, 257, 330, 90]
    targets = [0, 3, 64, 1, 100, 0, 129, 0, 60, 2, 200, 90]
    wl = _mid_workload(57, lengths, targets, 3)
    g = torch.Generator().manual_seed(13)
    dout = torch.randn(wl.T, wl.H, 128, generator=g).to(torch.bfloat16).float()
    scale = (0.5 + 1.5 * torch.rand(wl.T, generator=g)) / 300
    rab = torch.randn(wl.H, 2 * wl.max_seq_len - 1, generator=g) if with_rab else None
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                           attn_scale=scale.numpy(), rab=None if rab is None else rab.numpy(), contextual_seq_len=3)
    got = run_hip_bwd(wl, dout, attn_scale=scale, rab=rab)
    assert _lib.last_kernel() == ("bwd_tiled_d128_bf16_rab" if with_rab else "bwd_tiled_d128_bf16")
    assert_grads_close(got, want, int(wl.seq_offsets[-1]), BF16_REL, "per-token scale")
    flat = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                           attn_scale=np.float32(scale.mean().item()), rab=None if rab is None else rab.numpy(),
                           contextual_seq_len=3)
    assert error_stats(got[1], flat[1])["rel_fro"] > 5 * BF16_REL


def test_config3_backward_tiled_agrees_with_generic():
    """Config 3 (bias + contextual prefix) at full size: tiled against generic kernels."""
    from recir_amd import _lib, ops
    from recir_amd.workloads import make_config

    wl = make_config(3)
    g = torch.Generator().manual_seed(5)
    dout = torch.randn(wl.T, wl.H, 128, generator=g)
    got = run_hip_bwd(wl, dout, rab=wl.rab)
    assert _lib.last_kernel() == "bwd_tiled_d128_bf16_rab"
    with ops.force_kernel(ops.KERNEL_GENERIC):
        ref = run_hip_bwd(wl, dout, rab=wl.rab)
    assert _lib.last_kernel() == "bwd_generic_bf16"
    assert_grads_close(got, [r.float().cpu().numpy() for r in ref], int(wl.seq_offsets[-1]), BF16_REL, "config3")


@pytest.mark.timeout(600)
@pytest.mark.parametrize("config", [2, 3, 4])
def test_full_size_backward_matches_oracle(oracle, config):
    """Configurations 2, 3 (bias table + contextual prefix) and 4 (one 8192-token sequence) at full
    size: dq, dk, dv of the tiled MFMA kernels against the fp64 oracle on the same bf16 values."""
    from recir_amd import _lib
    from recir_amd.workloads import make_config

    wl = make_config(config)
    g = torch.Generator().manual_seed(40 + config)
    dout = torch.randn(wl.T, wl.H, 128, generator=g).to(torch.bfloat16).float()
    rab = wl.rab if config == 3 else None
    got = run_hip_bwd(wl, dout, rab=rab)
    assert _lib.last_kernel().startswith("bwd_tiled_d128_bf16")
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                           rab=None if rab is None else rab.numpy(), contextual_seq_len=wl.contextual_seq_len)
    assert_grads_close(got, want[:3], int(wl.seq_offsets[-1]), BF16_REL, f"config{config} backward")


@pytest.mark.parametrize("lengths", [[900] + [70] * 20, [260] * 16], ids=["one_long", "even"])
def test_tiled_backward_with_tiles_and_pairs_dealt(oracle, lengths):
    """The work lists of both backward kernels when single tiles are dealt to the XCDs (one sequence
    far longer than the rest) and when whole (sequence, head) pairs are."""
    from recir_amd import _lib

    wl = _mid_workload(77, lengths, [2] * len(lengths), 0)
    g = torch.Generator().manual_seed(10)
    dout = torch.randn(wl.T, wl.H, 128, generator=g).to(torch.bfloat16).float()
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                           attn_scale=np.float32(0.02), contextual_seq_len=0)
    got = run_hip_bwd(wl, dout, attn_scale=torch.tensor(0.02))
    assert _lib.last_kernel() == "bwd_tiled_d128_bf16"
    assert_grads_close(got, want, int(wl.seq_offsets[-1]), BF16_REL, f"lengths {lengths[:2]}")


def test_tiled_backward_agrees_with_generic_at_full_size():
    """Config 2 (B=32, up to 2048 tokens per sequence): the tiled MFMA kernels against the generic
    fp32-arithmetic kernels on the same bf16 tensors."""
    from recir_amd import _lib, ops
    from recir_amd.workloads import make_config

    wl = make_config(2)
    g = torch.Generator().manual_seed(3)
    dout = torch.randn(wl.T, wl.H, 128, generator=g)
    got = run_hip_bwd(wl, dout)
    assert _lib.last_kernel() == "bwd_tiled_d128_bf16"
    with ops.force_kernel(ops.KERNEL_GENERIC):
        ref = run_hip_bwd(wl, dout)
    assert _lib.last_kernel() == "bwd_generic_bf16"
    end = int(wl.seq_offsets[-1])
    assert_grads_close(got, [r.float().cpu().numpy() for r in ref], end, BF16_REL, "config2")


@pytest.mark.parametrize("A,F,ctx", [(64, 0, 0), (100, 37, 0), (33, 200, 0), (128, 64, 5)])
def test_semilocal_backward_matches_oracle(oracle, A, F, ctx):
    from recir_amd import _lib, ops
    from recir_amd.workloads import make_jagged

    wl = make_jagged([1, 63, 64, 65, 127, 129, 0, 300, 517, 90], [0, 3, 64, 1, 100, 0, 0, 60, 130, 90], 2, 128, 128,
                     max_seq_len=520, alpha=1.0 / 128, dtype="bf16", seed=60 + A, contextual_seq_len=ctx,
                     tail_rows=3, max_attn_len=A, full_attn_size=F)
    g = torch.Generator().manual_seed(4)
    dout = torch.randn(wl.T, wl.H, 128, generator=g).to(torch.bfloat16).float()
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                           contextual_seq_len=ctx, max_attn_len=A, full_attn_size=F)
    end = int(wl.seq_offsets[-1])
    got = run_hip_bwd(wl, dout)
    assert _lib.last_kernel() == "bwd_tiled_d128_bf16"
    assert_grads_close(got, want, end, BF16_REL, f"A{A} F{F}")
    with ops.force_kernel(ops.KERNEL_GENERIC):
        gotg = run_hip_bwd(wl, dout)
    assert_grads_close(gotg, want, end, BF16_REL, f"generic A{A} F{F}")


def _random_case(seed):
    """A seeded draw over everything the tiled kernels branch on: batch shape, lengths around tile
    boundaries, target counts, contextual prefix, semi-local window, bias, kind of output scale."""
    from recir_amd.workloads import make_jagged

    rng = np.random.default_rng(1000 + seed)
    B = int(rng.integers(1, 7))
    edges = np.array([0, 1, 31, 32, 33, 63, 64, 65, 127, 128, 129, 191, 192, 255, 256, 257])
    lengths = [int(rng.choice(edges)) if rng.random() < 0.5 else int(rng.integers(0, 420)) for _ in range(B)]
    targets = [int(rng.integers(0, n + 1)) if rng.random() < 0.6 else 0 for n in lengths]
    H = int(rng.integers(1, 4))
    ctx = int(rng.choice([0, 0, 3, 70]))
    A = int(rng.choice([0, 0, 33, 128]))
    F = int(rng.choice([0, 40])) if A else 0
    with_rab = bool(rng.random() < 0.4)
    scale_kind = str(rng.choice(["default", "scalar", "per_token"]))
    N = max(max(lengths), 1) + int(rng.integers(0, 9))
    # (seeds from 24 on also draw the mask type; the first 24 keep the cases they always had)
    mask_type = "full" if seed >= 24 and rng.random() < 0.2 else "lower_triangular"
    wl = make_jagged(lengths, targets, H, 128, 128, max_seq_len=N, alpha=1.0 / 128, dtype="bf16", seed=seed,
                     contextual_seq_len=ctx, tail_rows=int(rng.integers(0, 4)), max_attn_len=A, full_attn_size=F,
                     with_rab=with_rab, rab_std=0.5, mask_type=mask_type)
    g = torch.Generator().manual_seed(seed)
    scale = None
    if scale_kind == "scalar":
        scale = torch.tensor(0.01)
    elif scale_kind == "per_token":
        scale = (0.5 + torch.rand(wl.T, generator=g)) / 100
    dout = torch.randn(wl.T, wl.H, 128, generator=g).to(torch.bfloat16).float()
    return wl, scale, dout


@pytest.mark.parametrize("seed", range(48))
def test_randomized_cases_forward_and_backward(oracle, seed):
    """Forward and backward of the tiled kernels against the oracle on seeded random cases."""
    from recir_amd import _lib
    from tests.parity_util import assert_bf16_close, run_hip, run_oracle

    wl, scale, dout = _random_case(seed)
    what = (f"seed {seed}: lengths {wl.lengths.tolist()} targets {wl.num_targets.tolist()} H {wl.H} ctx "
            f"{wl.contextual_seq_len} A {wl.max_attn_len} F {wl.full_attn_size} rab {wl.rab is not None} mask {wl.mask_type}")
    causal = wl.mask_type == "lower_triangular"
    out = run_hip(wl, attn_scale=scale)
    if wl.T:
        assert _lib.last_kernel().startswith("tiled_d128" if causal else "mfma_bf16_d128"), what
    assert_bf16_close(out, run_oracle(oracle, wl, attn_scale=scale), what)
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                           attn_scale=_scale_np(scale), rab=None if wl.rab is None else wl.rab.numpy(),
                           contextual_seq_len=wl.contextual_seq_len, max_attn_len=wl.max_attn_len,
                           full_attn_size=wl.full_attn_size, mask_type=wl.mask_type)
    got = run_hip_bwd(wl, dout, attn_scale=scale, rab=wl.rab)
    if wl.T:
        assert _lib.last_kernel().startswith("bwd_tiled_d128" if causal else "bwd_mfma_bf16_d128"), what
    if want[0].size and np.abs(want[0]).max() > 0:
        assert_grads_close(got, want, int(wl.seq_offsets[-1]), BF16_REL, what)


@pytest.mark.parametrize("case", ["tiled", "tiled_semilocal_per_token", "general_fp32", "general_fp32_elems", "generic_fp32", "config3"])
def test_gradient_of_the_bias_table(oracle, case):
    """d rab[h, m - j + N - 1] = sum of dS(m, j) (no counterpart in the reference, which has no bias;
    the oracle's form is pinned by torch autograd through a dense restatement).  Float atomics: the
    tolerance is that of a sum, not bitwise."""
    import recir_amd
    from recir_amd import _lib
    from recir_amd.workloads import make_config, make_jagged

    scale = None
    if case == "tiled":
        wl = make_jagged([300, 129, 64, 1, 0, 517], [40, 129, 0, 0, 0, 6], 2, 128, 128, max_seq_len=600, alpha=1 / 128,
                         dtype="bf16", seed=51, with_rab=True, rab_std=0.5, contextual_seq_len=3, tail_rows=5)
    elif case == "tiled_semilocal_per_token":
        wl = make_jagged([260, 100], [30, 0], 2, 128, 128, max_seq_len=300, alpha=1 / 128, dtype="bf16", seed=52,
                         with_rab=True, rab_std=0.5, max_attn_len=70, full_attn_size=40)
        scale = torch.rand(wl.T, generator=torch.Generator().manual_seed(3)) * 0.01 + 0.001
    elif case in ("general_fp32", "general_fp32_elems", "generic_fp32"):
        # head dims 16 / 24 on fp32 MFMAs; 18 / 22 the same with rows that are not multiples of 16 bytes; above 128 the generic kernels
        dqk, dv = {"general_fp32": (16, 24), "general_fp32_elems": (18, 22), "generic_fp32": (132, 130)}[case]
        wl = make_jagged([70, 0, 5, 33], [9, 0, 5, 1], 2, dqk, dv, max_seq_len=80, alpha=0.2, dtype="fp32", seed=53,
                         with_rab=True, rab_std=0.5, contextual_seq_len=2)
    else:
        wl = make_config(3)
    dout = torch.randn(wl.T, wl.H, wl.v.shape[2], generator=torch.Generator().manual_seed(7))
    if wl.dtype == "bf16":
        dout = dout.bfloat16().float()
    q, k, v, off, nt = to_device(wl)
    sc = None if scale is None else scale.cuda()
    kw = dict(max_seq_len=wl.max_seq_len, alpha=wl.alpha, contextual_seq_len=wl.contextual_seq_len, rab=wl.rab.cuda(),
              max_attn_len=wl.max_attn_len, full_attn_size=wl.full_attn_size)
    dq, dk, dv, drab = recir_amd.jagged_hstu_attention_backward(dout.to(q.device, q.dtype), q, k, v, off, nt, sc,
                                                                rab_grad=True, **kw)
    torch.cuda.synchronize()
    assert _lib.last_kernel().startswith({"general_fp32": "bwd_mfma_fp32_d32", "general_fp32_elems": "bwd_mfma_fp32_d32_elems", "generic_fp32": "bwd_generic_fp32"}.get(case, "bwd_tiled_d128"))
    assert drab.shape == wl.rab.shape and drab.dtype == torch.float32
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                           attn_scale=None if scale is None else scale.numpy(), rab=wl.rab.numpy(),
                           contextual_seq_len=wl.contextual_seq_len, max_attn_len=wl.max_attn_len,
                           full_attn_size=wl.full_attn_size, rab_grad=True)
    tol = 2e-4 if case.endswith("fp32") else BF16_REL
    assert_grads_close((dq, dk, dv), want[:3], int(wl.seq_offsets[-1]), tol, case)
    st = error_stats(drab, want[3])
    print(f"[parity] d rab {case}: {st}", flush=True)
    assert st["ref_max"] > 0 and st["rel_to_max"] <= tol and st["rel_fro"] <= tol, st
    # columns no pair touches stay exactly zero, and the three other gradients are what they are without it
    assert not drab.cpu().numpy()[np.asarray(want[3]) == 0].any()
    dq3, dk3, dv3 = recir_amd.jagged_hstu_attention_backward(dout.to(q.device, q.dtype), q, k, v, off, nt, sc, **kw)
    assert torch.equal(dq, dq3) and torch.equal(dk, dk3) and torch.equal(dv, dv3)


def test_autograd_reaches_a_learned_bias_table(oracle):
    """A bias table that requires grad gets one through the operator's autograd formula."""
    import recir_amd
    from recir_amd.workloads import make_jagged

    wl = make_jagged([200, 77], [20, 0], 2, 128, 128, max_seq_len=256, alpha=1 / 128, dtype="bf16", seed=61,
                     with_rab=True, rab_std=0.5)
    q, k, v, off, nt = to_device(wl)
    rab = wl.rab.cuda().requires_grad_(True)
    q.requires_grad_(True)
    out = recir_amd.jagged_hstu_attention(q, k, v, off, nt, max_seq_len=wl.max_seq_len, alpha=wl.alpha, rab=rab)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(2)).bfloat16()
    out.backward(dout.cuda())
    torch.cuda.synchronize()
    want = oracle.attn_bwd(dout.float().numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha, rab=wl.rab.numpy(),
                           rab_grad=True)
    st = error_stats(rab.grad, want[3])
    assert rab.grad.shape == rab.shape and st["rel_to_max"] <= BF16_REL and st["rel_fro"] <= BF16_REL, st
    assert error_stats(q.grad, want[0])["rel_fro"] <= BF16_REL


def test_backward_with_more_sequences_than_the_single_block_work_list_builder_holds(oracle):
    """1300 sequences: both backward work lists (query tiles with the shifted cut, key tiles in
    reverse order) come from the general builder."""
    from recir_amd import _lib
    from recir_amd.workloads import make_jagged

    rng = np.random.default_rng(15)
    lengths = rng.integers(0, 40, size=1300)
    lengths[11] = 300
    lengths[700] = 129
    targets = np.minimum(rng.integers(0, 4, size=1300), lengths)
    wl = make_jagged(lengths, targets, 2, 128, 128, max_seq_len=320, alpha=1 / 128, dtype="bf16", seed=19)
    dout = torch.randn(wl.T, wl.H, 128, generator=torch.Generator().manual_seed(4)).bfloat16().float()
    got = run_hip_bwd(wl, dout)
    assert _lib.last_kernel().startswith("bwd_tiled_d128")
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha)
    assert_grads_close(got, want, int(wl.seq_offsets[-1]), BF16_REL, "B=1300 backward")


def test_no_sequences_through_the_c_abi_zero_the_outputs():
    """B = 0 with T > 0 rows of padding: the C entry points fill the outputs with zeros (the Python
    front ends reject an offsets tensor without a sequence, as the reference's validator does,
    recir/ops/pallas/jagged_hstu_attention.py:1498-1515)."""
    import ctypes

    from recir_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda:0")
    T, H, D = 5, 2, 128
    x = torch.randn(T, H, D, device=dev).bfloat16()
    off = torch.zeros(1, dtype=torch.int64, device=dev)
    out = torch.full_like(x, float("nan"))
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.recir_hstu_attn_fwd(p(x), p(x), p(x), p(out), p(off), None, None, None, None, None, T, 0, H, D, D, 16, 0, 0, 0,
                                 0.1, _lib.DTYPE_BF16, 0, None, 0, s)
    assert rc == 0, lib.recir_hstu_last_error().decode()
    grads = [torch.full_like(x, float("nan")) for _ in range(3)]
    rc = lib.recir_hstu_attn_bwd(p(x), p(x), p(x), p(x), p(grads[0]), p(grads[1]), p(grads[2]), None, p(off), None, None, None,
                                 T, 0, H, D, D, 16, 0, 0, 0, 0.1, _lib.DTYPE_BF16, 0, None, 0, s)
    assert rc == 0, lib.recir_hstu_last_error().decode()
    torch.cuda.synchronize()
    for t in [out] + grads:
        assert not t.float().abs().any().item() and torch.isfinite(t.float()).all().item()


def test_backward_with_reused_work_lists_repeats_itself(oracle):
    """The key-tile kernel's workgroups draw their items from counters in the workspace and the launch
    puts them back itself: with the work lists reused (no plan kernel between the calls) a second and a
    third call must still visit every item exactly once."""
    import recir_amd
    from recir_amd import ops

    wl = _mid_workload(81, [700, 130, 64, 1, 333, 255] * 11, [9, 0, 64, 1, 40, 0] * 11, 0)  # 41 items per list: more than workgroups
    g = torch.Generator().manual_seed(12)
    dout = torch.randn(wl.T, wl.H, 128, generator=g).to(torch.bfloat16).float()
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                           attn_scale=np.float32(0.02), contextual_seq_len=0)
    q, k, v, off, nt = to_device(wl)
    d = dout.to(q.device, q.dtype)
    with recir_amd.plan_cache_scope():
        before = dict(ops.plan_cache_stats)
        runs = [recir_amd.jagged_hstu_attention_backward(d, q, k, v, off, nt, torch.tensor(0.02),
                                                         max_seq_len=wl.max_seq_len, alpha=wl.alpha) for _ in range(3)]
        torch.cuda.synchronize()
        assert ops.plan_cache_stats["hits"] - before["hits"] == 2
    assert_grads_close(runs[0], want, int(wl.seq_offsets[-1]), BF16_REL, "lists built")
    for later in runs[1:]:
        for a, b in zip(runs[0], later):
            assert torch.equal(a, b)


def test_noncausal_mask_through_autograd_and_with_a_bias(oracle):
    """A mask type other than "lower_triangular": the operator's autograd formula hands the type on to
    the backward operator, and the gradient of a bias table follows the same mask."""
    import recir_amd
    from recir_amd import _lib
    from recir_amd.workloads import make_jagged

    wl = make_jagged([90, 33, 1, 0, 140], [10, 33, 0, 0, 150], 2, 128, 128, max_seq_len=160, alpha=1 / 128,
                     dtype="bf16", seed=71, with_rab=True, rab_std=0.5, contextual_seq_len=2, tail_rows=2,
                     max_attn_len=12, full_attn_size=5, mask_type="full")
    dout = torch.randn(wl.T, wl.H, 128, generator=torch.Generator().manual_seed(9)).bfloat16().float()
    q, k, v, off, nt = to_device(wl)
    q.requires_grad_(True); k.requires_grad_(True); v.requires_grad_(True)
    rab = wl.rab.cuda().requires_grad_(True)
    out = recir_amd.jagged_hstu_attention(q, k, v, off, nt, max_seq_len=wl.max_seq_len, alpha=wl.alpha,
                                          contextual_seq_len=2, rab=rab, max_attn_len=12, full_attn_size=5,
                                          invalid_attn_mask_type="full")
    assert _lib.last_kernel() == "mfma_bf16_d128"
    out.backward(dout.to(out.device, out.dtype))
    torch.cuda.synchronize()  # (the backward ran on autograd's thread: the kernel name kept per thread is not this thread's)
    kw = dict(max_seq_len=wl.max_seq_len, alpha=wl.alpha, rab=wl.rab.numpy(), contextual_seq_len=2, max_attn_len=12,
              full_attn_size=5, mask_type="full")
    ref = oracle.attn_fwd(wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(), wl.num_targets.numpy(), **kw)
    from tests.parity_util import assert_bf16_close
    assert_bf16_close(out.detach(), ref, "non-causal forward")
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), rab_grad=True, **kw)
    assert_grads_close((q.grad, k.grad, v.grad), want[:3], int(wl.seq_offsets[-1]), BF16_REL, "non-causal autograd")
    st = error_stats(rab.grad, want[3])
    print(f"[parity] d rab non-causal: {st}", flush=True)
    assert st["ref_max"] > 0 and st["rel_to_max"] <= BF16_REL and st["rel_fro"] <= BF16_REL, st
    # the causal call on the same tensors differs: the type is not ignored
    out_c = recir_amd.jagged_hstu_attention(q.detach(), k.detach(), v.detach(), off, nt, max_seq_len=wl.max_seq_len,
                                            alpha=wl.alpha, contextual_seq_len=2, rab=wl.rab.cuda(), max_attn_len=12,
                                            full_attn_size=5)
    assert not torch.equal(out_c, out.detach())


def test_a_bias_with_alpha_zero_runs_on_the_general_kernels(oracle):
    """The head-dim-128 kernels keep the bias divided by alpha in their score accumulators; with alpha = 0 the
    scores are the bias alone and the call goes to the general MFMA kernels, forward and backward."""
    from recir_amd import _lib, ops
    from recir_amd.workloads import make_jagged
    from tests.parity_util import assert_bf16_close, run_hip, run_oracle

    wl = make_jagged([150, 64, 1, 0, 200], [20, 64, 0, 0, 7], 2, 128, 128, max_seq_len=256, alpha=0.0, dtype="bf16",
                     seed=81, with_rab=True, rab_std=0.7, contextual_seq_len=2, tail_rows=1)
    out = run_hip(wl)
    assert _lib.last_kernel() == "mfma_bf16_d128"
    assert_bf16_close(out, run_oracle(oracle, wl), "alpha 0 forward")
    dout = torch.randn(wl.T, wl.H, 128, generator=torch.Generator().manual_seed(5)).bfloat16().float()
    got = run_hip_bwd(wl, dout, rab=wl.rab)
    assert _lib.last_kernel() == "bwd_mfma_bf16_d128"
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=0.0, rab=wl.rab.numpy(),
                           contextual_seq_len=2)
    # dq and dk are exactly zero (the scores do not depend on q or k); dv follows the bias
    assert not got[0].float().abs().max().item() and not got[1].float().abs().max().item()
    st = error_stats(got[2], want[2])
    assert st["rel_to_max"] <= BF16_REL and st["rel_fro"] <= BF16_REL, st
    with ops.force_kernel(ops.KERNEL_TILED_DIRECT), pytest.raises(ValueError, match="head-dim-128 backward needs"):
        run_hip_bwd(wl, dout, rab=wl.rab)


@pytest.mark.parametrize("dout_mul,v_mul", [(3.0e4, 1.0e-3), (1.0e-5, 1.0), (1.0, 2.0e3)])
def test_bias_table_gradient_far_from_unit_scale(oracle, dout_mul, v_mul):
    """With a scalar output scale the tiled dQ kernel sums dS along the diagonals as fixed-point
    integers whose scale follows the data (largest |dout| of the item's rows, largest |v| of the call):
    the result must not depend on the magnitude of either."""
    import recir_amd
    from recir_amd import _lib
    from recir_amd.workloads import make_jagged

    wl = make_jagged([300, 129, 64, 1, 0, 517], [40, 129, 0, 0, 0, 6], 2, 128, 128, max_seq_len=600, alpha=1 / 128,
                     dtype="bf16", seed=91, with_rab=True, rab_std=0.5, contextual_seq_len=3, tail_rows=2)
    wl.v.mul_(v_mul)
    wl.v.copy_(wl.v.bfloat16().float())
    dout = (torch.randn(wl.T, wl.H, 128, generator=torch.Generator().manual_seed(11)) * dout_mul).bfloat16().float()
    # a few rows far above the rest: the scale must follow the largest, the small ones keep their share
    dout[5] *= 64.0
    dout = dout.bfloat16().float()
    q, k, v, off, nt = to_device(wl)
    kw = dict(max_seq_len=wl.max_seq_len, alpha=wl.alpha, contextual_seq_len=3, rab=wl.rab.cuda())
    dq, dk, dv, drab = recir_amd.jagged_hstu_attention_backward(dout.to(q.device, q.dtype), q, k, v, off, nt, rab_grad=True, **kw)
    torch.cuda.synchronize()
    assert _lib.last_kernel() == "bwd_tiled_d128_bf16_rab"
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha, rab=wl.rab.numpy(),
                           contextual_seq_len=3, rab_grad=True)
    st = error_stats(drab, want[3])
    print(f"[parity] d rab, dout x {dout_mul:g}, v x {v_mul:g}: {st}", flush=True)
    assert st["ref_max"] > 0 and st["rel_to_max"] <= BF16_REL and st["rel_fro"] <= BF16_REL, st
    assert not drab.cpu().numpy()[np.asarray(want[3]) == 0].any()


@pytest.mark.parametrize("per_token", [False, True])
def test_bias_table_gradient_is_the_same_bit_for_bit_whatever_the_order(oracle, per_token):
    """The tiled kernels sum the table's gradient in fixed point with one scale per head: repeated
    calls, and a call whose work lists are ordered differently (grouped lists), give the same bits --
    the property the reference asks of its kernels (block-size invariance,
    recir/ops/pallas/tests/test_jagged_hstu_attention.py:178-195).  Checked against the oracle too."""
    import recir_amd
    from recir_amd import _lib, ops
    from recir_amd.workloads import make_jagged

    wl = make_jagged([700, 129, 64, 1, 0, 517, 1000, 333], [40, 129, 0, 0, 0, 6, 64, 3], 4, 128, 128, max_seq_len=1024,
                     alpha=1 / 128, dtype="bf16", seed=97, with_rab=True, rab_std=0.5, contextual_seq_len=3, tail_rows=2)
    dout = torch.randn(wl.T, wl.H, 128, generator=torch.Generator().manual_seed(17)).bfloat16().float()
    q, k, v, off, nt = to_device(wl)
    sc = None
    if per_token:
        sc = (torch.rand(wl.T, generator=torch.Generator().manual_seed(18)) * 0.02 + 0.001)
    kw = dict(max_seq_len=wl.max_seq_len, alpha=wl.alpha, contextual_seq_len=3, rab=wl.rab.cuda(),
              attn_scale=None if sc is None else sc.cuda())

    def run():
        out = recir_amd.jagged_hstu_attention_backward(dout.to(q.device, q.dtype), q, k, v, off, nt, rab_grad=True, **kw)
        torch.cuda.synchronize()
        assert _lib.last_kernel() == "bwd_tiled_d128_bf16_rab"
        return out[3].clone()

    first = run()
    for _ in range(4):
        assert torch.equal(run(), first)
    with ops.extra_flags(_lib.FLAG_GROUPED_LISTS):
        assert torch.equal(run(), first)
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha, rab=wl.rab.numpy(),
                           contextual_seq_len=3, rab_grad=True, attn_scale=None if sc is None else sc.numpy())[3]
    st = error_stats(first, want)
    print(f"[parity] d rab, fixed-point table, per_token={per_token}: {st}", flush=True)
    assert st["ref_max"] > 0 and st["rel_to_max"] <= BF16_REL and st["rel_fro"] <= BF16_REL, st


def test_bias_table_gradient_needs_its_workspace():
    """Through the C ABI: with drab the workspace must also hold the fixed-point table; a workspace of
    the plain backward's size is rejected before any launch."""
    import ctypes

    from recir_amd import _lib

    L = _lib.load()
    T, B, H, N = 300, 2, 2, 256
    dev = torch.device("cuda:0")
    z = lambda: torch.zeros(T, H, 128, dtype=torch.bfloat16, device=dev)
    q, k, v, dout, dq, dk, dv = (z() for _ in range(7))
    off = torch.tensor([0, 200, 300], dtype=torch.int64, device=dev)
    rab = torch.zeros(H, 2 * N - 1, dtype=torch.float32, device=dev)
    drab = torch.empty_like(rab)
    plain = L.recir_hstu_attn_bwd_workspace_bytes(T, B, H, 128, 128, _lib.DTYPE_BF16)
    extra = L.recir_hstu_attn_bwd_rab_grad_workspace_bytes(H, N)
    assert extra >= H * (2 * N - 1) * 8
    ws = torch.empty(plain + extra, dtype=torch.uint8, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    def call(nbytes):
        return L.recir_hstu_attn_bwd(dout.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                                     dv.data_ptr(), drab.data_ptr(), off.data_ptr(), None, rab.data_ptr(), None, T, B, H, 128, 128,
                                     N, 0, 0, 0, 1 / 128, _lib.DTYPE_BF16, 0, ws.data_ptr(), nbytes, st)

    assert call(plain) == -3 and "recir_hstu_attn_bwd_rab_grad_workspace_bytes" in _lib.last_error()
    assert call(plain + extra) == 0
    torch.cuda.synchronize()
    assert not drab.any()  # zero inputs: zero gradient, every entry written


def test_bias_table_gradient_with_one_outlier_in_v(oracle):
    """One value of v a thousand times the rest coarsens the fixed-point resolution of every item (the
    scale follows the call's largest |v|); the terms are rounded to nearest, so what is left is noise
    without a sign: the table's gradient stays inside the bf16 bounds, whole tensor and per head."""
    import recir_amd
    from recir_amd import _lib
    from recir_amd.workloads import make_jagged

    wl = make_jagged([300, 129, 64, 517], [40, 129, 0, 6], 2, 128, 128, max_seq_len=600, alpha=1 / 128,
                     dtype="bf16", seed=93, with_rab=True, rab_std=0.5, contextual_seq_len=3, tail_rows=2)
    wl.v[401, 1, 17] = 1.0e3
    dout = torch.randn(wl.T, wl.H, 128, generator=torch.Generator().manual_seed(13)).bfloat16().float()
    q, k, v, off, nt = to_device(wl)
    kw = dict(max_seq_len=wl.max_seq_len, alpha=wl.alpha, contextual_seq_len=3, rab=wl.rab.cuda())
    drab = recir_amd.jagged_hstu_attention_backward(dout.to(q.device, q.dtype), q, k, v, off, nt, rab_grad=True, **kw)[3]
    torch.cuda.synchronize()
    assert _lib.last_kernel() == "bwd_tiled_d128_bf16_rab"
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha, rab=wl.rab.numpy(),
                           contextual_seq_len=3, rab_grad=True)[3]
    st = error_stats(drab, want)
    print(f"[parity] d rab with one outlier in v: {st}", flush=True)
    assert st["rel_to_max"] <= BF16_REL and st["rel_fro"] <= BF16_REL and st["worst_row_rel"] <= BF16_REL, st
    # no bias towards zero: the summed error is small against the summed magnitude
    err = drab.double().cpu().numpy() - np.asarray(want, dtype=np.float64)
    assert abs(err.sum()) <= 1e-3 * np.abs(want).sum(), (err.sum(), np.abs(want).sum())


def test_bias_table_gradient_of_non_finite_input_is_not_finite():
    """A NaN in dout must not come out as a plausible number (the fixed-point sums cannot carry it: the
    scale is then zero and the flushed values are NaN)."""
    import recir_amd
    from recir_amd.workloads import make_jagged

    wl = make_jagged([200, 70], [10, 0], 2, 128, 128, max_seq_len=256, alpha=1 / 128, dtype="bf16", seed=92,
                     with_rab=True, rab_std=0.5)
    dout = torch.randn(wl.T, wl.H, 128, generator=torch.Generator().manual_seed(12)).bfloat16()
    dout[17, 1, 5] = float("nan")
    q, k, v, off, nt = to_device(wl)
    out = recir_amd.jagged_hstu_attention_backward(dout.cuda(), q, k, v, off, nt, rab_grad=True, max_seq_len=256,
                                                   alpha=1 / 128, rab=wl.rab.cuda())
    torch.cuda.synchronize()
    assert torch.isnan(out[3][1]).any()  # head 1 holds the NaN
    assert torch.isfinite(out[3][0]).all()  # head 0 is untouched by it
