"""GPU parity of the general MFMA kernels (recir_amd/csrc/hstu_mfma_any.h): head dims other than 128
(rows of any length, tensors at any address), Dqk != Dv, fp16, the non-causal mask forms and a bias with
alpha = 0, forward and backward, against the oracle on the same values.  The reference's operator takes any head dims, any float dtype and any mask
string (recir/ops/kjt_split_per_feature.cpp:602-693); its accelerator kernel leaves Dv free
(recir/ops/pallas/jagged_hstu_attention.py:1498-1503)."""
import numpy as np
import pytest
import torch

from tests.parity_util import BF16_REL, FP16_REL, error_stats, report, run_hip, run_oracle, to_device
from tests.test_gpu_bwd import _scale_np, run_hip_bwd

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def oracle():
    from oracle import hstu_oracle

    hstu_oracle.build()
    return hstu_oracle


LENGTHS = [300, 129, 64, 1, 0, 517, 33]
TARGETS = [40, 129, 0, 0, 0, 6, 50]

# (Dqk, Dv): the padded tile is the next of 32, 64, 128, 256 of the larger one; rows that are not multiples
# of 16 bytes (the last five) run on the instantiations for rows aligned to the element only
DIMS = [(64, 64), (32, 32), (8, 8), (24, 40), (96, 96), (64, 128), (128, 64), (256, 256), (200, 72), (136, 128),
        (25, 25), (50, 30), (7, 3), (129, 64), (250, 255)]
# (mask_type, max_attn_len, full_attn_size, contextual_seq_len)
MASKS = {
    "causal": ("lower_triangular", 0, 0, 0),
    "causal_ctx": ("lower_triangular", 0, 0, 5),
    "semilocal": ("lower_triangular", 70, 30, 0),
    "semilocal_ctx": ("lower_triangular", 33, 0, 3),
    "noncausal_window": ("full", 50, 20, 2),
    "noncausal_diagonal": ("full", 0, 0, 0),
}


def _workload(dqk, dv, dtype, mask, seed, with_rab=False, H=2):
    from recir_amd.workloads import make_jagged

    mask_type, A, F, ctx = MASKS[mask]
    return make_jagged(LENGTHS, TARGETS, H, dqk, dv, max_seq_len=600, alpha=1.0 / np.sqrt(dqk), dtype=dtype, seed=seed,
                       with_rab=with_rab, rab_std=0.5, contextual_seq_len=ctx, tail_rows=5, max_attn_len=A,
                       full_attn_size=F, mask_type=mask_type)


FP16_QUANTUM = 2.0 ** -24  # spacing of fp16 below 2^-14: an absolute error no fp16 result can avoid


def _assert_close(out, ref, tol, what):
    """The three relative bounds of the bf16 parity tests; for fp16 results the per-row bound allows the
    absolute spacing of fp16's subnormal range on top (a row that keeps one pair with a score near zero
    is of the order of 1e-6 at these sizes, where fp16 has a handful of bits)."""
    st = error_stats(out, ref)
    report(what, st)
    assert st["rel_to_max"] <= tol and st["rel_fro"] <= tol, (what, st)
    if out.dtype != torch.float16:
        assert st["worst_row_rel"] <= tol, (what, st)
        return
    o = out.detach().float().cpu().numpy().astype(np.float64)
    r = np.asarray(ref, dtype=np.float64)
    d = r.shape[-1]
    row_err = np.abs(o - r).reshape(-1, d).max(axis=1)
    row_ref = np.abs(r).reshape(-1, d).max(axis=1)
    assert (row_err <= tol * (row_ref + st["row_floor"]) + FP16_QUANTUM).all(), (what, st)


def _expected_kernel(dtype, dqk, dv, bwd=False, aligned=True):
    d = max(dqk, dv)
    dp = 32 if d <= 32 else 64 if d <= 64 else 128 if d <= 128 else 256
    per_16 = 4 if dtype == "fp32" else 8
    elems = "" if (aligned and dqk % per_16 == 0 and dv % per_16 == 0) else "_elems"
    return f"{'bwd_' if bwd else ''}mfma_{dtype}_d{dp}{elems}"


@pytest.mark.parametrize("dims", DIMS, ids=lambda d: f"{d[0]}x{d[1]}")
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_forward_head_dims(oracle, dims, dtype):
    from recir_amd import _lib

    dqk, dv = dims
    wl = _workload(dqk, dv, dtype, "causal_ctx", seed=dqk + dv, with_rab=(dqk % 16 == 8))
    out = run_hip(wl)
    assert _lib.last_kernel() == _expected_kernel(dtype, dqk, dv), _lib.last_kernel()
    assert out.dtype == (torch.bfloat16 if dtype == "bf16" else torch.float16)
    ref = run_oracle(oracle, wl)
    _assert_close(out, ref, BF16_REL if dtype == "bf16" else FP16_REL, f"fwd {dtype} {dqk}x{dv}")
    assert not out[int(wl.seq_offsets[-1]):].float().cpu().numpy().any()


@pytest.mark.parametrize("mask", sorted(MASKS))
@pytest.mark.parametrize("dtype,dims", [("bf16", (64, 64)), ("fp16", (128, 128)), ("bf16", (128, 128))])
def test_forward_masks(oracle, mask, dtype, dims):
    from recir_amd import _lib, ops

    wl = _workload(dims[0], dims[1], dtype, mask, seed=11, with_rab=mask.endswith("ctx"))
    g = torch.Generator().manual_seed(5)
    scale = (0.5 + torch.rand(wl.T, generator=g)) / 50 if mask.startswith("semilocal") else None
    with ops.force_kernel(ops.KERNEL_MFMA_GENERAL):
        out = run_hip(wl, attn_scale=scale)
    assert _lib.last_kernel() == _expected_kernel(dtype, *dims)
    ref = run_oracle(oracle, wl, attn_scale=scale)
    _assert_close(out, ref, BF16_REL if dtype == "bf16" else FP16_REL, f"fwd {mask} {dtype} {dims}")
    # the zero rows of the reference (rows that keep no pair cannot exist: a row keeps itself) and the tail
    assert not out[int(wl.seq_offsets[-1]):].float().cpu().numpy().any()


@pytest.mark.parametrize("mask", ["causal_ctx", "semilocal", "noncausal_window"])
@pytest.mark.parametrize("dims", [(32, 32), (64, 64), (128, 128), (20, 12), (128, 64), (36, 100), (18, 22), (5, 127)],
                         ids=lambda d: f"{d[0]}x{d[1]}")
def test_fp32_forward_and_backward(oracle, dims, mask):
    """fp32 tensors on v_mfma_f32_32x32x2_f32 (head dims up to 128; the last two with rows that are not multiples of
    16 bytes): the fp32 tolerances of the generic kernel's tests, forward element-wise and backward on the three
    relative bounds."""
    from recir_amd import _lib
    from tests.test_gpu_bwd import BWD_FP32_TOL, assert_grads_close

    dqk, dv = dims
    wl = _workload(dqk, dv, "fp32", mask, seed=3 * dqk + dv, with_rab=(mask == "causal_ctx"))
    g = torch.Generator().manual_seed(8)
    scale = (0.5 + torch.rand(wl.T, generator=g)) / 50 if mask == "semilocal" else None
    out = run_hip(wl, attn_scale=scale)
    assert _lib.last_kernel() == _expected_kernel("fp32", dqk, dv), _lib.last_kernel()
    assert out.dtype == torch.float32
    ref = run_oracle(oracle, wl, attn_scale=scale)
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=2e-4, atol=2e-6)
    dout = torch.randn(wl.T, wl.H, dv, generator=g)
    got = run_hip_bwd(wl, dout, attn_scale=scale, rab=wl.rab)
    assert _lib.last_kernel() == _expected_kernel("fp32", dqk, dv, bwd=True), _lib.last_kernel()
    want = _backward_reference(oracle, wl, dout, scale)
    assert_grads_close(got, want[:3], int(wl.seq_offsets[-1]), BWD_FP32_TOL, f"fp32 {dims} {mask}")


def test_noncausal_mask_runs_on_the_matrix_cores_by_default(oracle):
    """Neither a forced selector nor the generic kernel: bf16 at head dim 128 under a non-causal mask."""
    from recir_amd import _lib

    wl = _workload(128, 128, "bf16", "noncausal_window", seed=3)
    out = run_hip(wl)
    assert _lib.last_kernel() == "mfma_bf16_d128"
    _assert_close(out, run_oracle(oracle, wl), BF16_REL, "noncausal default")


def test_bias_with_alpha_zero(oracle):
    """alpha = 0: the scores are the bias alone; the head-dim-128 kernels cannot stage bias / alpha."""
    from recir_amd import _lib
    from recir_amd.workloads import make_jagged

    wl = make_jagged([200, 70], [10, 0], 2, 128, 128, max_seq_len=256, alpha=0.0, dtype="bf16", seed=4, with_rab=True,
                     rab_std=1.0)
    out = run_hip(wl)
    assert _lib.last_kernel() == "mfma_bf16_d128"
    _assert_close(out, run_oracle(oracle, wl), BF16_REL, "alpha 0")


def _backward_reference(oracle, wl, dout, scale, rab_grad=False):
    return oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha, attn_scale=_scale_np(scale),
                           rab=None if wl.rab is None else wl.rab.numpy(), contextual_seq_len=wl.contextual_seq_len,
                           max_attn_len=wl.max_attn_len, full_attn_size=wl.full_attn_size, mask_type=wl.mask_type,
                           **({"rab_grad": True} if rab_grad else {}))


def _assert_grads(got, want, end, tol, what):
    for g, w, name in zip(got, want, ("dq", "dk", "dv")):
        _assert_close(g, w, tol, f"{what} {name}")
        assert not g[end:].float().cpu().numpy().any(), (what, name, "tail rows must be zero")


def _upstream(wl, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    d = torch.randn(wl.T, wl.H, wl.v.shape[2], generator=g)
    return (d.bfloat16() if dtype == "bf16" else d.half()).float()


@pytest.mark.parametrize("dims", [(64, 64), (32, 32), (8, 16), (96, 96), (64, 128), (128, 64), (24, 40), (256, 256), (200, 72), (136, 128)],
                         ids=lambda d: f"{d[0]}x{d[1]}")
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_backward_head_dims(oracle, dims, dtype):
    from recir_amd import _lib

    dqk, dv = dims
    wl = _workload(dqk, dv, dtype, "causal_ctx", seed=2 * dqk + dv, with_rab=(dqk % 16 == 8))
    dout = _upstream(wl, dtype, 9)
    got = run_hip_bwd(wl, dout, rab=wl.rab)
    assert _lib.last_kernel() == _expected_kernel(dtype, dqk, dv, bwd=True), _lib.last_kernel()
    want = _backward_reference(oracle, wl, dout, None)
    _assert_grads(got, want[:3], int(wl.seq_offsets[-1]), BF16_REL if dtype == "bf16" else FP16_REL,
                       f"bwd {dtype} {dqk}x{dv}")


@pytest.mark.parametrize("mask", sorted(MASKS))
@pytest.mark.parametrize("dtype,dims", [("bf16", (64, 64)), ("fp16", (128, 128)), ("bf16", (128, 128))])
@pytest.mark.parametrize("scale_kind", ["default", "per_token"])
def test_backward_masks(oracle, mask, dtype, dims, scale_kind):
    from recir_amd import _lib, ops

    wl = _workload(dims[0], dims[1], dtype, mask, seed=21, with_rab=mask.endswith("ctx"))
    g = torch.Generator().manual_seed(6)
    scale = (0.5 + torch.rand(wl.T, generator=g)) / 50 if scale_kind == "per_token" else None
    dout = _upstream(wl, dtype, 10)
    with ops.force_kernel(ops.KERNEL_MFMA_GENERAL):
        got = run_hip_bwd(wl, dout, attn_scale=scale, rab=wl.rab)
    assert _lib.last_kernel() == _expected_kernel(dtype, *dims, bwd=True)
    want = _backward_reference(oracle, wl, dout, scale)
    _assert_grads(got, want[:3], int(wl.seq_offsets[-1]), BF16_REL if dtype == "bf16" else FP16_REL,
                       f"bwd {mask} {dtype} {dims} {scale_kind}")


@pytest.mark.parametrize("case", [("bf16", 64, 64, "causal_ctx"), ("fp16", 96, 40, "semilocal_ctx"), ("fp32", 32, 32, "causal_ctx"),
                                  ("bf16", 128, 128, "noncausal_window"), ("bf16", 256, 256, "causal_ctx"),
                                  ("bf16", 50, 50, "causal_ctx")],
                         ids=lambda c: f"{c[0]}-{c[1]}x{c[2]}-{c[3]}")
@pytest.mark.parametrize("scale_kind", ["default", "per_token"])
def test_gradient_of_the_bias_table(oracle, case, scale_kind):
    """d rab from the dQ pass of the general kernels: dS summed along the diagonals of a tile in LDS as fixed-point
    integers, the band added to the head's 64-bit table per tile.  Against the oracle; columns no pair touches
    stay zero; two calls give the same bits."""
    import recir_amd
    from recir_amd import _lib

    dtype, dqk, dv, mask = case
    wl = _workload(dqk, dv, dtype, mask, seed=41, with_rab=True)
    g = torch.Generator().manual_seed(9)
    scale = (0.5 + torch.rand(wl.T, generator=g)) / 50 if scale_kind == "per_token" else None
    dout = _upstream(wl, dtype, 14) if dtype != "fp32" else torch.randn(wl.T, wl.H, dv, generator=g)
    q, k, v, off, nt = to_device(wl)
    mask_type, A, F, ctx = MASKS[mask]
    grads = recir_amd.jagged_hstu_attention_backward(dout.to(q.device, q.dtype), q, k, v, off, nt,
                                                     None if scale is None else scale.cuda(), rab_grad=True,
                                                     max_seq_len=wl.max_seq_len, alpha=wl.alpha, contextual_seq_len=ctx,
                                                     rab=wl.rab.cuda(), max_attn_len=A, full_attn_size=F,
                                                     invalid_attn_mask_type=mask_type)
    torch.cuda.synchronize()
    assert _lib.last_kernel() == _expected_kernel(dtype, dqk, dv, bwd=True), _lib.last_kernel()
    want = oracle.attn_bwd(dout.numpy(), wl.q.numpy(), wl.k.numpy(), wl.v.numpy(), wl.seq_offsets.numpy(),
                           wl.num_targets.numpy(), max_seq_len=wl.max_seq_len, alpha=wl.alpha, attn_scale=_scale_np(scale),
                           rab=wl.rab.numpy(), contextual_seq_len=ctx, max_attn_len=A, full_attn_size=F, mask_type=mask_type,
                           rab_grad=True)
    tol = {"bf16": BF16_REL, "fp16": FP16_REL, "fp32": 2e-4}[dtype]
    _assert_grads(grads[:3], want[:3], int(wl.seq_offsets[-1]), tol, f"rab grad {case} {scale_kind}")
    drab = grads[3]
    assert drab.shape == wl.rab.shape and drab.dtype == torch.float32
    st = error_stats(drab, want[3])
    report(f"d rab {case} {scale_kind}", st)
    assert st["ref_max"] > 0 and st["rel_to_max"] <= tol and st["rel_fro"] <= tol, st
    assert not drab.cpu().numpy()[np.asarray(want[3]) == 0].any()
    # fixed-point sums: the same bits whatever order the workgroups run in
    again = recir_amd.jagged_hstu_attention_backward(dout.to(q.device, q.dtype), q, k, v, off, nt,
                                                     None if scale is None else scale.cuda(), rab_grad=True,
                                                     max_seq_len=wl.max_seq_len, alpha=wl.alpha, contextual_seq_len=ctx,
                                                     rab=wl.rab.cuda(), max_attn_len=A, full_attn_size=F,
                                                     invalid_attn_mask_type=mask_type)
    assert torch.equal(again[3], drab)


def test_fp16_backward_with_small_per_token_scales(oracle):
    """Per-token scales of the order of 1 / max_seq_len times P or dS fall below fp16's normal range (6e-5):
    the key-stationary kernel multiplies by a power of two taken from the largest scale of the rows it
    streams and divides it out of the fp32 accumulators.  Rows with a single pair (the diagonal-only mask)
    show the difference: their gradient is one product."""
    from recir_amd import _lib

    wl = _workload(64, 24, "fp16", "noncausal_diagonal", seed=31, with_rab=True)
    g = torch.Generator().manual_seed(7)
    scale = (0.5 + torch.rand(wl.T, generator=g)) / 2000
    dout = _upstream(wl, "fp16", 13)
    got = run_hip_bwd(wl, dout, attn_scale=scale, rab=wl.rab)
    assert _lib.last_kernel() == "bwd_mfma_fp16_d64"
    want = _backward_reference(oracle, wl, dout, scale)
    _assert_grads(got, want[:3], int(wl.seq_offsets[-1]), FP16_REL, "fp16 small per-token scales")


def test_general_and_head_dim_128_kernels_agree_at_full_size(oracle):
    """Configuration 2 (the benchmark's shapes) through both MFMA families, forward and backward."""
    from recir_amd import ops
    from recir_amd.workloads import make_config

    wl = make_config(2)
    dout = _upstream(wl, "bf16", 12)
    with ops.force_kernel(ops.KERNEL_TILED_DIRECT):
        a = run_hip(wl, dtype="bf16")
        ga = run_hip_bwd(wl, dout, dtype="bf16")
    with ops.force_kernel(ops.KERNEL_MFMA_GENERAL):
        b = run_hip(wl, dtype="bf16")
        gb = run_hip_bwd(wl, dout, dtype="bf16")
    assert error_stats(b, a.float().cpu().numpy())["rel_to_max"] <= 2 ** -7
    for x, y, name in zip(ga, gb, ("dq", "dk", "dv")):
        st = error_stats(y, x.float().cpu().numpy())
        report(f"config 2 {name}: general against head-dim-128 kernels", st)
        assert st["rel_to_max"] <= BF16_REL and st["rel_fro"] <= BF16_REL, (name, st)


@pytest.mark.parametrize("alpha", [0.0, -0.1, 3.0])
@pytest.mark.parametrize("d", [64, 128, 50])
def test_alpha_zero_negative_and_large_without_a_bias(oracle, d, alpha):
    """alpha = 0 without a bias gives exact zeros (silu(0) = 0) in every kernel family, also where alpha is applied
    to the output rows instead of the scores; a negative and a large alpha match the oracle on the relative bounds
    (the outputs are of the order of 1 at alpha = 3, so no absolute bound here)."""
    from recir_amd.workloads import make_jagged

    wl = make_jagged([300, 70, 5], [20, 0, 5], 2, d, d, max_seq_len=320, alpha=alpha, dtype="bf16", seed=3, tail_rows=2)
    out = run_hip(wl)
    ref = run_oracle(oracle, wl)
    if alpha == 0.0:
        assert not out.float().abs().sum().item() and not np.abs(ref).sum()
        return
    st = error_stats(out, ref)
    report(f"alpha {alpha} head dim {d}", st)
    assert st["rel_to_max"] <= BF16_REL and st["rel_fro"] <= BF16_REL and st["worst_row_rel"] <= BF16_REL, st


def test_tensors_that_start_between_16_byte_multiples(oracle):
    """Contiguous tensors whose first element sits 2 bytes (bf16) or 4 bytes (fp32) past a 16-byte multiple, at
    head dim 128 (not the head-dim-128 kernels' then) and at 64 / 40: the general kernels read such rows in
    pieces aligned to the element only.  Forward and backward, with a bias, its gradient and a per-token scale."""
    import recir_amd
    from recir_amd import _lib
    from tests.test_gpu_bwd import BWD_FP32_TOL, assert_grads_close

    def shifted(t, dt):  # a contiguous tensor of t's values that starts one element past an aligned address
        buf = torch.full((t.numel() + 9,), 7.0, dtype=dt, device="cuda")
        buf[1:1 + t.numel()] = t.reshape(-1).to("cuda", dt)
        return buf, buf[1:1 + t.numel()].view(t.shape)

    for dtype, dqk, dv in (("bf16", 128, 128), ("bf16", 64, 40), ("fp32", 32, 32)):
        dt = torch.bfloat16 if dtype == "bf16" else torch.float32
        wl = _workload(dqk, dv, dtype, "semilocal_ctx", seed=77, with_rab=True)
        g = torch.Generator().manual_seed(9)
        scale = (0.5 + torch.rand(wl.T, generator=g)) / 50
        dout = torch.randn(wl.T, wl.H, dv, generator=g).to(dt).float()
        (_, q), (_, k), (_, v), (_, do) = (shifted(t, dt) for t in (wl.q, wl.k, wl.v, dout))
        assert q.data_ptr() % 16 == dt.itemsize and q.is_contiguous()
        off, nt, rab, sc = wl.seq_offsets.cuda(), wl.num_targets.cuda(), wl.rab.cuda(), scale.cuda()
        kw = dict(max_seq_len=wl.max_seq_len, alpha=wl.alpha, contextual_seq_len=wl.contextual_seq_len, rab=rab,
                  max_attn_len=wl.max_attn_len, full_attn_size=wl.full_attn_size)
        out = recir_amd.jagged_hstu_attention(q, k, v, off, nt, attn_scale=sc, **kw)
        assert _lib.last_kernel() == _expected_kernel(dtype, dqk, dv, aligned=False), _lib.last_kernel()
        ref = run_oracle(oracle, wl, attn_scale=scale)
        if dtype == "bf16":
            _assert_close(out, ref, BF16_REL, f"shifted {dtype} {dqk}x{dv}")
        else:
            np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=2e-4, atol=2e-6)
        got = recir_amd.jagged_hstu_attention_backward(do, q, k, v, off, nt, sc, rab_grad=True, **kw)
        assert _lib.last_kernel() == _expected_kernel(dtype, dqk, dv, bwd=True, aligned=False), _lib.last_kernel()
        want = _backward_reference(oracle, wl, dout, scale, rab_grad=True)
        end = int(wl.seq_offsets[-1])
        assert_grads_close([t.float().cpu() for t in got[:3]], want[:3], end, BF16_REL if dtype == "bf16" else BWD_FP32_TOL,
                           f"shifted {dtype} {dqk}x{dv} backward")
        st = error_stats(got[3], want[3])
        assert st["rel_to_max"] <= (BF16_REL if dtype == "bf16" else 2e-4), st


def test_outputs_between_16_byte_multiples_leave_their_surroundings_alone():
    """The C ABI with every tensor one element past a 16-byte multiple and head dims 25 / 50: the elements
    before and after each output stay as they were (forward and backward write whole rows, nothing else)."""
    import ctypes

    from recir_amd import _lib
    from recir_amd.workloads import make_jagged

    lib = _lib.load()
    wl = make_jagged([130, 64, 7], [9, 0, 7], 2, 25, 50, max_seq_len=130, alpha=0.2, dtype="bf16", seed=5, tail_rows=3)
    dev = torch.device("cuda:0")

    def shifted(shape, values=None):
        n = int(np.prod(shape))
        buf = torch.full((n + 16,), 7.0, dtype=torch.bfloat16, device=dev)
        view = buf[1:1 + n].view(shape)
        if values is not None:
            view.copy_(values.to(dev, torch.bfloat16))
        return buf, view

    T, H, Dqk = wl.q.shape
    Dv = wl.v.shape[2]
    (_, q), (_, k), (_, v) = shifted(wl.q.shape, wl.q), shifted(wl.k.shape, wl.k), shifted(wl.v.shape, wl.v)
    _, dout = shifted(wl.v.shape, torch.randn(wl.v.shape, generator=torch.Generator().manual_seed(2)))
    (ob, out), (qb, dq), (kb, dk), (vb, dv) = shifted(wl.v.shape), shifted(wl.q.shape), shifted(wl.k.shape), shifted(wl.v.shape)
    off, nt = wl.seq_offsets.to(dev), wl.num_targets.to(dev)
    ws = torch.empty(lib.recir_hstu_attn_bwd_workspace_bytes(T, wl.B, H, Dqk, Dv, _lib.DTYPE_BF16), dtype=torch.uint8, device=dev)
    ptr = lambda t: ctypes.c_void_p(0 if t is None else t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    tail = (wl.max_seq_len, 0, 0, 0, wl.alpha, _lib.DTYPE_BF16, 0)
    rc = lib.recir_hstu_attn_fwd(ptr(q), ptr(k), ptr(v), ptr(out), ptr(off), ptr(nt), None, None, None, None, T, wl.B, H, Dqk, Dv,
                                 *tail, ptr(ws), ws.numel(), stream)
    assert rc == 0, lib.recir_hstu_last_error().decode()
    assert _lib.last_kernel() == "mfma_bf16_d64_elems"
    rc = lib.recir_hstu_attn_bwd(ptr(dout), ptr(q), ptr(k), ptr(v), ptr(dq), ptr(dk), ptr(dv), None, ptr(off), ptr(nt), None, None,
                                 T, wl.B, H, Dqk, Dv, *tail, ptr(ws), ws.numel(), stream)
    assert rc == 0, lib.recir_hstu_last_error().decode()
    assert _lib.last_kernel() == "bwd_mfma_bf16_d64_elems"
    torch.cuda.synchronize()
    for name, buf, view in (("out", ob, out), ("dq", qb, dq), ("dk", kb, dk), ("dv", vb, dv)):
        n = view.numel()
        assert (buf[:1] == 7.0).all() and (buf[1 + n:] == 7.0).all(), name
        end = int(wl.seq_offsets[-1])
        assert not view[end:].float().abs().sum().item(), name  # the rows behind the last sequence are zero
        assert (view[:end].float() != 7.0).any(), name


def test_what_still_runs_on_the_generic_kernels():
    """Head dims above 256."""
    import recir_amd
    from recir_amd import _lib
    from recir_amd.workloads import make_jagged

    prev = recir_amd.set_generic_kernel_policy("silent")
    try:
        wl = make_jagged([50, 20], [5, 0], 2, 264, 260, max_seq_len=64, alpha=0.05, dtype="bf16", seed=1)
        run_hip(wl)
        assert _lib.last_kernel() == "generic_bf16"
        q, k, v, off, nt = to_device(wl)
        recir_amd.jagged_hstu_attention_backward(torch.ones_like(v), q, k, v, off, nt, max_seq_len=64, alpha=0.05)
        assert _lib.last_kernel() == "bwd_generic_bf16"
        wl = make_jagged([50, 20], [5, 0], 2, 264, 260, max_seq_len=64, alpha=0.05, dtype="fp16", seed=1)
        out = run_hip(wl)
        assert _lib.last_kernel() == "generic_fp16" and out.dtype == torch.float16
        from oracle import hstu_oracle
        hstu_oracle.build()
        _assert_close(out, run_oracle(hstu_oracle, wl), FP16_REL, "generic fp16")
        dout = _upstream(wl, "fp16", 3)
        got = run_hip_bwd(wl, dout)
        assert _lib.last_kernel() == "bwd_generic_fp16"
        _assert_grads(got, _backward_reference(hstu_oracle, wl, dout, None)[:3], int(wl.seq_offsets[-1]), FP16_REL, "generic fp16 backward")
    finally:
        recir_amd.set_generic_kernel_policy(prev)
