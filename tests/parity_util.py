"""Shared helpers of the GPU parity tests: run the HIP operator on a workload, run the oracle on the
same values, compare with the stated tolerances."""
import numpy as np
import torch

# Stated tolerances (output vs the fp32 oracle on identical inputs)
BF16_MAX_ABS = 1e-2   # absolute
BF16_REL = 2e-2       # relative to the largest reference magnitude, and of the Frobenius norm
FP16_REL = 4e-3       # fp16 operands (11 significant bits against bf16's 8): the same three relative bounds
FP8_MAX_ABS = 5e-2
FP32_RTOL, FP32_ATOL = 2e-4, 2e-6


def expected_kernel(dqk, dv, dtype="bf16", *, causal=True, bwd=False, rab=False, alpha=1.0, rab_grad=False, fp8=False,
                    aligned=True):
    """Name of the kernel the library picks for a call (recir_hstu_last_kernel), from the rule in
    include/recir_hstu.h: the head-dim-128 kernels, else the general MFMA kernels (``_elems``: rows that do
    not all start at multiples of 16 bytes), else the generic ones.
    ``aligned``: every tensor of the call starts at a multiple of 16 bytes."""
    pre = "bwd_" if bwd else ""
    if (dtype == "bf16" or fp8) and dqk == dv == 128 and causal and not (rab and alpha == 0) and aligned:
        return pre + "tiled_d128_" + ("fp8qk" if fp8 else "bf16") + ("_rab" if rab else "")
    d = max(dqk, dv)
    per_chunk, top = (4, 128) if dtype == "fp32" else (8, 256)  # elements in 16 bytes; fp32 tiles are twice as wide
    if dtype in ("bf16", "fp16", "fp32") and d <= top:
        by_16 = aligned and dqk % per_chunk == 0 and dv % per_chunk == 0
        return f"{pre}mfma_{dtype}_d{32 if d <= 32 else 64 if d <= 64 else 128 if d <= 128 else 256}{'' if by_16 else '_elems'}"
    return f"{pre}generic_{dtype}"


def to_device(wl, dtype=None):
    dt = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16, "fp8": torch.bfloat16}[dtype or wl.dtype]
    dev = torch.device("cuda:0")
    return (wl.q.to(dev, dt), wl.k.to(dev, dt), wl.v.to(dev, dt), wl.seq_offsets.to(dev),
            wl.num_targets.to(dev))


def run_hip(wl, *, attn_scale=None, num_targets="default", rab="default", ctx="default", dtype=None,
            offsets_dtype=None, fp8=False):
    import recir_amd

    q, k, v, off, nt = to_device(wl, dtype)
    if num_targets != "default":
        nt = num_targets
    if offsets_dtype is not None:
        off = off.to(offsets_dtype)
        nt = None if nt is None else nt.to(offsets_dtype)
    rb = wl.rab if rab == "default" else rab
    if rb is not None:
        rb = rb.to(q.device)
    sc = attn_scale
    if isinstance(sc, torch.Tensor):
        sc = sc.to(q.device)
    fn = recir_amd.jagged_hstu_attention_fp8 if fp8 else recir_amd.jagged_hstu_attention
    out = fn(q, k, v, off, nt, max_seq_len=wl.max_seq_len, alpha=wl.alpha, attn_scale=sc,
             contextual_seq_len=wl.contextual_seq_len if ctx == "default" else ctx, rab=rb,
             max_attn_len=wl.max_attn_len, full_attn_size=wl.full_attn_size,
             **({} if fp8 else {"invalid_attn_mask_type": wl.mask_type}))
    torch.cuda.synchronize()
    return out


def run_oracle(oracle, wl, *, attn_scale=None, num_targets="default", rab="default", ctx="default",
               ctx_mode=0, q=None, k=None, **kw):
    nt = wl.num_targets.numpy() if num_targets == "default" else num_targets
    rb = wl.rab if rab == "default" else rab
    sc = attn_scale
    if isinstance(sc, torch.Tensor):
        sc = sc.numpy() if sc.dim() else np.float32(sc.item())
    elif sc is not None:
        sc = np.float32(sc)
    return oracle.attn_fwd((wl.q if q is None else q).numpy(), (wl.k if k is None else k).numpy(),
                           wl.v.numpy(), wl.seq_offsets.numpy(), nt, max_seq_len=wl.max_seq_len,
                           alpha=wl.alpha, attn_scale=sc, rab=None if rb is None else rb.numpy(),
                           contextual_seq_len=wl.contextual_seq_len if ctx == "default" else ctx,
                           ctx_mode=ctx_mode, max_attn_len=wl.max_attn_len,
                           full_attn_size=wl.full_attn_size, mask_type=wl.mask_type, **kw)


def error_stats(out, ref):
    """Error of ``out`` against ``ref`` over the whole tensor and per row.  A row is one (token, head)
    vector of the last dimension: ``worst_row_rel`` is the largest ``max|err row| / (max|ref row| +
    floor)`` with ``floor`` the smallest non-zero row maximum of the reference, so that a short-prefix
    row of magnitude 1e-4 counts as much as a row of magnitude 1e-2.  The floor is not taken below
    1e-5 of the largest reference magnitude: a gradient row whose only pair sits where silu' crosses
    zero (x = -1.278) is ten orders below its neighbours by cancellation, and its relative error says
    nothing (seen once in 4,300 random cases: row maximum 3e-12 against 1e-2)."""
    out = out.detach().float().cpu().numpy().astype(np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(out - ref)
    ref_max = max(np.abs(ref).max(), 1e-30) if ref.size else 1.0
    fro = np.sqrt((err ** 2).sum() / max((ref ** 2).sum(), 1e-30)) if ref.size else 0.0
    worst_row_rel, row_floor = 0.0, 0.0
    if ref.size and ref.ndim >= 2:
        d = ref.shape[-1]
        row_ref = np.abs(ref).reshape(-1, d).max(axis=1)
        row_err = err.reshape(-1, d).max(axis=1)
        nz = row_ref[row_ref > 0]
        row_floor = max(float(nz.min()), 1e-5 * float(ref_max)) if nz.size else 0.0
        denom = row_ref + row_floor
        ok = denom > 0
        worst_row_rel = float((row_err[ok] / denom[ok]).max()) if ok.any() else 0.0
        if (~ok).any() and row_err[~ok].max() > 0:  # reference rows that are all zero must come out zero
            worst_row_rel = float("inf")
    return dict(max_abs=float(err.max()) if err.size else 0.0,
                rel_to_max=float(err.max() / ref_max) if err.size else 0.0, rel_fro=float(fro),
                worst_row_rel=worst_row_rel, row_floor=row_floor, ref_max=float(ref_max))


def report(what, st):
    """One line per comparison, picked up from a ``pytest -s`` log for the error table."""
    print(f"[parity] {what}: max_abs={st['max_abs']:.3e} rel_to_max={st['rel_to_max']:.3e} "
          f"rel_fro={st['rel_fro']:.3e} worst_row_rel={st['worst_row_rel']:.3e} ref_max={st['ref_max']:.3e}",
          flush=True)


def assert_bf16_close(out, ref, what=""):
    """bf16 tolerance against the fp32 oracle: max-abs 1e-2, 2e-2 relative to the largest reference
    magnitude and of the Frobenius norm, and 2e-2 relative per row (the absolute bound alone says
    nothing where the outputs themselves are below 1e-2, as at the benchmark sizes)."""
    st = error_stats(out, ref)
    report(what, st)
    assert st["max_abs"] <= BF16_MAX_ABS, (what, st)
    assert st["rel_to_max"] <= BF16_REL, (what, st)
    assert st["rel_fro"] <= BF16_REL, (what, st)
    assert st["worst_row_rel"] <= BF16_REL, (what, st)
    return st


def assert_same_zero_structure(out, ref, end_row):
    """Rows after the last sequence are exactly zero, and rows inside sequences are not spuriously
    zeroed (a valid row always keeps its diagonal key)."""
    o = out.detach().float().cpu().numpy()
    assert not o[end_row:].any(), "tail rows must be exactly zero"
    ref = np.asarray(ref)
    ref_zero_rows = ~ref.reshape(ref.shape[0], -1).any(axis=1)
    out_zero_rows = ~o.reshape(o.shape[0], -1).any(axis=1)
    np.testing.assert_array_equal(out_zero_rows[end_row:], ref_zero_rows[end_row:])
