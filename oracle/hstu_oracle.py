"""CPU oracle for the HSTU jagged attention forward.  TEST INFRASTRUCTURE ONLY.

Only tests, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module; the product package never does.

Two independent restatements of the reference live here:

* ``attn_fwd``  -- ctypes front end of ``hstu_oracle.c`` (per-sequence loop form,
  follows recir/ops/kjt_split_per_feature.cpp:602-693).
* ``attn_fwd_padded`` -- numpy pad-then-compute form (follows
  recir/ops/helion/jagged_hstu_attention.py:154-257: jagged->padded, einsum,
  silu, keep mask, einsum, padded->jagged).

plus ``ref_op`` which loads the reference's own C++ operator when
``oracle/_ref/libkjt_ref.so`` has been built (``make -C oracle ref``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "libhstu_oracle.so")
_REF_SO = os.path.join(_HERE, "_ref", "libkjt_ref.so")

CTX_PREFIX = 0  # keys j < contextual_seq_len are visible to every query
CTX_REFCPP = 1  # reference C++ rule: keys whose clamped id is 0 are visible
MASK_NONCAUSAL = 2  # added to a ctx mode: the mask of a mask type other than "lower_triangular"


def _mode(ctx_mode, mask_type):
    return int(ctx_mode) | (0 if mask_type == "lower_triangular" else MASK_NONCAUSAL)

_lib = None


def build(force: bool = False) -> str:
    """Compile the C oracle (and, when the reference checkout is present, _ref)."""
    if force or not os.path.exists(_SO):
        subprocess.check_call(["make", "-C", _HERE, "libhstu_oracle.so"] + (["-B"] if force else []))
    return _SO


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(_SO)
        i64, c_int, dbl = ctypes.c_int64, ctypes.c_int, ctypes.c_double
        vp = ctypes.c_void_p
        for name in ("hstu_oracle_keep", "hstu_oracle_keep_clamp_id"):
            fn = getattr(L, name)
            fn.argtypes = [i64, i64, i64, i64, i64, c_int]
            fn.restype = c_int
        L.hstu_oracle_count_pairs.argtypes = [i64, i64, i64, c_int]
        L.hstu_oracle_count_pairs.restype = i64
        L.hstu_oracle_attn_fwd.argtypes = [vp, vp, vp, vp, vp, vp, vp, c_int, vp,
                                           i64, i64, i64, i64, i64, i64, i64, c_int, dbl, c_int]
        L.hstu_oracle_attn_fwd.restype = c_int
        L.hstu_oracle_attn_bwd.argtypes = [vp] * 10 + [c_int, vp] + [i64] * 7 + [c_int, ctypes.c_double, c_int]
        L.hstu_oracle_attn_bwd.restype = c_int
        L.hstu_oracle_attn_fwd_sl.argtypes = L.hstu_oracle_attn_fwd.argtypes + [i64, i64]
        L.hstu_oracle_attn_fwd_sl.restype = c_int
        L.hstu_oracle_attn_bwd_sl.argtypes = L.hstu_oracle_attn_bwd.argtypes + [i64, i64]
        L.hstu_oracle_attn_bwd_sl.restype = c_int
        L.hstu_oracle_attn_bwd_rab.argtypes = [vp] * 11 + [c_int, vp] + [i64] * 7 + [c_int, ctypes.c_double, c_int, i64, i64]
        L.hstu_oracle_attn_bwd_rab.restype = c_int
        for name in ("hstu_oracle_keep_sl", "hstu_oracle_keep_sl_clamp_id", "hstu_oracle_keep_nc",
                     "hstu_oracle_keep_nc_clamp_id"):
            fn = getattr(L, name)
            fn.argtypes = [i64, i64, i64, i64, i64, c_int, i64, i64]
            fn.restype = c_int
        L.hstu_oracle_count_pairs_sl.argtypes = [i64, i64, i64, c_int, i64, i64]
        L.hstu_oracle_count_pairs_sl.restype = i64
        L.hstu_oracle_e4m3_encode.argtypes = [ctypes.c_float]
        L.hstu_oracle_e4m3_encode.restype = ctypes.c_uint8
        L.hstu_oracle_e4m3_decode.argtypes = [ctypes.c_uint8]
        L.hstu_oracle_e4m3_decode.restype = ctypes.c_float
        L.hstu_oracle_quant_e4m3_per_head.argtypes = [vp, vp, vp, i64, i64, i64]
        L.hstu_oracle_quant_e4m3_per_head.restype = None
        _lib = L
    return _lib


def keep(m, j, n, t, ctx=0, ctx_mode=CTX_PREFIX) -> bool:
    return bool(lib().hstu_oracle_keep(m, j, n, t, ctx, ctx_mode))


def keep_sl(m, j, n, t, ctx=0, ctx_mode=CTX_PREFIX, max_attn_len=0, full_attn_size=0,
            mask_type="lower_triangular") -> bool:
    return bool(lib().hstu_oracle_keep_sl(m, j, n, t, ctx, _mode(ctx_mode, mask_type), max_attn_len, full_attn_size))


def keep_sl_clamp_id(m, j, n, t, ctx=0, ctx_mode=CTX_PREFIX, max_attn_len=0, full_attn_size=0,
                     mask_type="lower_triangular") -> bool:
    return bool(lib().hstu_oracle_keep_sl_clamp_id(m, j, n, t, ctx, _mode(ctx_mode, mask_type), max_attn_len,
                                                   full_attn_size))


def keep_nc(m, j, n, t, ctx=0, ctx_mode=CTX_PREFIX, max_attn_len=0, full_attn_size=0) -> bool:
    """Mask of a mask type other than "lower_triangular", in words."""
    return bool(lib().hstu_oracle_keep_nc(m, j, n, t, ctx, ctx_mode, max_attn_len, full_attn_size))


def keep_nc_clamp_id(m, j, n, t, ctx=0, ctx_mode=CTX_PREFIX, max_attn_len=0, full_attn_size=0) -> bool:
    """The same mask built the way the reference builds it."""
    return bool(lib().hstu_oracle_keep_nc_clamp_id(m, j, n, t, ctx, ctx_mode, max_attn_len, full_attn_size))


def count_pairs_sl(n, t, ctx=0, ctx_mode=CTX_PREFIX, max_attn_len=0, full_attn_size=0,
                   mask_type="lower_triangular") -> int:
    return int(lib().hstu_oracle_count_pairs_sl(n, t, ctx, _mode(ctx_mode, mask_type), max_attn_len, full_attn_size))


def keep_clamp_id(m, j, n, t, ctx=0, ctx_mode=CTX_PREFIX) -> bool:
    return bool(lib().hstu_oracle_keep_clamp_id(m, j, n, t, ctx, ctx_mode))


def count_pairs(n, t, ctx=0, ctx_mode=CTX_PREFIX) -> int:
    return int(lib().hstu_oracle_count_pairs(n, t, ctx, ctx_mode))


def _f32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def attn_fwd(q, k, v, seq_offsets, num_targets=None, *, max_seq_len, alpha, attn_scale=None,
             rab=None, contextual_seq_len=0, ctx_mode=CTX_PREFIX, round_p_bf16=False,
             max_attn_len=0, full_attn_size=0, mask_type="lower_triangular"):
    """Per-sequence loop oracle.  q,k [T,H,Dqk], v [T,H,Dv] float arrays -> out [T,H,Dv] float32.

    ``attn_scale``: None (1/max_seq_len), a python/0-d scalar, or a [T] per-token array.
    ``mask_type``: "lower_triangular" is the causal mask, any other string the reference's other
    branch (absolute distances; kjt_split_per_feature.cpp:650-660).
    """
    q, k, v = _f32(q), _f32(k), _f32(v)
    T, H, Dqk = q.shape
    Dv = v.shape[2]
    assert k.shape == q.shape and v.shape[:2] == (T, H)
    off = np.ascontiguousarray(np.asarray(seq_offsets, dtype=np.int64))
    B = off.shape[0] - 1
    nt = None if num_targets is None else np.ascontiguousarray(np.asarray(num_targets, dtype=np.int64))
    if nt is not None:
        assert nt.shape == (B,)
    rb = None
    if rab is not None:
        rb = _f32(rab)
        assert rb.shape == (H, 2 * max_seq_len - 1)
    kind, sc = 0, None
    if attn_scale is not None:
        sc = _f32(attn_scale).reshape(-1)
        kind = 1 if sc.size == 1 and np.ndim(attn_scale) == 0 else 2
        if kind == 2:
            assert sc.shape == (T,)
    out = np.empty((T, H, Dv), dtype=np.float32)
    rc = lib().hstu_oracle_attn_fwd_sl(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(off), _ptr(nt),
                                       _ptr(rb), kind, _ptr(sc), T, B, H, Dqk, Dv, int(max_seq_len),
                                       int(contextual_seq_len), _mode(ctx_mode, mask_type), float(alpha),
                                       1 if round_p_bf16 else 0, int(max_attn_len), int(full_attn_size))
    if rc != 0:
        raise ValueError("invalid jagged range in seq_offsets")
    return out


def attn_bwd(dout, q, k, v, seq_offsets, num_targets=None, *, max_seq_len, alpha, attn_scale=None,
             rab=None, contextual_seq_len=0, ctx_mode=CTX_PREFIX, round_bf16=False,
             max_attn_len=0, full_attn_size=0, rab_grad=False, mask_type="lower_triangular"):
    """Gradients (dq, dk, dv) of ``attn_fwd`` for the upstream gradient ``dout`` [T,H,Dv]; float32 arrays.

    Same argument conventions as ``attn_fwd``.  ``round_bf16`` rounds P and dS to bf16 before the
    products that consume them (what a bf16 kernel does).  With ``rab_grad`` a fourth array is
    returned, the gradient of the bias table ``[H, 2*max_seq_len-1]`` in float64 (the sum of dS over
    the kept pairs of every diagonal; no counterpart in the reference).
    """
    dout, q, k, v = _f32(dout), _f32(q), _f32(k), _f32(v)
    T, H, Dqk = q.shape
    Dv = v.shape[2]
    assert k.shape == q.shape and v.shape[:2] == (T, H) and dout.shape == v.shape
    off = np.ascontiguousarray(np.asarray(seq_offsets, dtype=np.int64))
    B = off.shape[0] - 1
    nt = None if num_targets is None else np.ascontiguousarray(np.asarray(num_targets, dtype=np.int64))
    rb = None
    if rab is not None:
        rb = _f32(rab)
        assert rb.shape == (H, 2 * max_seq_len - 1)
    kind, sc = 0, None
    if attn_scale is not None:
        sc = _f32(attn_scale).reshape(-1)
        kind = 1 if sc.size == 1 and np.ndim(attn_scale) == 0 else 2
        if kind == 2:
            assert sc.shape == (T,)
    dq = np.empty((T, H, Dqk), dtype=np.float32)
    dk = np.empty((T, H, Dqk), dtype=np.float32)
    dv = np.empty((T, H, Dv), dtype=np.float32)
    drab = None
    if rab_grad:
        if rb is None:
            raise ValueError("rab_grad needs rab")
        drab = np.zeros((H, 2 * max_seq_len - 1), dtype=np.float64)
    rc = lib().hstu_oracle_attn_bwd_rab(_ptr(dout), _ptr(q), _ptr(k), _ptr(v), _ptr(dq), _ptr(dk), _ptr(dv),
                                        _ptr(drab), _ptr(off), _ptr(nt), _ptr(rb), kind, _ptr(sc), T, B, H, Dqk, Dv,
                                        int(max_seq_len), int(contextual_seq_len), _mode(ctx_mode, mask_type),
                                        float(alpha), 1 if round_bf16 else 0, int(max_attn_len),
                                        int(full_attn_size))
    if rc != 0:
        raise ValueError("invalid jagged range in seq_offsets")
    if rab_grad:
        return dq, dk, dv, drab
    return dq, dk, dv


def keep_mask_dense(max_seq_len, lengths, num_targets, contextual_seq_len=0):
    """[B,N,N] bool keep mask, vectorised (helion:185-208) + prefix-mode contextual keys."""
    N = max_seq_len
    lengths = np.asarray(lengths, dtype=np.int64)
    B = lengths.shape[0]
    ids = np.arange(N)
    if num_targets is None:
        cap = lengths.reshape(B, 1, 1)
    else:
        cap = (lengths - np.asarray(num_targets, dtype=np.int64)).reshape(B, 1, 1)
    row = ids.reshape(1, N, 1)
    col = ids.reshape(1, 1, N)
    keepm = ((row >= col) & (col < cap)) | (row == col)
    if contextual_seq_len > 0:
        keepm = keepm | (col < contextual_seq_len)
    inb = (row < lengths.reshape(B, 1, 1)) & (col < lengths.reshape(B, 1, 1))
    return keepm & inb


def attn_fwd_padded(q, k, v, seq_offsets, num_targets=None, *, max_seq_len, alpha, attn_scale=None,
                    rab=None, contextual_seq_len=0):
    """Pad-then-compute oracle in float64 numpy (prefix-mode contextual keys only)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    T, H, Dqk = q.shape
    Dv = v.shape[2]
    off = np.asarray(seq_offsets, dtype=np.int64)
    B = off.shape[0] - 1
    N = int(max_seq_len)
    lengths = off[1:] - off[:-1]

    def pad(x):
        D = x.shape[2]
        o = np.zeros((B, N, H, D))
        for b in range(B):
            n = min(int(lengths[b]), N)
            o[b, :n] = x[off[b]:off[b] + n]
        return o.transpose(0, 2, 1, 3)  # [B,H,N,D]

    pq, pk, pv = pad(q), pad(k), pad(v)
    s = np.einsum("bhxa,bhya->bhxy", pq, pk) * alpha
    if rab is not None:
        rb = np.asarray(rab, dtype=np.float64)
        idx = np.arange(N).reshape(N, 1) - np.arange(N).reshape(1, N) + N - 1
        s = s + rb[:, idx][None]
    p = s / (1.0 + np.exp(-s))
    if attn_scale is None:
        p = p / N
    elif np.ndim(attn_scale) == 0:
        p = p * float(attn_scale)
    else:
        sc = np.asarray(attn_scale, dtype=np.float64)
        psc = np.zeros((B, N))
        for b in range(B):
            n = min(int(lengths[b]), N)
            psc[b, :n] = sc[off[b]:off[b] + n]
        p = p * psc[:, None, :, None]
    km = keep_mask_dense(N, lengths, num_targets, contextual_seq_len)
    p = p * km[:, None]
    o = np.einsum("bhxy,bhyd->bhxd", p, pv).transpose(0, 2, 1, 3)  # [B,N,H,Dv]
    out = np.zeros((T, H, Dv))
    for b in range(B):
        n = int(lengths[b])
        out[off[b]:off[b] + n] = o[b, :n]
    return out.astype(np.float32)


def e4m3_encode(x) -> np.ndarray:
    x = _f32(x)
    L = lib()
    return np.array([L.hstu_oracle_e4m3_encode(float(t)) for t in x.reshape(-1)], dtype=np.uint8).reshape(x.shape)


def e4m3_decode(b) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint8)
    L = lib()
    table = np.array([L.hstu_oracle_e4m3_decode(i) for i in range(256)], dtype=np.float32)
    return table[b]


def quant_e4m3_per_head(x):
    """[T,H,D] float -> (codes uint8 [T,H,D], scale float32 [H])."""
    x = _f32(x)
    T, H, D = x.shape
    codes = np.empty((T, H, D), dtype=np.uint8)
    scale = np.empty((H,), dtype=np.float32)
    lib().hstu_oracle_quant_e4m3_per_head(_ptr(x), _ptr(codes), _ptr(scale), T, H, D)
    return codes, scale


def pairs_closed_form(n, t, ctx=0) -> int:
    """Kept pairs of one sequence: h(h+1)/2 + t(h+1) + c(c-1)/2 with h = n - t history tokens.

    The prefix term counts the pairs m < j < c that the causal rule alone would drop; it is valid
    while the prefix lies inside the history (c <= h), which is the only case this form is used for.
    """
    t = min(max(int(t), 0), int(n))
    h = n - t
    c = min(int(ctx), n)
    if c > h:
        raise ValueError("closed form needs contextual_seq_len <= history length")
    return h * (h + 1) // 2 + t * (h + 1) + (c * (c - 1) // 2 if c > 0 else 0)


# --------------------------------------------------------------------------
# The reference's own compiled operator (oracle/_ref), when built.
# --------------------------------------------------------------------------
_ref_loaded = None


def ref_available() -> bool:
    return os.path.exists(_REF_SO)


def ref_op():
    """torch.ops.hammer.triton_ragged_attention_fwd from the reference's C++ translation unit."""
    global _ref_loaded
    import torch

    if _ref_loaded is None:
        if not ref_available():
            raise FileNotFoundError(_REF_SO + " not built (make -C oracle ref)")
        torch.ops.load_library(_REF_SO)
        _ref_loaded = torch.ops.hammer.triton_ragged_attention_fwd
    return _ref_loaded


def ref_attn_fwd(q, k, v, seq_offsets, num_targets=None, *, max_seq_len, alpha, attn_scale=None,
                 contextual_seq_len=0, max_attn_len=0, full_attn_size=0, mask_type="lower_triangular"):
    """Run the reference C++ op on torch CPU tensors; returns out [seq_offsets[-1], H, Dv]."""
    op = ref_op()
    out, _aux = op(int(max_seq_len), float(alpha), q, k, v, seq_offsets, str(mask_type),
                   num_targets, attn_scale, int(max_attn_len), int(contextual_seq_len),
                   int(full_attn_size), 0)
    return out
