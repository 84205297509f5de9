"""Host side of the HSTU jagged attention (forward and backward): operator registration and front ends.

``recir::hstu_jagged_attention_fwd`` keeps the positional argument list of
``hammer::triton_ragged_attention_fwd`` (recir/ops/kjt_split_per_feature.cpp:780-783) so that
RecIR's ``swap_ops`` (recir/lowering/op_swap.py:78-97), which rewrites only ``node.target``, can
retarget a traced node without touching its arguments.  One trailing optional ``rab`` is added.
The registration follows the pattern of recir/ops/seq_embedding_op.py:83-95, :238-299: a
``torch.library`` FRAGMENT in namespace ``recir``, an opaque device implementation and a fake
(Meta) kernel, which is what recir/lowering/partial_lower.py:414-427 requires to keep the node
inside a lowered region.

There is deliberately no CPU or eager implementation: a CPU tensor, or a missing
``librecir_hstu.so``, raises.
"""
from __future__ import annotations

import collections
import math
import threading
import warnings
from typing import Optional, Tuple

import torch

from . import _lib

KERNEL_AUTO = 0
KERNEL_GENERIC = 1
KERNEL_MFMA_GENERAL = 2  # MFMA kernels for any head dim (multiples of 8), bf16 or fp16, every mask
KERNEL_TILED_DIRECT = 3  # MFMA kernels written for head dim 128 (bf16, fp8 q/k), K/V copied global -> LDS directly

class _CallState(threading.local):
    """Per-thread switches the context managers below set and every launch reads: a thread that
    enters ``reference_contextual_rule()`` or ``force_kernel()`` changes its own calls only."""

    forced_kernel = KERNEL_AUTO
    extra_flags = 0
    ctx_reference_rule = False


_state = _CallState()

# What happens when a bf16 or fp16 call can only run on the generic kernels (one wave per token and head, two
# orders of magnitude slower than the MFMA kernels: head dims above 256): "warn" (once per process and
# reason), "error" (the C ABI rejects the call, RECIR_HSTU_FLAG_TILED_ONLY) or "silent".  fp32 tensors (MFMA
# kernels up to head dim 128) never warn.
_generic_policy = "warn"
_generic_warned = set()


def set_generic_kernel_policy(policy: str) -> str:
    """Choose what a bf16 or fp16 call that only the slow generic kernels cover does: ``"warn"`` (default),
    ``"error"`` or ``"silent"``.  Returns the previous setting."""
    global _generic_policy
    if policy not in ("warn", "error", "silent"):
        raise ValueError("policy must be 'warn', 'error' or 'silent'")
    prev, _generic_policy = _generic_policy, policy
    return prev


def _note_generic(kernel: str, q, v, rab_grad=False) -> None:
    if _generic_policy != "warn" or not kernel.startswith(("generic_bf16", "bwd_generic_bf16", "generic_fp16", "bwd_generic_fp16")):
        return
    if _state.forced_kernel == KERNEL_GENERIC:
        return
    reason = f"head dims {q.shape[2]} / {v.shape[2]} (the MFMA kernels take head dims up to 256)"
    if reason in _generic_warned:
        return
    _generic_warned.add(reason)
    warnings.warn(f"recir HSTU attention ran on the generic kernel ({kernel}), two orders of magnitude slower than the MFMA "
                  f"kernels, because of {reason}; recir_amd.set_generic_kernel_policy('error') rejects such calls, "
                  f"'silent' stops this message", RuntimeWarning, stacklevel=3)


class extra_flags:
    """Context manager for tests and tuning: C-ABI flag bits added to every call of this thread
    (for example ``_lib.FLAG_GROUPED_LISTS``)."""

    def __init__(self, flags: int):
        self.flags = int(flags)

    def __enter__(self):
        self._prev = _state.extra_flags
        _state.extra_flags = self._prev | self.flags
        return self

    def __exit__(self, *exc):
        _state.extra_flags = self._prev
        return False


class force_kernel:
    """Context manager for tests and tuning: pin the kernel variant the C ABI selects (calls of
    this thread)."""

    def __init__(self, variant: int):
        self.variant = int(variant)

    def __enter__(self):
        self._prev = _state.forced_kernel
        _state.forced_kernel = self.variant
        return self

    def __exit__(self, *exc):
        _state.forced_kernel = self._prev
        return False


class reference_contextual_rule:
    """Context manager: use the contextual-prefix rule of the reference C++ fallback
    (kjt_split_per_feature.cpp:672-674: keys whose target-clamped id is 0 are visible to all)
    instead of "keys j < contextual_seq_len are visible to all", for the calls of this thread."""

    def __enter__(self):
        self._prev = _state.ctx_reference_rule
        _state.ctx_reference_rule = True
        return self

    def __exit__(self, *exc):
        _state.ctx_reference_rule = self._prev
        return False


_SCHEMA = (
    "hstu_jagged_attention_fwd(int N, float alpha, Tensor q, Tensor k, Tensor v, "
    "Tensor seq_offsets, str invalid_attn_mask_type, Tensor? num_targets, Tensor? attn_scale, "
    "int max_attn_len, int contextual_seq_len, int full_attn_size, int num_softmax_heads=0, "
    "Tensor? rab=None) -> (Tensor, Tensor)"
)
_FP8_SCHEMA = (
    "hstu_jagged_attention_fp8_fwd(int N, float alpha, Tensor q_fp8, Tensor k_fp8, Tensor v, "
    "Tensor q_scale, Tensor k_scale, Tensor seq_offsets, Tensor? num_targets, Tensor? attn_scale, "
    "int contextual_seq_len, Tensor? rab=None, int max_attn_len=0, int full_attn_size=0, "
    "bool reference_contextual_rule=False) -> (Tensor, Tensor)"
)
_QUANT_SCHEMA = "hstu_quantize_e4m3_per_head(Tensor x, Tensor? seq_offsets=None) -> (Tensor, Tensor)"
_BWD_SCHEMA = (
    "hstu_jagged_attention_bwd(Tensor dout, int N, float alpha, Tensor q, Tensor k, Tensor v, "
    "Tensor seq_offsets, Tensor? num_targets, Tensor? attn_scale, int contextual_seq_len, "
    "Tensor? rab=None, int max_attn_len=0, int full_attn_size=0, "
    "str invalid_attn_mask_type=\"lower_triangular\") -> (Tensor, Tensor, Tensor)"
)

# The reference's own schema (recir/ops/kjt_split_per_feature.cpp:780-783), argument for argument and
# with the reference's contextual rule (:672-674): the operator a swapped graph node is retargeted to.
_REF_SCHEMA = (
    "triton_ragged_attention_fwd(int N, float alpha, Tensor q, Tensor k, Tensor v, "
    "Tensor seq_offsets, str invalid_attn_mask_type, Tensor? num_targets, Tensor? attn_scale, "
    "int max_attn_len, int contextual_seq_len, int full_attn_size, int num_softmax_heads=0) "
    "-> (Tensor, Tensor)"
)
_REF_BWD_SCHEMA = (
    "triton_ragged_attention_bwd(Tensor dout, int N, float alpha, Tensor q, Tensor k, Tensor v, "
    "Tensor seq_offsets, Tensor? num_targets, Tensor? attn_scale, int contextual_seq_len, "
    "int max_attn_len=0, int full_attn_size=0, str invalid_attn_mask_type=\"lower_triangular\") "
    "-> (Tensor, Tensor, Tensor)"
)

# the backward with the gradient of the bias table as a fourth output
_BWD_RAB_SCHEMA = (
    "hstu_jagged_attention_bwd_rab(Tensor dout, int N, float alpha, Tensor q, Tensor k, Tensor v, "
    "Tensor seq_offsets, Tensor? num_targets, Tensor? attn_scale, int contextual_seq_len, "
    "Tensor rab, int max_attn_len=0, int full_attn_size=0, "
    "str invalid_attn_mask_type=\"lower_triangular\") -> (Tensor, Tensor, Tensor, Tensor)"
)

_LIBRARY = torch.library.Library("recir", "FRAGMENT")
_LIBRARY.define(_SCHEMA)
_LIBRARY.define(_FP8_SCHEMA)
_LIBRARY.define(_QUANT_SCHEMA)
_LIBRARY.define(_BWD_SCHEMA)
_LIBRARY.define(_BWD_RAB_SCHEMA)
_LIBRARY.define(_REF_SCHEMA)
_LIBRARY.define(_REF_BWD_SCHEMA)


def _check_common(q, k, v, seq_offsets, num_targets, max_seq_len) -> int:
    """Shape rules of recir/ops/pallas/jagged_hstu_attention.py:1486-1515 (same messages)."""
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q, k, and v must have shape [T, H, D]")
    if q.shape[:2] != k.shape[:2] or q.shape[:2] != v.shape[:2]:
        raise ValueError("q, k, and v must share packed-token and head dimensions")
    if q.shape[2] != k.shape[2]:
        raise ValueError("q and k must share their feature dimension")
    if seq_offsets.dim() != 1 or seq_offsets.shape[0] < 2:
        raise ValueError("seq_offsets must have shape [B + 1]")
    num_sequences = seq_offsets.shape[0] - 1
    if num_targets is not None and tuple(num_targets.shape) != (num_sequences,):
        raise ValueError("num_targets must have shape [B]")
    if max_seq_len <= 0:
        raise ValueError("max_seq_len must be positive")
    return num_sequences


def _index_tensors(seq_offsets, num_targets, dev=None):
    """Offsets and targets as one integer width the kernels read (int64 or int32), on ``dev``.  The
    reference operator accepts them on any device (it copies them to the host,
    recir/ops/kjt_split_per_feature.cpp:623-626), so they are moved rather than rejected: a host
    pointer must never reach a kernel."""
    if seq_offsets.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"seq_offsets must be int32 or int64, got {seq_offsets.dtype}")
    dev = seq_offsets.device if dev is None else dev
    off = seq_offsets.to(dev).contiguous()
    nt = None
    if num_targets is not None:
        if num_targets.dtype not in (torch.int32, torch.int64):
            raise ValueError(f"num_targets must be int32 or int64, got {num_targets.dtype}")
        nt = num_targets.to(device=dev, dtype=off.dtype).contiguous()
    return off, nt, (_lib.FLAG_OFFSETS_I32 if off.dtype == torch.int32 else 0)


def _check_same_device(dev, **tensors):
    """Value tensors must live where q lives (the reference checks the same of its inputs,
    recir/ops/kjt_split_per_feature.cpp:112-114); raised before anything is launched."""
    for name, t in tensors.items():
        if t is not None and t.device != dev:
            raise ValueError(f"{name} is on {t.device}, q on {dev}")


def _prepare(opname, q, k, v, seq_offsets, num_targets, attn_scale, rab, N, ctx_reference=False,
             mask_type="lower_triangular"):
    """Checks and device-side argument tensors shared by the forward and backward launches."""
    dev = q.device
    if dev.type != "cuda":
        raise RuntimeError(
            f"recir::{opname} runs on the GPU only (got a tensor on "
            f"'{dev}'); this package has no CPU path")
    _check_same_device(dev, k=k, v=v)
    B = _check_common(q, k, v, seq_offsets, num_targets, N)
    T, H, _ = q.shape
    off, nt, flags = _index_tensors(seq_offsets, num_targets, dev)
    if _state.ctx_reference_rule or ctx_reference:
        flags |= _lib.FLAG_CTX_REFERENCE
    flags |= (_state.forced_kernel & 0xFF) << _lib.FLAG_KERNEL_SHIFT
    flags |= _state.extra_flags
    if _generic_policy == "error" and q.dtype != torch.float32 and _state.forced_kernel != KERNEL_GENERIC:
        flags |= _lib.FLAG_TILED_ONLY
    if mask_type != "lower_triangular":
        # any other string selects the reference's other branch (kjt_split_per_feature.cpp:650-660)
        flags |= _lib.FLAG_MASK_NONCAUSAL
    sc = None
    if attn_scale is not None:
        sc = attn_scale.to(device=dev, dtype=torch.float32).contiguous()
        if sc.dim() == 0:
            sc = sc.reshape(1)
        elif sc.dim() == 1 and sc.shape[0] == T:
            flags |= _lib.FLAG_SCALE_PER_TOKEN
        else:
            raise ValueError("attn_scale must be a 0-d tensor or have shape [T]")
    rb = None
    if rab is not None:
        if tuple(rab.shape) != (H, 2 * N - 1):
            raise ValueError(f"rab must have shape [H, 2*max_seq_len-1] = [{H}, {2 * N - 1}]")
        rb = rab.to(device=dev, dtype=torch.float32).contiguous()
    return B, off, nt, sc, rb, flags


def _ptr(t):
    return None if t is None else t.data_ptr()


def _raise_status(entry, rc):
    msg = _lib.last_error()
    if rc < 0:
        raise ValueError(f"{entry} rejected the call ({rc}): {msg}")
    raise RuntimeError(f"{entry} launch failed (hipError {rc}): {msg}")


def _check_window(max_attn_len, full_attn_size):
    if max_attn_len < 0 or full_attn_size < 0:
        raise ValueError("max_attn_len and full_attn_size must be non-negative")


# Work lists depend only on the sequence layout, which the layers of one model step share
# (cf. RECIR_HSTU_FLAG_REUSE_PLAN).  On request the operator keeps the workspace of the last few
# layouts and lets later calls with the very same offset tensors skip the list construction.  Off
# by default: an entry is trusted on the identity, storage and version counter of the offset
# tensors, and a write that bypasses the version counter (``t.data.copy_``, a DLPack or numpy
# alias, a kernel torch does not know of, ``set_``) would leave stale lists in use without an error.
# Callers that own their offsets for the length of a step turn it on for that step
# (``with plan_cache_scope(): ...``), which also drops the entries, and the references they hold, at
# the end of the step.
_PLAN_CACHE_ENTRIES = 8
_plan_cache = collections.OrderedDict()
_plan_cache_enabled = False
_plan_cache_lock = threading.Lock()
plan_cache_stats = {"hits": 0, "misses": 0}


def set_plan_cache(enabled: bool) -> None:
    """Enable or disable (the default) the reuse of work lists between calls that pass the same,
    unchanged offset tensors.  Either way the cache is emptied."""
    global _plan_cache_enabled
    with _plan_cache_lock:
        _plan_cache_enabled = bool(enabled)
        _plan_cache.clear()


class plan_cache_scope:
    """Context manager for one model step: work lists are reused by the calls inside it that pass the
    same offset tensors (the layers of the step), and forgotten when it ends."""

    def __enter__(self):
        self._prev = _plan_cache_enabled
        set_plan_cache(True)
        return self

    def __exit__(self, *exc):
        set_plan_cache(self._prev)
        return False


def _tensor_key(t):
    if t is None:
        return None
    return (id(t), t.data_ptr(), t.storage_offset(), t.dtype, tuple(t.shape), t._version)


def _workspace(kind, seq_offsets, num_targets, layout, ws_bytes, dev, stream):
    """Workspace for one launch and the flag to pass with it: a cached one whose lists are valid
    (flag = reuse), or a new one (flag = 0) that is remembered for the next call."""
    size = max(int(ws_bytes), 16)
    # under stream capture a launch is recorded, not run: lists "built" there do not exist yet
    if not _plan_cache_enabled or torch.cuda.is_current_stream_capturing():
        return torch.empty((size,), dtype=torch.uint8, device=dev), 0, None
    try:
        key = (kind, _tensor_key(seq_offsets), _tensor_key(num_targets), layout, dev.index, stream, size)
    except RuntimeError:  # inference tensors carry no version counter: nothing to validate an entry with
        return torch.empty((size,), dtype=torch.uint8, device=dev), 0, None
    with _plan_cache_lock:
        hit = _plan_cache.get(key)
        if hit is not None and hit[0] is seq_offsets and hit[1] is num_targets:
            _plan_cache.move_to_end(key)
            plan_cache_stats["hits"] += 1
            return hit[2], _lib.FLAG_REUSE_PLAN, key
        plan_cache_stats["misses"] += 1
        ws = torch.empty((size,), dtype=torch.uint8, device=dev)
        _plan_cache[key] = (seq_offsets, num_targets, ws)
        while len(_plan_cache) > _PLAN_CACHE_ENTRIES:
            _plan_cache.popitem(last=False)
    return ws, 0, key


def _launch(q, k, v, seq_offsets, num_targets, attn_scale, rab, q_scale, k_scale, N, alpha,
            contextual_seq_len, dtype_code, max_attn_len=0, full_attn_size=0, ctx_reference=False,
            mask_type="lower_triangular") -> torch.Tensor:
    _check_window(max_attn_len, full_attn_size)
    L = _lib.load()
    dev = q.device
    B, off, nt, sc, rb, flags = _prepare("hstu_jagged_attention_fwd", q, k, v, seq_offsets, num_targets,
                                         attn_scale, rab, N, ctx_reference, mask_type)
    T, H, Dqk = q.shape
    Dv = v.shape[2]
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    out = torch.empty((T, H, Dv), dtype=v.dtype, device=dev)
    if T == 0:
        return out
    ws_bytes = L.recir_hstu_attn_fwd_workspace_bytes(T, B, H, Dqk, Dv, dtype_code)
    stream = torch.cuda.current_stream(dev).cuda_stream
    # what the lists depend on besides the offset tensors themselves
    layout = (T, B, H, Dqk, Dv, dtype_code, int(N), int(contextual_seq_len), int(max_attn_len), int(full_attn_size), flags)
    ws, reuse, key = _workspace("fwd", seq_offsets, num_targets, layout, ws_bytes, dev, stream)
    with torch.cuda.device(dev):
        rc = L.recir_hstu_attn_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(off), _ptr(nt), _ptr(rb),
                                   _ptr(sc), _ptr(q_scale), _ptr(k_scale), T, B, H, Dqk, Dv, int(N),
                                   int(contextual_seq_len), int(max_attn_len), int(full_attn_size),
                                   float(alpha), dtype_code, flags | reuse, _ptr(ws), ws.numel(), stream)
    if rc != 0:
        if key is not None:
            with _plan_cache_lock:
                _plan_cache.pop(key, None)
        _raise_status("recir_hstu_attn_fwd", rc)
    _note_generic(_lib.last_kernel(), q, v)
    return out


def _dtype_code(q, k, v):
    if q.dtype == torch.bfloat16:
        code = _lib.DTYPE_BF16
    elif q.dtype == torch.float32:
        code = _lib.DTYPE_FP32
    elif q.dtype == torch.float16:
        code = _lib.DTYPE_FP16
    else:
        raise ValueError(f"q must be bfloat16, float16 or float32, got {q.dtype}")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k and v must share one dtype")
    return code


def _bwd_device(dout, N, alpha, q, k, v, seq_offsets, num_targets, attn_scale, contextual_seq_len,
                rab=None, max_attn_len=0, full_attn_size=0, ctx_reference=False, rab_grad=False,
                mask_type="lower_triangular"):
    _check_window(max_attn_len, full_attn_size)
    L = _lib.load()
    dev = q.device
    code = _dtype_code(q, k, v)
    B, off, nt, sc, rb, flags = _prepare("hstu_jagged_attention_bwd", q, k, v, seq_offsets, num_targets,
                                         attn_scale, rab, N, ctx_reference, mask_type)
    if dout.shape != v.shape:
        raise ValueError("dout must have the shape of v, [T, H, Dv]")
    if dout.device != dev:
        raise ValueError(f"dout is on {dout.device}, q on {dev}")
    T, H, Dqk = q.shape
    Dv = v.shape[2]
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    dout = dout.to(q.dtype).contiguous()
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    drab = None
    if rab_grad:
        if rb is None:
            raise ValueError("the gradient of rab needs rab")
        drab = torch.zeros((H, 2 * int(N) - 1), dtype=torch.float32, device=dev) if T == 0 else \
            torch.empty((H, 2 * int(N) - 1), dtype=torch.float32, device=dev)
    if T == 0:
        return (dq, dk, dv, drab) if rab_grad else (dq, dk, dv)
    ws_bytes = L.recir_hstu_attn_bwd_workspace_bytes(T, B, H, Dqk, Dv, code)
    if rab_grad:  # the fixed-point table of the sums along the diagonals, behind the work lists
        ws_bytes += L.recir_hstu_attn_bwd_rab_grad_workspace_bytes(H, int(N))
    stream = torch.cuda.current_stream(dev).cuda_stream
    layout = (T, B, H, Dqk, Dv, code, int(N), int(contextual_seq_len), int(max_attn_len), int(full_attn_size), flags,
              bool(rab_grad))
    ws, reuse, key = _workspace("bwd", seq_offsets, num_targets, layout, ws_bytes, dev, stream)
    with torch.cuda.device(dev):
        rc = L.recir_hstu_attn_bwd(_ptr(dout), _ptr(q), _ptr(k), _ptr(v), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(drab),
                                   _ptr(off), _ptr(nt), _ptr(rb), _ptr(sc), T, B, H, Dqk, Dv, int(N),
                                   int(contextual_seq_len), int(max_attn_len), int(full_attn_size),
                                   float(alpha), code, flags | reuse, _ptr(ws), ws.numel(), stream)
    if rc != 0:
        if key is not None:
            with _plan_cache_lock:
                _plan_cache.pop(key, None)
        _raise_status("recir_hstu_attn_bwd", rc)
    _note_generic(_lib.last_kernel(), q, v, rab_grad)
    return (dq, dk, dv, drab) if rab_grad else (dq, dk, dv)


def _bwd_op_device(dout, N, alpha, q, k, v, seq_offsets, num_targets, attn_scale, contextual_seq_len,
                   rab=None, max_attn_len=0, full_attn_size=0, invalid_attn_mask_type="lower_triangular"):
    return _bwd_device(dout, N, alpha, q, k, v, seq_offsets, num_targets, attn_scale, contextual_seq_len,
                       rab, max_attn_len, full_attn_size, False, False, invalid_attn_mask_type)


def _bwd_rab_device(dout, N, alpha, q, k, v, seq_offsets, num_targets, attn_scale, contextual_seq_len,
                    rab, max_attn_len=0, full_attn_size=0, invalid_attn_mask_type="lower_triangular"):
    return _bwd_device(dout, N, alpha, q, k, v, seq_offsets, num_targets, attn_scale, contextual_seq_len,
                       rab, max_attn_len, full_attn_size, False, True, invalid_attn_mask_type)


def _fwd_device(N, alpha, q, k, v, seq_offsets, invalid_attn_mask_type, num_targets, attn_scale,
                max_attn_len, contextual_seq_len, full_attn_size, num_softmax_heads=0, rab=None,
                ctx_reference=False):
    # same rejections as the reference fallback (kjt_split_per_feature.cpp:616-622); like it, any
    # mask type other than "lower_triangular" selects its other branch (:650-660)
    if num_softmax_heads != 0:
        raise ValueError("softmax attention heads are unsupported")
    code = _dtype_code(q, k, v)
    out = _launch(q, k, v, seq_offsets, num_targets, attn_scale, rab, None, None, N, alpha,
                  contextual_seq_len, code, max_attn_len, full_attn_size, ctx_reference, invalid_attn_mask_type)
    return out, torch.zeros((1,), dtype=torch.float32, device=q.device)


def _ref_fwd_device(N, alpha, q, k, v, seq_offsets, invalid_attn_mask_type, num_targets, attn_scale,
                    max_attn_len, contextual_seq_len, full_attn_size, num_softmax_heads=0):
    return _fwd_device(N, alpha, q, k, v, seq_offsets, invalid_attn_mask_type, num_targets, attn_scale,
                       max_attn_len, contextual_seq_len, full_attn_size, num_softmax_heads, None, True)


def _ref_bwd_device(dout, N, alpha, q, k, v, seq_offsets, num_targets, attn_scale, contextual_seq_len,
                    max_attn_len=0, full_attn_size=0, invalid_attn_mask_type="lower_triangular"):
    return _bwd_device(dout, N, alpha, q, k, v, seq_offsets, num_targets, attn_scale, contextual_seq_len,
                       None, max_attn_len, full_attn_size, True, False, invalid_attn_mask_type)


def _fp8_fwd_device(N, alpha, q_fp8, k_fp8, v, q_scale, k_scale, seq_offsets, num_targets,
                    attn_scale, contextual_seq_len, rab=None, max_attn_len=0, full_attn_size=0,
                    reference_contextual_rule=False):
    # reference_contextual_rule: the rule of the reference operator (keys whose target-clamped id is
    # 0, kjt_split_per_feature.cpp:672-674) instead of "keys j < contextual_seq_len"
    ok = (torch.float8_e4m3fn, torch.uint8)
    if q_fp8.dtype not in ok or k_fp8.dtype not in ok:
        raise ValueError("q_fp8 and k_fp8 must be float8_e4m3fn (or its uint8 bytes)")
    if v.dtype != torch.bfloat16:
        raise ValueError("v must be bfloat16")
    H = q_fp8.shape[1] if q_fp8.dim() == 3 else -1
    for name, s in (("q_scale", q_scale), ("k_scale", k_scale)):
        if tuple(s.shape) != (H,):
            raise ValueError(f"{name} must have shape [H]")
    qs = q_scale.to(device=v.device, dtype=torch.float32).contiguous()
    ks = k_scale.to(device=v.device, dtype=torch.float32).contiguous()
    out = _launch(q_fp8.view(torch.uint8), k_fp8.view(torch.uint8), v, seq_offsets, num_targets,
                  attn_scale, rab, qs, ks, N, alpha, contextual_seq_len, _lib.DTYPE_FP8_E4M3,
                  max_attn_len, full_attn_size, bool(reference_contextual_rule))
    return out, torch.zeros((1,), dtype=torch.float32, device=v.device)


def _quant_device(x, seq_offsets=None):
    L = _lib.load()
    if x.device.type != "cuda":
        raise RuntimeError("recir::hstu_quantize_e4m3_per_head runs on the GPU only")
    if x.dim() != 3 or x.dtype != torch.bfloat16:
        raise ValueError("x must be a bfloat16 tensor of shape [T, H, D]")
    x = x.contiguous()
    T, H, D = x.shape
    codes = torch.empty((T, H, D), dtype=torch.uint8, device=x.device)
    scale = torch.empty((H,), dtype=torch.float32, device=x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    off, flags, B = None, 0, 0
    if seq_offsets is not None:  # rows at and after seq_offsets[-1] are padding: kept out of the scales
        off, _, flags = _index_tensors(seq_offsets, None, x.device)
        B = off.shape[0] - 1
    with torch.cuda.device(x.device):
        rc = L.recir_hstu_quantize_e4m3_per_head_rows(x.data_ptr(), codes.data_ptr(), scale.data_ptr(),
                                                      T, H, D, _ptr(off), B, flags, stream)
    if rc != 0:
        raise (ValueError if rc < 0 else RuntimeError)(
            f"recir_hstu_quantize_e4m3_per_head failed ({rc}): {_lib.last_error()}")
    return codes.view(torch.float8_e4m3fn), scale


def _no_cpu(*args, **kwargs):
    raise RuntimeError(
        "recir HSTU attention has no CPU implementation: the operator is backed only by the "
        "gfx950 HIP library (librecir_hstu.so); move the tensors to the GPU")


_LIBRARY.impl("hstu_jagged_attention_fwd", _fwd_device, "CUDA")
_LIBRARY.impl("hstu_jagged_attention_fp8_fwd", _fp8_fwd_device, "CUDA")
_LIBRARY.impl("hstu_quantize_e4m3_per_head", _quant_device, "CUDA")
_LIBRARY.impl("hstu_jagged_attention_bwd", _bwd_op_device, "CUDA")
_LIBRARY.impl("hstu_jagged_attention_bwd_rab", _bwd_rab_device, "CUDA")
_LIBRARY.impl("hstu_jagged_attention_bwd_rab", _no_cpu, "CPU")
_LIBRARY.impl("triton_ragged_attention_fwd", _ref_fwd_device, "CUDA")
_LIBRARY.impl("triton_ragged_attention_bwd", _ref_bwd_device, "CUDA")
_LIBRARY.impl("triton_ragged_attention_fwd", _no_cpu, "CPU")
_LIBRARY.impl("triton_ragged_attention_bwd", _no_cpu, "CPU")
_LIBRARY.impl("hstu_jagged_attention_bwd", _no_cpu, "CPU")
_LIBRARY.impl("hstu_jagged_attention_fwd", _no_cpu, "CPU")
_LIBRARY.impl("hstu_jagged_attention_fp8_fwd", _no_cpu, "CPU")
_LIBRARY.impl("hstu_quantize_e4m3_per_head", _no_cpu, "CPU")


@torch.library.register_fake("recir::hstu_jagged_attention_fwd")
def _fwd_fake(N, alpha, q, k, v, seq_offsets, invalid_attn_mask_type, num_targets, attn_scale,
              max_attn_len, contextual_seq_len, full_attn_size, num_softmax_heads=0, rab=None):
    _check_common(q, k, v, seq_offsets, num_targets, N)
    # packed layout is kept: dim 0 of the output is dim 0 of q (recir/compiler/batch_dim.py:309-318)
    return v.new_empty((q.shape[0], q.shape[1], v.shape[2])), q.new_empty((1,), dtype=torch.float32)


@torch.library.register_fake("recir::triton_ragged_attention_fwd")
def _ref_fwd_fake(N, alpha, q, k, v, seq_offsets, invalid_attn_mask_type, num_targets, attn_scale,
                  max_attn_len, contextual_seq_len, full_attn_size, num_softmax_heads=0):
    _check_common(q, k, v, seq_offsets, num_targets, N)
    return v.new_empty((q.shape[0], q.shape[1], v.shape[2])), q.new_empty((1,), dtype=torch.float32)


@torch.library.register_fake("recir::triton_ragged_attention_bwd")
def _ref_bwd_fake(dout, N, alpha, q, k, v, seq_offsets, num_targets, attn_scale, contextual_seq_len,
                  max_attn_len=0, full_attn_size=0, invalid_attn_mask_type="lower_triangular"):
    _check_common(q, k, v, seq_offsets, num_targets, N)
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


@torch.library.register_fake("recir::hstu_jagged_attention_fp8_fwd")
def _fp8_fwd_fake(N, alpha, q_fp8, k_fp8, v, q_scale, k_scale, seq_offsets, num_targets, attn_scale,
                  contextual_seq_len, rab=None, max_attn_len=0, full_attn_size=0,
                  reference_contextual_rule=False):
    _check_common(q_fp8, k_fp8, v, seq_offsets, num_targets, N)
    return v.new_empty((q_fp8.shape[0], q_fp8.shape[1], v.shape[2])), v.new_empty((1,), dtype=torch.float32)


@torch.library.register_fake("recir::hstu_quantize_e4m3_per_head")
def _quant_fake(x, seq_offsets=None):
    return x.new_empty(x.shape, dtype=torch.float8_e4m3fn), x.new_empty((x.shape[1],), dtype=torch.float32)


@torch.library.register_fake("recir::hstu_jagged_attention_bwd")
def _bwd_fake(dout, N, alpha, q, k, v, seq_offsets, num_targets, attn_scale, contextual_seq_len, rab=None,
              max_attn_len=0, full_attn_size=0, invalid_attn_mask_type="lower_triangular"):
    _check_common(q, k, v, seq_offsets, num_targets, N)
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


@torch.library.register_fake("recir::hstu_jagged_attention_bwd_rab")
def _bwd_rab_fake(dout, N, alpha, q, k, v, seq_offsets, num_targets, attn_scale, contextual_seq_len, rab,
                  max_attn_len=0, full_attn_size=0, invalid_attn_mask_type="lower_triangular"):
    _check_common(q, k, v, seq_offsets, num_targets, N)
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), rab.new_empty(rab.shape, dtype=torch.float32)


def _setup_context(ctx, inputs, output):
    (N, alpha, q, k, v, seq_offsets, mask_type, num_targets, attn_scale, max_attn_len,
     contextual_seq_len, full_attn_size, _num_softmax_heads, rab) = inputs
    ctx.save_for_backward(q, k, v, seq_offsets, num_targets, attn_scale, rab)
    ctx.hstu_args = (int(N), float(alpha), int(contextual_seq_len), int(max_attn_len), int(full_attn_size), str(mask_type))


def _autograd_backward(ctx, grad_out, _grad_aux):
    q, k, v, seq_offsets, num_targets, attn_scale, rab = ctx.saved_tensors
    N, alpha, contextual_seq_len, max_attn_len, full_attn_size, mask_type = ctx.hstu_args
    drab = None
    if rab is not None and ctx.needs_input_grad[13]:  # a learned bias table: its gradient as well
        dq, dk, dv, drab = torch.ops.recir.hstu_jagged_attention_bwd_rab(
            grad_out, N, alpha, q, k, v, seq_offsets, num_targets, attn_scale, contextual_seq_len, rab,
            max_attn_len, full_attn_size, mask_type)
        drab = drab.to(rab.dtype)
    else:
        dq, dk, dv = torch.ops.recir.hstu_jagged_attention_bwd(
            grad_out, N, alpha, q, k, v, seq_offsets, num_targets, attn_scale, contextual_seq_len, rab,
            max_attn_len, full_attn_size, mask_type)
    # one gradient slot per forward argument; attn_scale receives none
    return (None, None, dq, dk, dv, None, None, None, None, None, None, None, None, drab)


# gradients of q, k and v flow through the backward operator (the reference attaches its backward
# the same way: recir/ops/pallas/hstu_attention.py:451-459, custom vjp around the kernels)
torch.library.register_autograd("recir::hstu_jagged_attention_fwd", _autograd_backward,
                                setup_context=_setup_context)



def _ref_setup_context(ctx, inputs, output):
    (N, alpha, q, k, v, seq_offsets, mask_type, num_targets, attn_scale, max_attn_len,
     contextual_seq_len, full_attn_size, _num_softmax_heads) = inputs
    ctx.save_for_backward(q, k, v, seq_offsets, num_targets, attn_scale)
    ctx.hstu_args = (int(N), float(alpha), int(contextual_seq_len), int(max_attn_len), int(full_attn_size), str(mask_type))


def _ref_autograd_backward(ctx, grad_out, _grad_aux):
    q, k, v, seq_offsets, num_targets, attn_scale = ctx.saved_tensors
    N, alpha, contextual_seq_len, max_attn_len, full_attn_size, mask_type = ctx.hstu_args
    dq, dk, dv = torch.ops.recir.triton_ragged_attention_bwd(
        grad_out, N, alpha, q, k, v, seq_offsets, num_targets, attn_scale, contextual_seq_len,
        max_attn_len, full_attn_size, mask_type)
    return (None, None, dq, dk, dv, None, None, None, None, None, None, None, None)


torch.library.register_autograd("recir::triton_ragged_attention_fwd", _ref_autograd_backward,
                                setup_context=_ref_setup_context)

hstu_jagged_attention_fwd = torch.ops.recir.hstu_jagged_attention_fwd
hstu_jagged_attention_bwd = torch.ops.recir.hstu_jagged_attention_bwd
triton_ragged_attention_fwd = torch.ops.recir.triton_ragged_attention_fwd


def jagged_hstu_attention(q, k, v, seq_offsets, num_targets=None, *, max_seq_len: int,
                          alpha: Optional[float] = None, attn_scale=None,
                          contextual_seq_len: int = 0, rab=None, max_attn_len: int = 0,
                          full_attn_size: int = 0, invalid_attn_mask_type: str = "lower_triangular") -> torch.Tensor:
    """Packed HSTU attention with the defaults of the accelerator entry point it replaces
    (recir/ops/pallas/jagged_hstu_attention.py:1550-1555, recir/ops/helion/jagged_hstu_attention.py:
    798-804): ``num_targets=None`` means no targets, ``alpha=None`` means ``1/sqrt(Dqk)``,
    ``attn_scale=None`` means ``1/max_seq_len``.  Returns ``out [T, H, Dv]`` with rows at and
    after ``seq_offsets[-1]`` zero.  ``attn_scale`` may be a float, a 0-d tensor or a ``[T]`` tensor.
    ``max_attn_len > 0`` selects the semi-local mask of the reference operator
    (recir/ops/kjt_split_per_feature.cpp:654-668; the reference's accelerator kernels fix it to 256 /
    256, recir/ops/helion/jagged_hstu_attention.py:95-147): history keys within ``max_attn_len``
    positions, and full causal attention for the rows from ``full_attn_size`` before the targets on.
    ``invalid_attn_mask_type`` other than ``"lower_triangular"`` selects, as in the reference operator
    (recir/ops/kjt_split_per_feature.cpp:650-660), the mask on absolute distances: positions at most
    ``max_attn_len`` apart either way round, only the diagonal without a window.
    """
    _check_common(q, k, v, seq_offsets, num_targets, max_seq_len)
    if alpha is None:
        alpha = 1.0 / math.sqrt(q.shape[2])
    if attn_scale is not None and not isinstance(attn_scale, torch.Tensor):
        attn_scale = torch.tensor(float(attn_scale), dtype=torch.float32, device=q.device)
    out, _ = hstu_jagged_attention_fwd(int(max_seq_len), float(alpha), q, k, v, seq_offsets,
                                       str(invalid_attn_mask_type), num_targets, attn_scale, int(max_attn_len),
                                       int(contextual_seq_len), int(full_attn_size), 0, rab)
    return out


def jagged_hstu_attention_backward(dout, q, k, v, seq_offsets, num_targets=None, attn_scale=None, *,
                                   max_seq_len: int, alpha: Optional[float] = None,
                                   contextual_seq_len: int = 0, rab=None, max_attn_len: int = 0,
                                   full_attn_size: int = 0, rab_grad: bool = False,
                                   invalid_attn_mask_type: str = "lower_triangular"):
    """``(dq, dk, dv)`` of ``jagged_hstu_attention`` for the upstream gradient ``dout [T, H, Dv]``;
    argument order and defaults of ``pallas_jagged_hstu_attention_backward``
    (recir/ops/pallas/jagged_hstu_attention.py:1343-1358; called that way by its own test,
    recir/ops/pallas/tests/test_jagged_hstu_attention.py:248-262) and of ``hstu_ragged_attention_bwd_jax_fn``
    (recir/ops/helion/jagged_hstu_attention.py:875-920).  Rows at and after ``seq_offsets[-1]`` of
    the three gradients are zero.  With ``rab_grad`` the gradient of the bias table ``[H, 2N-1]``
    (float32) is returned as a fourth tensor; no gradient is produced for ``attn_scale``."""
    _check_common(q, k, v, seq_offsets, num_targets, max_seq_len)
    if alpha is None:
        alpha = 1.0 / math.sqrt(q.shape[2])
    if attn_scale is not None and not isinstance(attn_scale, torch.Tensor):
        attn_scale = torch.tensor(float(attn_scale), dtype=torch.float32, device=q.device)
    if rab_grad:
        return torch.ops.recir.hstu_jagged_attention_bwd_rab(dout, int(max_seq_len), float(alpha), q, k, v, seq_offsets,
                                                             num_targets, attn_scale, int(contextual_seq_len), rab,
                                                             int(max_attn_len), int(full_attn_size),
                                                             str(invalid_attn_mask_type))
    return hstu_jagged_attention_bwd(dout, int(max_seq_len), float(alpha), q, k, v, seq_offsets,
                                     num_targets, attn_scale, int(contextual_seq_len), rab,
                                     int(max_attn_len), int(full_attn_size), str(invalid_attn_mask_type))


def quantize_e4m3_per_head(x: torch.Tensor, seq_offsets: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """bf16 ``[T,H,D]`` -> (float8_e4m3fn codes, float32 scale ``[H]``), scale = amax_h / 448.

    The arithmetic is the reference's row-wise recipe (recir/ops/kjt_split_per_feature.cpp:493-502)
    at per-head granularity.  With ``seq_offsets`` the rows at and after ``seq_offsets[-1]`` (padding,
    possibly uninitialised) stay out of the maxima and get zero codes."""
    return torch.ops.recir.hstu_quantize_e4m3_per_head(x, seq_offsets)


def jagged_hstu_attention_fp8(q, k, v, seq_offsets, num_targets=None, *, max_seq_len: int,
                              alpha: Optional[float] = None, attn_scale=None,
                              contextual_seq_len: int = 0, rab=None, max_attn_len: int = 0,
                              full_attn_size: int = 0) -> torch.Tensor:
    """Inference variant: bf16 q and k are quantised per head to e4m3 on the device, the scores are
    contracted in fp8 and dequantised with ``q_scale[h] * k_scale[h]``; v, P.V and out stay bf16."""
    _check_common(q, k, v, seq_offsets, num_targets, max_seq_len)
    if alpha is None:
        alpha = 1.0 / math.sqrt(q.shape[2])
    if attn_scale is not None and not isinstance(attn_scale, torch.Tensor):
        attn_scale = torch.tensor(float(attn_scale), dtype=torch.float32, device=q.device)
    q8, qs = quantize_e4m3_per_head(q, seq_offsets)
    k8, ks = quantize_e4m3_per_head(k, seq_offsets)
    out, _ = torch.ops.recir.hstu_jagged_attention_fp8_fwd(
        int(max_seq_len), float(alpha), q8, k8, v, qs, ks, seq_offsets, num_targets, attn_scale,
        int(contextual_seq_len), rab, int(max_attn_len), int(full_attn_size))
    return out


def _reference_rule_targets():
    """Operators whose contextual rule is the reference's (kjt_split_per_feature.cpp:672-674): the
    reference's own ``hammer::`` operator when it is loaded, and this package's drop-in for it."""
    targets = [triton_ragged_attention_fwd, triton_ragged_attention_fwd.default]
    try:
        src = torch.ops.hammer.triton_ragged_attention_fwd
        targets += [src, src.default]
    except (AttributeError, RuntimeError):
        pass
    return targets


def hstu_attention_matcher(node) -> bool:
    """``OpMatcher`` of RecIR's training-to-inference swap
    (recir/region_transforms/inference_swap.py:73-77): true for a graph node that calls the HSTU
    attention operator, under this package's name or the reference's."""
    if node.op != "call_function":
        return False
    targets = [hstu_jagged_attention_fwd, hstu_jagged_attention_fwd.default] + _reference_rule_targets()
    return any(node.target is t for t in targets)


def _via_fp8(reference_rule, N, alpha, q, k, v, seq_offsets, invalid_attn_mask_type, num_targets, attn_scale,
             max_attn_len, contextual_seq_len, full_attn_size, num_softmax_heads, rab):
    if num_softmax_heads != 0:
        raise ValueError("softmax attention heads are unsupported")
    if invalid_attn_mask_type != "lower_triangular":
        raise ValueError("the fp8 kernel covers the causal mask ('lower_triangular') only")
    q8, qs = quantize_e4m3_per_head(q, seq_offsets)
    k8, ks = quantize_e4m3_per_head(k, seq_offsets)
    return torch.ops.recir.hstu_jagged_attention_fp8_fwd(
        int(N), float(alpha), q8, k8, v, qs, ks, seq_offsets, num_targets, attn_scale,
        int(contextual_seq_len), rab, int(max_attn_len), int(full_attn_size), bool(reference_rule))


def attention_via_fp8(N, alpha, q, k, v, seq_offsets, invalid_attn_mask_type, num_targets, attn_scale,
                      max_attn_len, contextual_seq_len, full_attn_size, num_softmax_heads=0, rab=None):
    """The positional signature of ``recir::hstu_jagged_attention_fwd`` and its contextual rule (keys
    ``j < contextual_seq_len``), computed with q and k quantised per head to fp8 e4m3 (v, the
    accumulation and the output stay as they are).  Module level on purpose: it becomes a
    ``call_function`` target of the inference graph, and a saved GraphModule names its targets by
    qualified name (recir/region_transforms/inference_swap.py:89-104)."""
    return _via_fp8(False, N, alpha, q, k, v, seq_offsets, invalid_attn_mask_type, num_targets, attn_scale,
                    max_attn_len, contextual_seq_len, full_attn_size, num_softmax_heads, rab)


def attention_via_fp8_reference_rule(N, alpha, q, k, v, seq_offsets, invalid_attn_mask_type, num_targets,
                                     attn_scale, max_attn_len, contextual_seq_len, full_attn_size,
                                     num_softmax_heads=0):
    """The same for a node that called the reference's operator (``hammer::`` or
    ``recir::triton_ragged_attention_fwd``): its signature (no bias) and its contextual rule, keys
    whose target-clamped id is 0 (recir/ops/kjt_split_per_feature.cpp:672-674), so that the swapped
    node keeps the set of pairs of the node it replaces for every ``contextual_seq_len``."""
    return _via_fp8(True, N, alpha, q, k, v, seq_offsets, invalid_attn_mask_type, num_targets, attn_scale,
                    max_attn_len, contextual_seq_len, full_attn_size, num_softmax_heads, None)


class Fp8AttentionRegion:
    """Callable the factory below returns.  It is spliced into the host graph as a ``call_function``
    target (recir/region_transforms/core.py:358-362), which needs a ``__name__``; it holds a copy of
    the region in which every attention node runs ``attention_via_fp8`` (or its reference-rule twin).  It pickles by value (the
    class and the rewritten region are importable); a host graph that names it as a target can be
    run, not re-loaded from a file in another process."""

    def __init__(self, gm):
        self.gm = gm
        self.__name__ = "fp8_attention_region"
        self.__qualname__ = "fp8_attention_region"

    def __call__(self, *inputs):
        return self.gm(*inputs)


def fp8_attention_region(region_gm):
    """``RegionFactory`` of the same swap: given the sub-GraphModule extracted around the matched
    node(s), returns the callable that replaces it.  It takes the region's external inputs
    positionally and returns the region's outputs, whatever else (getitem, casts) the region holds."""
    import copy

    gm = copy.deepcopy(region_gm)
    hits = 0
    for node in gm.graph.nodes:
        if hstu_attention_matcher(node):
            # the replacement keeps the contextual rule of the operator the node called
            by_reference_rule = any(node.target is t for t in _reference_rule_targets())
            node.target = attention_via_fp8_reference_rule if by_reference_rule else attention_via_fp8
            hits += 1
    if hits == 0:
        raise ValueError("the region holds no HSTU attention node")
    gm.graph.lint()
    gm.recompile()
    return Fp8AttentionRegion(gm)


def register_swaps(registry) -> int:
    """Fill a RecIR ``OpSwapRegistry`` (recir/lowering/op_swap.py:16-75) with every source operator
    present in this process that the HIP operator can replace argument-for-argument.  Returns the
    number of mappings added.

    ``hammer::triton_ragged_attention_fwd`` maps onto ``recir::triton_ragged_attention_fwd``: the same
    schema and the same contextual rule as the operator it replaces (keys whose target-clamped id is
    0, recir/ops/kjt_split_per_feature.cpp:672-674), so a swapped graph returns the numbers of the
    original for every ``contextual_seq_len``.  ``recir::hstu_jagged_attention_fwd`` (prefix rule,
    optional bias) is for direct callers."""
    added = 0
    candidates = (("hammer", "triton_ragged_attention_fwd"),)
    for ns, name in candidates:
        try:
            packet = getattr(getattr(torch.ops, ns), name)
        except (AttributeError, RuntimeError):
            continue
        for target in (packet, getattr(packet, "default", None)):
            if target is not None:
                replacement = triton_ragged_attention_fwd if target is packet else triton_ragged_attention_fwd.default
                registry.register(target, replacement)
                added += 1
    return added
