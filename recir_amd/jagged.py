"""Host side of the jagged neighbours of the attention path: packed <-> padded conversion and
per-sample concatenation / splitting, as ``torch.library`` operators backed by the HIP row-gather
kernels (C ABI in ``include/recir_jagged.h``).

Operator names and argument lists follow the reference:
``recir::jagged_to_padded_dense``, ``recir::dense_to_jagged``, ``recir::concat_2d_jagged``,
``recir::split_2d_jagged`` (recir/ops/jagged_ops.py:114-131) and, with the argument lists of the
third-party operators RecIR meets in traced graphs, ``recir::concat_2D_jagged_fwd`` /
``recir::split_2D_jagged_fwd`` (generative_recommenders::concat_2D_jagged_fwd_op and
split_2D_jagged_fwd_op, recir/ops/kjt_split_per_feature.cpp:721-723, :736-738).  When the reference's
own module has already defined an operator in this process, only the device kernel is attached to it.

There is no CPU implementation here: CPU tensors raise.
"""
from __future__ import annotations

import struct
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib

_DEF = torch.library.Library("recir", "FRAGMENT")

_SCHEMAS = {
    "jagged_to_padded_dense": "jagged_to_padded_dense(Tensor values, Tensor[] offsets, int[] max_lengths, float padding_value=0) -> Tensor",
    "dense_to_jagged": "dense_to_jagged(Tensor dense, Tensor[] offsets, int? total_L=None) -> (Tensor, Tensor)",
    "concat_2d_jagged": "concat_2d_jagged(Tensor values_left, Tensor offsets_left, Tensor values_right, Tensor offsets_right) -> Tensor",
    "split_2d_jagged": "split_2d_jagged(Tensor values, Tensor offsets_left, Tensor offsets_right, SymInt seq_len_a, SymInt seq_len_b) -> (Tensor, Tensor)",
    "concat_2D_jagged_fwd": "concat_2D_jagged_fwd(int max_seq_len, Tensor values_a, Tensor values_b, Tensor? offsets_a, Tensor? offsets_b, bool is_replace, int n_prefix_from_right) -> Tensor",
    "split_2D_jagged_fwd": "split_2D_jagged_fwd(Tensor values, int max_seq_len, Tensor offsets_a, Tensor offsets_b, int seq_len_a, int seq_len_b, bool is_dense_a, bool is_dense_b, int dense_size, int n_prefix_to_right, int B) -> (Tensor, Tensor)",
    # hammer::add_ts_pos_emb_fwd_op, recir/ops/kjt_split_per_feature.cpp:776-779
    "add_ts_pos_emb_fwd": "add_ts_pos_emb_fwd(Tensor seq_embeddings, Tensor seq_offsets, Tensor pos_embeddings, Tensor ts_embeddings, Tensor timestamps, Tensor seq_lengths, Tensor? num_targets, int max_seq_len, int max_contextual_seq_len, bool interleave_targets, str time_bucket_fn) -> (Tensor, Tensor, Tensor, Tensor, Tensor)",
}
_defined_here = set()


def _already_defined(name: str) -> bool:
    try:
        torch._C._dispatch_find_schema_or_throw(f"recir::{name}", "")
        return True
    except RuntimeError:
        return False


for _name, _schema in _SCHEMAS.items():
    if not _already_defined(_name):
        _DEF.define(_schema)
        _defined_here.add(_name)


def _need_cuda(op: str, t: torch.Tensor):
    if t.device.type != "cuda":
        raise RuntimeError(f"recir::{op} runs on the GPU only (got a tensor on '{t.device}'); "
                           "this package has no CPU path")


def _no_cpu(*args, **kwargs):
    raise RuntimeError("the recir jagged operators of this package have no CPU implementation: they are "
                       "backed only by the gfx950 HIP library (librecir_hstu.so); move the tensors to the GPU")


def _offsets(off: torch.Tensor, like: Optional[torch.Tensor] = None, dev=None):
    """Offsets as the kernels read them: int32 or int64, contiguous, on the device of the values
    (index tensors may arrive on any device, as with the reference operators, and are moved: a host
    pointer must never reach a kernel)."""
    if off.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"offsets must be int32 or int64, got {off.dtype}")
    if like is not None and off.dtype != like.dtype:
        off = off.to(like.dtype)
    if dev is not None:
        off = off.to(dev)
    return off.contiguous(), (_lib.FLAG_OFFSETS_I32 if off.dtype == torch.int32 else 0)


def _same_device(dev, **tensors):
    """Value tensors must share one device (recir/ops/kjt_split_per_feature.cpp:112-114 checks the
    same); raised before anything is launched."""
    for name, t in tensors.items():
        if t is not None and t.device != dev:
            raise ValueError(f"{name} is on {t.device}, the values on {dev}")


def _row_bytes(t: torch.Tensor, lead_dims: int) -> int:
    n = t.element_size()
    for d in t.shape[lead_dims:]:
        n *= int(d)
    return n


def _status(entry: str, rc: int):
    if rc != 0:
        msg = _lib.last_error()
        if rc < 0:
            raise ValueError(f"{entry} rejected the call ({rc}): {msg}")
        raise RuntimeError(f"{entry} launch failed (hipError {rc}): {msg}")


def _pad_bits(value: float, dtype: torch.dtype) -> Tuple[int, int]:
    """(element size, bit pattern) of a padding value in ``dtype``."""
    t = torch.tensor([value], dtype=dtype)
    size = t.element_size()
    if size not in (1, 2, 4, 8):
        raise ValueError(f"jagged_to_padded_dense supports 1-, 2-, 4- and 8-byte element types, got {dtype}")
    raw = t.view(torch.uint8).numpy().tobytes()
    return size, int.from_bytes(raw, "little")


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


# ---------------------------------------------------------------------------------------------
# device implementations
# ---------------------------------------------------------------------------------------------
def _jagged_to_padded_dense_device(values, offsets: List[torch.Tensor], max_lengths: Sequence[int],
                                   padding_value: float = 0.0):
    _need_cuda("jagged_to_padded_dense", values)
    L = _lib.load()
    if len(offsets) != 1 or len(max_lengths) != 1:
        raise ValueError("one jagged dimension is supported (one offsets tensor, one max length)")
    off, flags = _offsets(offsets[0], dev=values.device)
    B, max_len = off.shape[0] - 1, int(max_lengths[0])
    values = values.contiguous()
    out = values.new_empty((B, max_len) + tuple(values.shape[1:]))
    row_bytes = _row_bytes(values, 1)
    if out.numel() == 0:
        return out
    if row_bytes == 0:
        return out
    size, bits = _pad_bits(padding_value, values.dtype)
    with torch.cuda.device(values.device):
        rc = L.recir_jagged_to_padded_dense(values.data_ptr(), out.data_ptr(), off.data_ptr(), values.shape[0], B,
                                            max_len, row_bytes, size, bits, flags, _stream(values.device))
    _status("recir_jagged_to_padded_dense", rc)
    return out


def _dense_to_jagged_device(dense, offsets: List[torch.Tensor], total_L: Optional[int] = None):
    _need_cuda("dense_to_jagged", dense)
    L = _lib.load()
    off, flags = _offsets(offsets[0], dev=dense.device)
    if total_L is None:
        total_L = int(off[-1].item())  # the reference reads it from the device as well
    dense = dense.contiguous()
    B, N = dense.shape[0], dense.shape[1]
    out = dense.new_empty((int(total_L),) + tuple(dense.shape[2:]))
    row_bytes = _row_bytes(dense, 2)
    if out.numel() > 0:
        with torch.cuda.device(dense.device):
            rc = L.recir_dense_to_jagged(dense.data_ptr(), out.data_ptr(), off.data_ptr(), int(total_L), B, N,
                                         row_bytes, flags, _stream(dense.device))
        _status("recir_dense_to_jagged", rc)
    return out, offsets[0]


def _concat_impl(values_a, values_b, offsets_a, offsets_b, is_replace: bool, n_prefix: int):
    _need_cuda("concat_2d_jagged", values_a)
    L = _lib.load()
    _same_device(values_a.device, values_b=values_b)
    if offsets_a is None and offsets_b is None:
        raise ValueError("at least one input must be jagged")
    if values_a.dtype != values_b.dtype:
        raise ValueError("values_a and values_b must have the same dtype")
    if values_a.shape[-1:] != values_b.shape[-1:] and values_a.dim() > 1:
        raise ValueError("values_a and values_b must have the same embedding dimension")
    values_a, values_b = values_a.contiguous(), values_b.contiguous()
    flags = 0
    oa = ob = None
    dense_a = dense_b = 0
    if offsets_a is not None:
        oa, flags = _offsets(offsets_a, dev=values_a.device)
    if offsets_b is not None:
        ob, flags = _offsets(offsets_b, oa, dev=values_a.device)
        if oa is not None and oa.dtype != ob.dtype:
            oa = oa.to(ob.dtype)
    if oa is None:
        if values_a.dim() != 3:
            raise ValueError("dense values_a must be three-dimensional")
        B, dense_a = values_a.shape[0], values_a.shape[1]
        if ob.shape[0] != B + 1:
            raise ValueError("offsets_b size must match the dense batch size")
        flat_a = values_a.reshape(B * dense_a, -1)
    else:
        B = oa.shape[0] - 1
        flat_a = values_a
    if ob is None:
        if values_b.dim() != 3:
            raise ValueError("dense values_b must be three-dimensional")
        dense_b = values_b.shape[1]
        if values_b.shape[0] != B:
            raise ValueError("offsets_a size must match the dense batch size")
        flat_b = values_b.reshape(B * dense_b, -1)
    else:
        if ob.shape[0] != B + 1:
            raise ValueError("offsets_a and offsets_b must have the same size")
        flat_b = values_b
    rows_a, rows_b = flat_a.shape[0], flat_b.shape[0]
    out_rows = rows_a if is_replace else rows_a + rows_b
    out = flat_a.new_empty((out_rows,) + tuple(flat_a.shape[1:]))
    row_bytes = _row_bytes(flat_a, 1)
    if out.numel() > 0:
        with torch.cuda.device(values_a.device):
            rc = L.recir_concat_2d_jagged(flat_a.data_ptr(), flat_b.data_ptr(), out.data_ptr(),
                                          None if oa is None else oa.data_ptr(), None if ob is None else ob.data_ptr(),
                                          B, dense_a, dense_b, rows_a, rows_b, row_bytes, int(bool(is_replace)),
                                          int(n_prefix), flags, _stream(values_a.device))
        _status("recir_concat_2d_jagged", rc)
    elif n_prefix < 0:
        raise ValueError("n_prefix_from_right must be non-negative")
    if is_replace and values_a.dim() == 3:
        return out.view_as(values_a)
    return out


def _split_impl(values, offsets_a, offsets_b, rows_a: int, rows_b: int, dense_a: int, dense_b: int, n_prefix: int,
                B: Optional[int] = None):
    _need_cuda("split_2d_jagged", values)
    L = _lib.load()
    values = values.contiguous()
    if values.shape[0] != rows_a + rows_b:
        raise ValueError("split lengths do not match values")
    oa = ob = None
    flags = 0
    if not dense_a:
        oa, flags = _offsets(offsets_a, dev=values.device)
    if not dense_b:
        ob, flags = _offsets(offsets_b, oa, dev=values.device)
        if oa is not None and oa.dtype != ob.dtype:
            oa = oa.to(ob.dtype)
    if B is None:
        B = (oa if oa is not None else ob).shape[0] - 1
    out_a = values.new_empty((rows_a,) + tuple(values.shape[1:]))
    out_b = values.new_empty((rows_b,) + tuple(values.shape[1:]))
    row_bytes = _row_bytes(values, 1)
    if values.numel() > 0:
        with torch.cuda.device(values.device):
            rc = L.recir_split_2d_jagged(values.data_ptr(), out_a.data_ptr(), out_b.data_ptr(),
                                         None if oa is None else oa.data_ptr(), None if ob is None else ob.data_ptr(),
                                         int(B), int(dense_a), int(dense_b), rows_a, rows_b, row_bytes, int(n_prefix),
                                         flags, _stream(values.device))
        _status("recir_split_2d_jagged", rc)
    return out_a, out_b


def _concat_2d_jagged_device(values_left, offsets_left, values_right, offsets_right):
    return _concat_impl(values_left, values_right, offsets_left, offsets_right, False, 0)


def _split_2d_jagged_device(values, offsets_left, offsets_right, seq_len_a, seq_len_b):
    return _split_impl(values, offsets_left, offsets_right, int(seq_len_a), int(seq_len_b), 0, 0, 0)


def _concat_2D_jagged_fwd_device(max_seq_len, values_a, values_b, offsets_a, offsets_b, is_replace,
                                 n_prefix_from_right):
    if n_prefix_from_right < 0:
        raise ValueError(f"n_prefix_from_right must be non-negative, got {n_prefix_from_right}")
    if is_replace and n_prefix_from_right != 0:
        raise ValueError("n_prefix_from_right is not supported when is_replace is true")
    if n_prefix_from_right != 0 and (offsets_a is None or offsets_b is None):
        raise ValueError("n_prefix_from_right is only supported for two jagged inputs")
    return _concat_impl(values_a, values_b, offsets_a, offsets_b, bool(is_replace), int(n_prefix_from_right))


def _split_2D_jagged_fwd_device(values, max_seq_len, offsets_a, offsets_b, seq_len_a, seq_len_b, is_dense_a,
                                is_dense_b, dense_size, n_prefix_to_right, B):
    rows_a = B * dense_size if is_dense_a else int(seq_len_a)
    rows_b = B * dense_size if is_dense_b else int(seq_len_b)
    a, b = _split_impl(values, offsets_a, offsets_b, rows_a, rows_b, dense_size if is_dense_a else 0,
                       dense_size if is_dense_b else 0, int(n_prefix_to_right), int(B))
    if is_dense_a:
        a = a.view((B, dense_size) + tuple(values.shape[1:]))
    if is_dense_b:
        b = b.view((B, dense_size) + tuple(values.shape[1:]))
    return a, b


def _add_ts_pos_emb_fwd_device(seq_embeddings, seq_offsets, pos_embeddings, ts_embeddings, timestamps, seq_lengths,
                               num_targets, max_seq_len, max_contextual_seq_len, interleave_targets, time_bucket_fn):
    """Argument checks and messages of the reference (recir/ops/kjt_split_per_feature.cpp:320-347)."""
    _need_cuda("add_ts_pos_emb_fwd", seq_embeddings)
    L = _lib.load()
    if seq_embeddings.dim() != 2:
        raise ValueError("sequence embeddings must be two-dimensional")
    if pos_embeddings.dim() != 2 or ts_embeddings.dim() != 2:
        raise ValueError("position and timestamp embeddings must be two-dimensional")
    if timestamps.dim() != 2:
        raise ValueError("timestamps must be two-dimensional")
    if seq_lengths.dim() != 1:
        raise ValueError("sequence lengths must be one-dimensional")
    D = seq_embeddings.shape[1]
    if pos_embeddings.shape[1] != D or ts_embeddings.shape[1] != D:
        raise ValueError("all embeddings must have the same dimension")
    if ts_embeddings.shape[0] < 2049:
        raise ValueError("timestamp embeddings must contain 2049 buckets")
    B = seq_lengths.numel()
    if seq_offsets.numel() != B + 1:
        raise ValueError("sequence offsets size must match the batch size")
    if timestamps.shape[0] != B:
        raise ValueError("timestamps size must match the batch size")
    if num_targets is not None and num_targets.numel() != B:
        raise ValueError("num_targets size must match the batch size")
    if time_bucket_fn not in ("log", "sqrt"):
        raise ValueError("time_bucket_fn must be 'log' or 'sqrt'")
    codes = {torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_FP32}
    if seq_embeddings.dtype not in codes or pos_embeddings.dtype not in codes or ts_embeddings.dtype != pos_embeddings.dtype:
        raise ValueError("embeddings must be bfloat16 or float32, and both tables of one dtype")
    if timestamps.dtype == torch.float32:
        ts_float = 1
    elif timestamps.dtype == torch.int64:
        ts_float = 0
    else:
        raise ValueError(f"timestamps must be int64 or float32, got {timestamps.dtype}")
    dev = seq_embeddings.device
    _same_device(dev, pos_embeddings=pos_embeddings, ts_embeddings=ts_embeddings, timestamps=timestamps)
    off, flags = _offsets(seq_offsets, dev=dev)
    lens = seq_lengths.to(device=dev, dtype=off.dtype).contiguous()
    nt = None if num_targets is None else num_targets.to(device=dev, dtype=off.dtype).contiguous()
    seq = seq_embeddings.contiguous()
    pos, ts_tab, stamps = pos_embeddings.contiguous(), ts_embeddings.contiguous(), timestamps.contiguous()
    rows = seq.shape[0]
    dev = seq.device
    out = torch.empty_like(seq)
    idx = [torch.empty((rows,), dtype=torch.int32, device=dev) for _ in range(4)]
    if rows > 0:
        ws_bytes = L.recir_add_timestamp_position_embeddings_workspace_bytes(rows, pos.shape[0], ts_tab.shape[0])
        ws = torch.empty((ws_bytes + 256,), dtype=torch.uint8, device=dev)
        base = (ws.data_ptr() + 255) // 256 * 256
        with torch.cuda.device(dev):
            rc = L.recir_add_timestamp_position_embeddings(
                seq.data_ptr(), out.data_ptr(), off.data_ptr(), pos.data_ptr(), ts_tab.data_ptr(), stamps.data_ptr(),
                lens.data_ptr(), None if nt is None else nt.data_ptr(), idx[0].data_ptr(), idx[1].data_ptr(),
                idx[2].data_ptr(), idx[3].data_ptr(), rows, B, D, pos.shape[0], ts_tab.shape[0], stamps.shape[1],
                int(max_contextual_seq_len), int(bool(interleave_targets)), int(time_bucket_fn == "log"),
                codes[seq.dtype], codes[pos.dtype], ts_float, flags, base, ws_bytes, _stream(dev))
        _status("recir_add_timestamp_position_embeddings", rc)
    return out, idx[0], idx[1], idx[2], idx[3]


_IMPLS = {
    "add_ts_pos_emb_fwd": _add_ts_pos_emb_fwd_device,
    "jagged_to_padded_dense": _jagged_to_padded_dense_device,
    "dense_to_jagged": _dense_to_jagged_device,
    "concat_2d_jagged": _concat_2d_jagged_device,
    "split_2d_jagged": _split_2d_jagged_device,
    "concat_2D_jagged_fwd": _concat_2D_jagged_fwd_device,
    "split_2D_jagged_fwd": _split_2D_jagged_fwd_device,
}
_IMPL = torch.library.Library("recir", "IMPL")
for _name, _fn in _IMPLS.items():
    _IMPL.impl(_name, _fn, "CUDA")
    if _name in _defined_here:
        _IMPL.impl(_name, _no_cpu, "CPU")


# ---------------------------------------------------------------------------------------------
# fake kernels and autograd for the operators defined here (the reference brings its own otherwise)
# ---------------------------------------------------------------------------------------------
if "jagged_to_padded_dense" in _defined_here:
    @torch.library.register_fake("recir::jagged_to_padded_dense")
    def _j2pd_fake(values, offsets, max_lengths, padding_value=0.0):
        return values.new_empty((offsets[0].shape[0] - 1, max_lengths[0]) + tuple(values.shape[1:]))

    def _j2pd_setup(ctx, inputs, output):
        values, offsets, _max_lengths, _pad = inputs
        ctx.save_for_backward(offsets[0])
        ctx.total_rows = values.shape[0]

    def _j2pd_backward(ctx, grad):
        (off,) = ctx.saved_tensors
        g, _ = torch.ops.recir.dense_to_jagged(grad.contiguous(), [off], ctx.total_rows)
        # arguments left at their defaults are not passed by the dispatcher and get no slot
        return (g, [None], None, None)[: len(ctx.needs_input_grad)]

    torch.library.register_autograd("recir::jagged_to_padded_dense", _j2pd_backward, setup_context=_j2pd_setup)

if "dense_to_jagged" in _defined_here:
    @torch.library.register_fake("recir::dense_to_jagged")
    def _d2j_fake(dense, offsets, total_L=None):
        if total_L is None:
            total_L = torch.library.get_ctx().new_dynamic_size()
        return dense.new_empty((total_L,) + tuple(dense.shape[2:])), torch.empty_like(offsets[0])

    def _d2j_setup(ctx, inputs, output):
        dense, offsets, _total = inputs
        ctx.save_for_backward(offsets[0])
        ctx.max_len = dense.shape[1]

    def _d2j_backward(ctx, grad, _grad_off):
        (off,) = ctx.saved_tensors
        g = torch.ops.recir.jagged_to_padded_dense(grad.contiguous(), [off], [ctx.max_len], 0.0)
        return (g, [None], None)[: len(ctx.needs_input_grad)]

    torch.library.register_autograd("recir::dense_to_jagged", _d2j_backward, setup_context=_d2j_setup)

if "concat_2d_jagged" in _defined_here:
    @torch.library.register_fake("recir::concat_2d_jagged")
    def _concat_fake(values_left, offsets_left, values_right, offsets_right):
        return values_left.new_empty((values_left.shape[0] + values_right.shape[0],) + tuple(values_left.shape[1:]))

    def _concat_setup(ctx, inputs, output):
        values_left, offsets_left, values_right, offsets_right = inputs
        ctx.save_for_backward(offsets_left, offsets_right)
        ctx.rows = (values_left.shape[0], values_right.shape[0])

    def _concat_backward(ctx, grad):
        off_l, off_r = ctx.saved_tensors
        gl, gr = torch.ops.recir.split_2d_jagged(grad.contiguous(), off_l, off_r, ctx.rows[0], ctx.rows[1])
        return gl, None, gr, None

    torch.library.register_autograd("recir::concat_2d_jagged", _concat_backward, setup_context=_concat_setup)

if "split_2d_jagged" in _defined_here:
    @torch.library.register_fake("recir::split_2d_jagged")
    def _split_fake(values, offsets_left, offsets_right, seq_len_a, seq_len_b):
        return (values.new_empty((seq_len_a,) + tuple(values.shape[1:])),
                values.new_empty((seq_len_b,) + tuple(values.shape[1:])))

    def _split_setup(ctx, inputs, output):
        _values, offsets_left, offsets_right, _a, _b = inputs
        ctx.save_for_backward(offsets_left, offsets_right)

    def _split_backward(ctx, grad_a, grad_b):
        off_l, off_r = ctx.saved_tensors
        return (torch.ops.recir.concat_2d_jagged(grad_a.contiguous(), off_l, grad_b.contiguous(), off_r),
                None, None, None, None)

    torch.library.register_autograd("recir::split_2d_jagged", _split_backward, setup_context=_split_setup)

if "concat_2D_jagged_fwd" in _defined_here:
    @torch.library.register_fake("recir::concat_2D_jagged_fwd")
    def _concat2D_fake(max_seq_len, values_a, values_b, offsets_a, offsets_b, is_replace, n_prefix_from_right):
        rows_a = values_a.shape[0] * (values_a.shape[1] if offsets_a is None else 1)
        rows_b = values_b.shape[0] * (values_b.shape[1] if offsets_b is None else 1)
        if is_replace:
            return torch.empty_like(values_a) if values_a.dim() == 3 else values_a.new_empty(values_a.shape)
        return values_a.new_empty((rows_a + rows_b, values_a.shape[-1]))

if "split_2D_jagged_fwd" in _defined_here:
    @torch.library.register_fake("recir::split_2D_jagged_fwd")
    def _split2D_fake(values, max_seq_len, offsets_a, offsets_b, seq_len_a, seq_len_b, is_dense_a, is_dense_b,
                      dense_size, n_prefix_to_right, B):
        tail = tuple(values.shape[1:])
        a = values.new_empty(((B, dense_size) if is_dense_a else (seq_len_a,)) + tail)
        b = values.new_empty(((B, dense_size) if is_dense_b else (seq_len_b,)) + tail)
        return a, b


if "add_ts_pos_emb_fwd" in _defined_here:
    @torch.library.register_fake("recir::add_ts_pos_emb_fwd")
    def _add_ts_pos_fake(seq_embeddings, seq_offsets, pos_embeddings, ts_embeddings, timestamps, seq_lengths, num_targets,
                         max_seq_len, max_contextual_seq_len, interleave_targets, time_bucket_fn):
        n = seq_embeddings.shape[0]
        i32 = [seq_embeddings.new_empty((n,), dtype=torch.int32) for _ in range(4)]
        return (torch.empty_like(seq_embeddings), *i32)


add_ts_pos_emb_fwd = torch.ops.recir.add_ts_pos_emb_fwd
jagged_to_padded_dense = torch.ops.recir.jagged_to_padded_dense
dense_to_jagged = torch.ops.recir.dense_to_jagged
concat_2d_jagged = torch.ops.recir.concat_2d_jagged
split_2d_jagged = torch.ops.recir.split_2d_jagged
concat_2D_jagged_fwd = torch.ops.recir.concat_2D_jagged_fwd
split_2D_jagged_fwd = torch.ops.recir.split_2D_jagged_fwd


def register_jagged_swaps(registry) -> int:
    """Map the third-party concat/split operators present in this process onto the HIP-backed ones
    (same positional arguments; recir/lowering/op_swap.py:78-97 rewrites only the node target)."""
    added = 0
    pairs = (("generative_recommenders", "concat_2D_jagged_fwd_op", concat_2D_jagged_fwd),
             ("generative_recommenders", "split_2D_jagged_fwd_op", split_2D_jagged_fwd),
             ("hammer", "add_ts_pos_emb_fwd_op", add_ts_pos_emb_fwd))
    for ns, name, repl in pairs:
        try:
            packet = getattr(getattr(torch.ops, ns), name)
        except (AttributeError, RuntimeError):
            continue
        registry.register(packet, repl)
        default = getattr(packet, "default", None)
        if default is not None:
            registry.register(default, repl.default)
            added += 1
        added += 1
    return added
