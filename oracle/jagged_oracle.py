"""CPU restatement of the jagged neighbours of the attention path.  TEST INFRASTRUCTURE ONLY: the
product (recir_amd) never imports this module.

Plain numpy / Python loops over samples, each function following the reference lines it cites:

  jagged_to_padded_dense   recir/ops/jagged_ops.py:27-66  (gather with clamped flat index, padding
                           value where i >= length, truncation at max_len)
  dense_to_jagged          recir/ops/jagged_ops.py:69-111 (segment = interior boundaries at or below
                           the row, row valid inside its segment, clamped flat source index)
  concat_2d_jagged         recir/ops/kjt_split_per_feature.cpp:100-195 (per sample
                           [b[:n_prefix], a, b[n_prefix:]]; replace mode [a[:len_a-len_b], b]; a
                           dense side is [B, S, D])
  split_2d_jagged          recir/ops/kjt_split_per_feature.cpp:430-489
  add_ts_pos_emb           recir/ops/kjt_split_per_feature.cpp:307-428 (position rule :371-382,
                           time buckets :384-392, sums in the tensors' own types :396-401, the two
                           sorted index lists :413-427); float32 arithmetic via numpy, bf16 via
                           explicit round-to-nearest-even

add_ts_pos_emb is pinned by the reference's known-answer test (KjtSplitPerFeatureTest.cpp:141-175)
and by the compiled reference operator on random inputs (values bit-exact for sqrt buckets; log
buckets compared away from integer boundaries, where one ulp of the logarithm decides).

Pins (tests/test_jagged_oracle.py): the reference's own known-answer tests
(recir/ops/tests/KjtSplitPerFeatureTest.cpp:50-91, :177-189), the reference's compiled C++ operators
on random inputs (oracle/_ref), concat/split and pad/unpad round trips, and per-sample slicing
written independently in the tests for the two Python-only reference functions.
"""
import numpy as np


def _lengths(offsets):
    offsets = np.asarray(offsets, dtype=np.int64)
    return offsets, offsets[1:] - offsets[:-1]


def jagged_to_padded_dense(values, offsets, max_len, padding_value=0.0):
    values = np.asarray(values)
    offsets, lengths = _lengths(offsets)
    B = len(lengths)
    out = np.full((B, max_len) + values.shape[1:], padding_value, dtype=values.dtype)
    L = values.shape[0]
    for b in range(B):
        for i in range(min(int(lengths[b]), max_len)):
            if L > 0:
                out[b, i] = values[min(max(int(offsets[b]) + i, 0), L - 1)]
    return out


def dense_to_jagged(dense, offsets, total_L=None):
    dense = np.asarray(dense)
    offsets, lengths = _lengths(offsets)
    B, N = dense.shape[0], dense.shape[1]
    if total_L is None:
        total_L = int(offsets[-1])
    out = np.zeros((total_L,) + dense.shape[2:], dtype=dense.dtype)
    flat = dense.reshape((B * N,) + dense.shape[2:])
    for j in range(total_L):
        seg = min(int(np.sum(offsets[1:B] <= j)), B - 1) if B > 0 else 0
        if B == 0 or N == 0:
            continue
        intra = j - int(offsets[seg])
        if j < offsets[B] and 0 <= intra < lengths[seg]:
            out[j] = flat[min(max(seg * N + intra, 0), B * N - 1)]
    return out


def _sample(values, offsets, b):
    """Rows of sample b: a slice of a jagged [L, ...] tensor or row b of a dense [B, S, ...] one."""
    if offsets is None:
        return values[b]
    return values[int(offsets[b]):int(offsets[b + 1])]


def concat_2d_jagged(values_a, values_b, offsets_a=None, offsets_b=None, is_replace=False, n_prefix_from_right=0):
    values_a, values_b = np.asarray(values_a), np.asarray(values_b)
    assert offsets_a is not None or offsets_b is not None
    B = values_a.shape[0] if offsets_a is None else len(offsets_a) - 1
    parts = []
    for b in range(B):
        a, bb = _sample(values_a, offsets_a, b), _sample(values_b, offsets_b, b)
        if is_replace:
            assert len(bb) <= len(a)
            parts += [a[: len(a) - len(bb)], bb]
        else:
            assert n_prefix_from_right <= len(bb)
            parts += [bb[:n_prefix_from_right], a, bb[n_prefix_from_right:]]
    tail = values_a.shape[2:] if offsets_a is None else values_a.shape[1:]
    out = np.concatenate(parts, axis=0) if parts else np.zeros((0,) + tail, dtype=values_a.dtype)
    if is_replace and values_a.ndim == 3 and offsets_a is None:
        out = out.reshape(values_a.shape)
    return out


def split_2d_jagged(values, offsets_a, offsets_b, dense_size_a=0, dense_size_b=0, n_prefix_to_right=0, B=None):
    values = np.asarray(values)
    if B is None:
        B = len(offsets_a if not dense_size_a else offsets_b) - 1
    pa, pb, pos = [], [], 0
    for b in range(B):
        la = dense_size_a if dense_size_a else int(offsets_a[b + 1] - offsets_a[b])
        lb = dense_size_b if dense_size_b else int(offsets_b[b + 1] - offsets_b[b])
        assert n_prefix_to_right <= lb
        rows = values[pos:pos + la + lb]
        pa.append(rows[n_prefix_to_right:n_prefix_to_right + la])
        pb += [rows[:n_prefix_to_right], rows[n_prefix_to_right + la:]]
        pos += la + lb
    assert pos == values.shape[0]
    empty = np.zeros((0,) + values.shape[1:], dtype=values.dtype)
    a = np.concatenate(pa, axis=0) if pa else empty
    bb = np.concatenate(pb, axis=0) if pb else empty
    if dense_size_a:
        a = a.reshape((B, dense_size_a) + values.shape[1:])
    if dense_size_b:
        bb = bb.reshape((B, dense_size_b) + values.shape[1:])
    return a, bb


def _round_bf16(x):
    """float32 array rounded to the nearest bfloat16 (ties to even), returned as float32."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def add_ts_pos_emb(seq, offsets, pos_emb, ts_emb, timestamps, seq_lengths, num_targets=None,
                   max_contextual_seq_len=0, interleave_targets=False, time_bucket_fn="sqrt",
                   seq_bf16=False, tab_bf16=False):
    """Returns (out [L, D] float32 holding values of the sequence type, position rows [L], buckets [L],
    and the pre-bucket float values [L] so that a test can tell how close a bucket boundary is)."""
    seq = np.asarray(seq, dtype=np.float32)
    pos_emb, ts_emb = np.asarray(pos_emb, dtype=np.float32), np.asarray(ts_emb, dtype=np.float32)
    offsets = np.asarray(offsets, dtype=np.int64)
    timestamps = np.asarray(timestamps)
    B = len(seq_lengths)
    out = np.array(seq, copy=True)
    pos_idx = np.zeros(seq.shape[0], dtype=np.int64)
    ts_idx = np.zeros(seq.shape[0], dtype=np.int64)
    pre = np.zeros(seq.shape[0], dtype=np.float32)
    P = pos_emb.shape[0]
    for b in range(B):
        s, e = int(offsets[b]), int(offsets[b + 1])
        n = e - s
        length = int(seq_lengths[b])
        high = length
        if num_targets is not None:
            high -= int(num_targets[b]) * (2 if interleave_targets else 1)
        i = np.arange(n, dtype=np.int64)
        pi = high - np.minimum(i, high) + max_contextual_seq_len
        pi = np.minimum(pi, P - 1)
        pi = np.where(i < max_contextual_seq_len, i, pi)
        row = timestamps[b]
        delta = (row[length - 1] - row[:n]).astype(np.float32)
        delta = np.maximum(delta, np.float32(1e-6)) / np.float32(60.0)
        x = np.log(delta) if time_bucket_fn == "log" else np.sqrt(delta)
        x = x.astype(np.float32)
        ti = np.clip(np.trunc(x).astype(np.int64), 0, 2048)
        add = pos_emb[pi] + ts_emb[ti]
        if tab_bf16:
            add = _round_bf16(add)
        if seq_bf16:
            add = _round_bf16(add)
            out[s:e] = _round_bf16(seq[s:e] + add)
        else:
            out[s:e] = seq[s:e] + add
        pos_idx[s:e], ts_idx[s:e], pre[s:e] = pi, ti, x
    return out, pos_idx, ts_idx, pre
