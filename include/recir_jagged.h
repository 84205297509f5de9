/*
 * C ABI of the jagged neighbours of the MI355X HSTU attention path: packed <-> padded conversion and
 * per-sample concatenation / splitting of two jagged tensors.  Same conventions as recir_hstu.h:
 * device pointers, sizes, a HIP stream; asynchronous; nothing allocated; offsets read on the device
 * (no host synchronisation, hence no data-dependent argument errors: out-of-range rows are clamped);
 * status 0 or a RECIR_HSTU_ERR_* code with text in recir_hstu_last_error().
 *
 * Rows are opaque byte strings of row_bytes bytes (any element type, any trailing shape).
 * flags: RECIR_HSTU_FLAG_OFFSETS_I32 when the offsets are int32 instead of int64.
 */
#ifndef RECIR_JAGGED_H_
#define RECIR_JAGGED_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * out[b, i, :] = values[offsets[b] + i, :] for i < min(offsets[b+1] - offsets[b], max_len), else the
 * padding element.  Replaces: recir::jagged_to_padded_dense, _jagged_to_padded_dense_impl
 * (recir/ops/jagged_ops.py:27-66, schema :121).
 * values [total_rows, row_bytes], out [B, max_len, row_bytes]; pad_bits = bit pattern of the padding
 * value in the element type (elem_bytes = 1, 2, 4 or 8).
 */
int recir_jagged_to_padded_dense(const void* values, void* out, const void* offsets,
                                 int64_t total_rows, int32_t B, int32_t max_len, int64_t row_bytes,
                                 int32_t elem_bytes, uint64_t pad_bits, uint32_t flags,
                                 void* hip_stream);

/*
 * out[j, :] = dense[b, j - offsets[b], :] for the sequence b that owns packed row j, 0 for rows owned
 * by none.  Replaces: recir::dense_to_jagged, _dense_to_jagged_forward_impl
 * (recir/ops/jagged_ops.py:69-111, schema :118).  dense [B, N, row_bytes], out [total_L, row_bytes].
 */
int recir_dense_to_jagged(const void* dense, void* out, const void* offsets, int64_t total_L,
                          int32_t B, int32_t N, int64_t row_bytes, uint32_t flags, void* hip_stream);

/*
 * Per sample b: out = [values_b[:n_prefix_from_right], values_a, values_b[n_prefix_from_right:]];
 * with is_replace: out = [values_a[:len_a - len_b], values_b].  A side is jagged (its offsets given)
 * or dense (offsets NULL, dense_len rows per sample).  Replaces: facebook::recir::concat2DJagged
 * behind generative_recommenders::concat_2D_jagged_fwd_op (recir/ops/kjt_split_per_feature.cpp:
 * 100-195, schema :721-723) and recir::concat_2d_jagged (recir/ops/jagged_ops.py:216-252).
 * out_rows = rows_a + rows_b (rows_a with is_replace).
 */
int recir_concat_2d_jagged(const void* values_a, const void* values_b, void* out,
                           const void* offsets_a, const void* offsets_b, int32_t B,
                           int32_t dense_len_a, int32_t dense_len_b, int64_t rows_a, int64_t rows_b,
                           int64_t row_bytes, int32_t is_replace, int32_t n_prefix_from_right,
                           uint32_t flags, void* hip_stream);

/*
 * Inverse of the concatenation: per sample, out_a = rows [n_prefix_to_right, n_prefix_to_right + len_a),
 * out_b = rows [0, n_prefix_to_right) followed by the rows after out_a's.  Replaces:
 * facebook::recir::split2DJagged behind generative_recommenders::split_2D_jagged_fwd_op
 * (recir/ops/kjt_split_per_feature.cpp:430-489, schema :736-738) and recir::split_2d_jagged
 * (recir/ops/jagged_ops.py:255-277).  values [rows_a + rows_b, row_bytes].
 */
int recir_split_2d_jagged(const void* values, void* out_a, void* out_b, const void* offsets_a,
                          const void* offsets_b, int32_t B, int32_t dense_len_a, int32_t dense_len_b,
                          int64_t rows_a, int64_t rows_b, int64_t row_bytes,
                          int32_t n_prefix_to_right, uint32_t flags, void* hip_stream);

/*
 * out[r] = seq[r] + (pos_emb[pos(r)] + ts_emb[bucket(r)]) for every packed token r, plus the position
 * rows and timestamp buckets used, each sorted ascending (stable) with its permutation.
 * Replaces: facebook::recir::addTimestampPositionEmbeddings
 * (recir/ops/kjt_split_per_feature.cpp:307-428; index rules :371-394).
 * seq, out [L, D] bf16 or fp32 (seq_dtype: RECIR_HSTU_DTYPE_BF16 / _FP32); pos_emb [P, D] and ts_emb
 * [TS >= 2049, D] share table_dtype; timestamps [B, Tmax] int64 (timestamps_float = 0) or float32;
 * seq_lengths [B], num_targets [B] or NULL, seq_offsets [B + 1]: int64, or int32 with
 * RECIR_HSTU_FLAG_OFFSETS_I32; sorted_pos, pos_order, sorted_ts, ts_order [L] int32.
 * time_bucket_log: 0 = sqrt, 1 = log (the float log of the device; a value within one ulp of an
 * integer can land in the neighbouring bucket of the host's).
 * Data-dependent argument errors of the reference (lengths outside the timestamp range, more targets
 * than tokens) are not raised: indices are clamped instead.
 */
int recir_add_timestamp_position_embeddings(
    const void* seq, void* out, const void* seq_offsets, const void* pos_emb, const void* ts_emb,
    const void* timestamps, const void* seq_lengths, const void* num_targets, int32_t* sorted_pos,
    int32_t* pos_order, int32_t* sorted_ts, int32_t* ts_order, int64_t L, int32_t B, int32_t D,
    int32_t P, int32_t TS, int32_t Tmax, int32_t max_contextual_seq_len, int32_t interleave_targets,
    int32_t time_bucket_log, int32_t seq_dtype, int32_t table_dtype, int32_t timestamps_float,
    uint32_t flags, void* workspace, size_t workspace_bytes, void* hip_stream);

/* Scratch size the call above needs for L tokens, a position table of P rows and a timestamp table
 * of TS rows (256-byte aligned scratch). */
size_t recir_add_timestamp_position_embeddings_workspace_bytes(int64_t L, int32_t P, int32_t TS);

#ifdef __cplusplus
}
#endif

#endif /* RECIR_JAGGED_H_ */
