// Position and timestamp embedding add in front of the attention path: for every packed token
//   out[r] = seq[r] + (pos_emb[pos(r)] + ts_emb[bucket(r)])
// plus the two index lists (position rows, timestamp buckets), each sorted with its permutation,
// which the reference hands to the embedding tables' backward.
// Reference: facebook::recir::addTimestampPositionEmbeddings, recir/ops/kjt_split_per_feature.cpp:307-428.
//   high    = seq_length[b] - num_targets[b] * (interleave_targets ? 2 : 1)
//   pos     = i < max_contextual_seq_len ? i : min(high - min(i, high) + max_contextual_seq_len, P - 1)
//   x       = max(float(ts[b, seq_length[b] - 1] - ts[b, i]), 1e-6) / 60;  x = log(x) or sqrt(x)
//   bucket  = clamp(trunc(x), 0, 2048)
// The sums are rounded the way the reference's tensor expression rounds them: table sum in the table
// type, converted to the sequence type, added in the sequence type (fp32 arithmetic, one rounding
// per step).  HBM-bound: one thread per 16-byte chunk of an output row.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hstu_common.h"

namespace recir_jagged {

using recir_hstu::bf16_bits_to_float;
using recir_hstu::float_to_bf16_bits;

struct TsPosParams {
  const void* seq; void* out; const void* offsets; const void* pos_emb; const void* ts_emb;
  const void* timestamps; const void* seq_lengths; const void* num_targets;
  int* pos_idx; int* ts_idx; int* iota;
  long long L; int B, D, P, TS, Tmax, max_ctx, interleave, use_log;
  int seq_bf16, tab_bf16, ts_is_float, i32;
};

__device__ __forceinline__ long long idx_at(const void* p, int i, int i32) {
  return i32 ? (long long)((const int*)p)[i] : ((const long long*)p)[i];
}

__global__ __launch_bounds__(256) void ts_pos_embeddings_kernel(TsPosParams p) {
  const int per = 8;  // elements per thread
  const long long chunks_per_row = (p.D + per - 1) / per;
  const long long total = p.L * chunks_per_row;
  for (long long idx = (long long)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (long long)gridDim.x * 256) {
    const long long r = idx / chunks_per_row;
    const int c = (int)(idx - r * chunks_per_row);
    // owner sequence: first b with offsets[b + 1] > r
    int lo = 0, hi = p.B;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (idx_at(p.offsets, mid + 1, p.i32) > r) hi = mid; else lo = mid + 1;
    }
    const int b = lo < p.B ? lo : p.B - 1;
    const long long start = idx_at(p.offsets, b, p.i32);
    long long i = r - start;
    if (i < 0) i = 0;
    const long long len = idx_at(p.seq_lengths, b, p.i32);
    long long high = len;
    if (p.num_targets) high -= idx_at(p.num_targets, b, p.i32) * (p.interleave ? 2 : 1);
    if (high < 0) high = 0;
    long long pos = high - (i < high ? i : high) + p.max_ctx;
    if (pos > p.P - 1) pos = p.P - 1;
    if (i < p.max_ctx) pos = i;
    pos = pos < 0 ? 0 : (pos > p.P - 1 ? p.P - 1 : pos);
    long long li = len - 1;
    li = li < 0 ? 0 : (li > p.Tmax - 1 ? p.Tmax - 1 : li);
    const long long ci = i > p.Tmax - 1 ? p.Tmax - 1 : i;
    float delta;
    if (p.ts_is_float) {
      const float* ts = (const float*)p.timestamps + (size_t)b * p.Tmax;
      delta = ts[li] - ts[ci];
    } else {
      const long long* ts = (const long long*)p.timestamps + (size_t)b * p.Tmax;
      delta = (float)(ts[li] - ts[ci]);
    }
    delta = fmaxf(delta, 1e-6f) / 60.0f;
    const float x = p.use_log ? logf(delta) : sqrtf(delta);
    long long bucket = (long long)x;  // truncation, as the tensor cast
    bucket = bucket < 0 ? 0 : (bucket > 2048 ? 2048 : bucket);
    if (bucket > p.TS - 1) bucket = p.TS - 1;
    if (c == 0) {
      p.pos_idx[r] = (int)pos;
      p.ts_idx[r] = (int)bucket;
      p.iota[r] = (int)r;
    }
    const int d0 = c * per;
#pragma unroll
    for (int e = 0; e < per; ++e) {
      const int d = d0 + e;
      if (d >= p.D) break;
      float a, t;
      if (p.tab_bf16) {
        a = bf16_bits_to_float(((const unsigned short*)p.pos_emb)[(size_t)pos * p.D + d]);
        t = bf16_bits_to_float(((const unsigned short*)p.ts_emb)[(size_t)bucket * p.D + d]);
      } else {
        a = ((const float*)p.pos_emb)[(size_t)pos * p.D + d];
        t = ((const float*)p.ts_emb)[(size_t)bucket * p.D + d];
      }
      float add = a + t;
      if (p.tab_bf16) add = bf16_bits_to_float(float_to_bf16_bits(add));
      if (p.seq_bf16) {
        add = bf16_bits_to_float(float_to_bf16_bits(add));
        const float s = bf16_bits_to_float(((const unsigned short*)p.seq)[(size_t)r * p.D + d]);
        ((unsigned short*)p.out)[(size_t)r * p.D + d] = float_to_bf16_bits(s + add);
      } else {
        ((float*)p.out)[(size_t)r * p.D + d] = ((const float*)p.seq)[(size_t)r * p.D + d] + add;
      }
    }
  }
}

}  // namespace recir_jagged
