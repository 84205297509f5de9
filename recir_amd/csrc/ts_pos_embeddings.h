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
// per step).  HBM-bound.
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

// position row and timestamp bucket of packed token r (integer rules of the reference; float32
// sqrt or log of the time delta)
__device__ __forceinline__ void ts_pos_of_token(const TsPosParams& p, long long r, int& pos_out, int& bucket_out) {
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
  pos_out = (int)pos;
  bucket_out = (int)bucket;
}

// E consecutive elements of a bf16 or fp32 row as floats, and back (E * element size <= 16 bytes is
// one access)
template <int E, bool BF16>
__device__ __forceinline__ void load_elems(const void* row, int d0, float (&x)[E]) {
  if (BF16) {
    union { unsigned short h[E]; unsigned w[(E + 1) / 2]; } u;
    if (E == 8) *(uint4*)u.w = *(const uint4*)((const unsigned short*)row + d0);
    else if (E == 4) *(uint2*)u.w = *(const uint2*)((const unsigned short*)row + d0);
    else u.h[0] = ((const unsigned short*)row)[d0];
#pragma unroll
    for (int e = 0; e < E; ++e) x[e] = bf16_bits_to_float(u.h[e]);
  } else {
    if (E == 8) {
      const float4 a = *(const float4*)((const float*)row + d0), b = *(const float4*)((const float*)row + d0 + 4);
      x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4 % E] = b.x; x[5 % E] = b.y; x[6 % E] = b.z; x[7 % E] = b.w;
    } else if (E == 4) {
      const float4 a = *(const float4*)((const float*)row + d0);
      x[0] = a.x; x[1 % E] = a.y; x[2 % E] = a.z; x[3 % E] = a.w;
    } else {
      x[0] = ((const float*)row)[d0];
    }
  }
}

template <int E, bool BF16>
__device__ __forceinline__ void store_elems(void* row, int d0, const float (&x)[E]) {
  if (BF16) {
    union { unsigned short h[E]; unsigned w[(E + 1) / 2]; } u;
#pragma unroll
    for (int e = 0; e < E; ++e) u.h[e] = float_to_bf16_bits(x[e]);
    if (E == 8) *(uint4*)((unsigned short*)row + d0) = *(const uint4*)u.w;
    else if (E == 4) *(uint2*)((unsigned short*)row + d0) = *(const uint2*)u.w;
    else ((unsigned short*)row)[d0] = u.h[0];
  } else {
    if (E == 8) {
      *(float4*)((float*)row + d0) = make_float4(x[0], x[1 % E], x[2 % E], x[3 % E]);
      *(float4*)((float*)row + d0 + 4) = make_float4(x[4 % E], x[5 % E], x[6 % E], x[7 % E]);
    } else if (E == 4) {
      *(float4*)((float*)row + d0) = make_float4(x[0], x[1 % E], x[2 % E], x[3 % E]);
    } else {
      ((float*)row)[d0] = x[0];
    }
  }
}

// A wave takes a block of tokens: its lanes find position row and bucket of one token each (the
// dependent loads -- owner search, lengths, two timestamps -- happen once per token, in parallel) and
// write the index lists; then groups of 2^lg lanes add the rows, E elements per lane and access,
// the two table rows of a token travelling from the lane that found them by a lane shuffle.
// E = 8 or 4 needs D % E == 0 and 16-byte aligned tensors; E = 1 is the path for everything else.
template <int E, bool SEQ_BF16, bool TAB_BF16>
__global__ __launch_bounds__(256) void ts_pos_embeddings_kernel(TsPosParams p, int lg) {
  const int lane = threadIdx.x & 63;
  const int G = 1 << lg, rpi = 64 >> lg;
  const int sub = lane >> lg, c0 = lane & (G - 1);
  const int cpr = p.D / E;
  const int RW = rpi * 8 < 64 ? rpi * 8 : 64;  // tokens per wave
  const int iters = RW / rpi;
  const long long wave_id = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const long long nwaves = (long long)gridDim.x * 4;
  const size_t seq_row = (size_t)p.D * (SEQ_BF16 ? 2 : 4), tab_row = (size_t)p.D * (TAB_BF16 ? 2 : 4);
  for (long long base = wave_id * RW; base < p.L; base += nwaves * RW) {
    const long long r_mine = base + lane;
    int pos_mine = 0, bucket_mine = 0;
    if (lane < RW && r_mine < p.L) {
      ts_pos_of_token(p, r_mine, pos_mine, bucket_mine);
      p.pos_idx[r_mine] = pos_mine;
      p.ts_idx[r_mine] = bucket_mine;
      p.iota[r_mine] = (int)r_mine;
    }
    for (int it = 0; it < iters; ++it) {
      const int j = it * rpi + sub;
      const long long r = base + j;
      const int pos = __shfl(pos_mine, j & 63), bucket = __shfl(bucket_mine, j & 63);
      if (r >= p.L) continue;
      const char* srow = (const char*)p.seq + (size_t)r * seq_row;
      char* orow = (char*)p.out + (size_t)r * seq_row;
      const char* prow = (const char*)p.pos_emb + (size_t)pos * tab_row;
      const char* trow = (const char*)p.ts_emb + (size_t)bucket * tab_row;
      for (int c = c0; c < cpr; c += G) {
        float a[E], t[E], sv[E], o[E];
        load_elems<E, TAB_BF16>(prow, c * E, a);
        load_elems<E, TAB_BF16>(trow, c * E, t);
        load_elems<E, SEQ_BF16>(srow, c * E, sv);
#pragma unroll
        for (int e = 0; e < E; ++e) {
          float add = a[e] + t[e];
          if (TAB_BF16) add = bf16_bits_to_float(float_to_bf16_bits(add));  // sum in the table type
          if (SEQ_BF16) add = bf16_bits_to_float(float_to_bf16_bits(add));  // converted to the sequence type
          o[e] = sv[e] + add;
        }
        store_elems<E, SEQ_BF16>(orow, c * E, o);
      }
    }
  }
}

}  // namespace recir_jagged
