// Row-gather kernels for the jagged neighbours of the attention path: packed <-> padded
// conversion and per-sample concatenation / splitting of two jagged tensors.  All four are pure
// data movement, bound by HBM: one thread moves one chunk (16, 4, 2 or 1 bytes, the largest the
// row size and the pointers allow) of one output row, and finds the row's source with a binary
// search over the offsets (read on the device; they stay in L2).
//
// Reference semantics:
//   jagged_to_padded_dense   recir/ops/jagged_ops.py:27-66
//   dense_to_jagged          recir/ops/jagged_ops.py:69-111
//   concat_2d_jagged         recir/ops/kjt_split_per_feature.cpp:100-195 (right prefix, replace
//                            mode, dense sides), recir/ops/jagged_ops.py:216-252
//   split_2d_jagged          recir/ops/kjt_split_per_feature.cpp:430-489, recir/ops/jagged_ops.py:255-277
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace recir_jagged {

struct Offsets {
  const void* ptr;  // [B + 1] or nullptr for a dense side
  int dense_len;    // rows per sample of a dense side
  int i32;          // offsets are int32 (else int64)
  __device__ __forceinline__ long long at(int b) const {
    if (!ptr) return (long long)b * dense_len;
    return i32 ? (long long)((const int*)ptr)[b] : ((const long long*)ptr)[b];
  }
};

// number of i in [1, B] with sum_offsets(i) <= r, clamped to [0, B - 1]: the sample that owns row r
template <typename F>
__device__ __forceinline__ int owner(int B, long long r, F sum_offsets) {
  int lo = 1, hi = B + 1;  // first i in [1, B] with sum_offsets(i) > r
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (sum_offsets(mid) > r) hi = mid; else lo = mid + 1;
  }
  const int b = lo - 1;
  return b < 0 ? 0 : (b > B - 1 ? B - 1 : b);
}

struct PadParams {
  const char* values; char* out; Offsets off;
  long long total_rows; int B, max_len; unsigned long long pad_bits; int elem_bytes;
};
struct UnpadParams {
  const char* dense; char* out; Offsets off; long long total_L; int B, N;
};
struct ConcatParams {
  const char* a; const char* b; char* out; Offsets oa, ob;
  long long rows_a, rows_b, out_rows; int B, is_replace, n_prefix;
};
struct SplitParams {
  const char* values; char* out_a; char* out_b; Offsets oa, ob;
  long long rows_a, rows_b, in_rows; int B, n_prefix;
};

// chunk number c of a row filled with the element's bit pattern (a chunk may be smaller than an
// element: the chunk size divides the row size, not necessarily the element size)
template <typename CH>
__device__ __forceinline__ CH pad_chunk(unsigned long long pad_bits, int elem_bytes, long long c) {
  union { CH c; unsigned char bytes[sizeof(CH)]; } u;
  const int first = (int)((c * (long long)sizeof(CH)) % elem_bytes);
#pragma unroll
  for (int i = 0; i < (int)sizeof(CH); ++i) u.bytes[i] = (unsigned char)(pad_bits >> (8 * ((first + i) % elem_bytes)));
  return u.c;
}

template <typename CH>
__device__ __forceinline__ CH zero_chunk() {
  union { CH c; unsigned char bytes[sizeof(CH)]; } u;
#pragma unroll
  for (int i = 0; i < (int)sizeof(CH); ++i) u.bytes[i] = 0;
  return u.c;
}

__device__ __forceinline__ long long clampll(long long x, long long lo, long long hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}

// out[b, i, :] = values[offsets[b] + i, :] for i < len_b, else the padding value
template <typename CH>
__global__ __launch_bounds__(256) void jagged_to_padded_dense_kernel(PadParams p, long long chunks_per_row) {
  const long long total = (long long)p.B * p.max_len * chunks_per_row;
  for (long long idx = (long long)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (long long)gridDim.x * 256) {
    const long long row = idx / chunks_per_row;
    const long long c = idx - row * chunks_per_row;
    const int b = (int)(row / p.max_len);
    const int i = (int)(row - (long long)b * p.max_len);
    const long long s = p.off.at(b), e = p.off.at(b + 1);
    CH v;
    if (i < e - s && p.total_rows > 0) {
      const long long src = clampll(s + i, 0, p.total_rows - 1);
      v = ((const CH*)p.values)[src * chunks_per_row + c];
    } else {
      v = pad_chunk<CH>(p.pad_bits, p.elem_bytes, c);
    }
    ((CH*)p.out)[idx] = v;
  }
}

// out[j, :] = dense[seg(j), j - offsets[seg(j)], :] for rows inside a sequence, else 0
template <typename CH>
__global__ __launch_bounds__(256) void dense_to_jagged_kernel(UnpadParams p, long long chunks_per_row) {
  const long long total = p.total_L * chunks_per_row;
  for (long long idx = (long long)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (long long)gridDim.x * 256) {
    const long long j = idx / chunks_per_row;
    const long long c = idx - j * chunks_per_row;
    // segment = number of interior boundaries offsets[1 .. B-1] at or below j
    int lo = 1, hi = p.B;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (p.off.at(mid) > j) hi = mid; else lo = mid + 1;
    }
    int seg = lo - 1;
    seg = seg < 0 ? 0 : (seg > p.B - 1 ? p.B - 1 : seg);
    const long long s = p.off.at(seg), e = p.off.at(seg + 1);
    const long long intra = j - s;
    const bool valid = j < p.off.at(p.B) && intra >= 0 && intra < e - s;
    CH v = zero_chunk<CH>();
    if (valid) {
      const long long src = clampll((long long)seg * p.N + intra, 0, (long long)p.B * p.N - 1);
      v = ((const CH*)p.dense)[src * chunks_per_row + c];
    }
    ((CH*)p.out)[idx] = v;
  }
}

// per sample: [b[:n_prefix], a, b[n_prefix:]]; replace mode: [a[:len_a - len_b], b]
template <typename CH>
__global__ __launch_bounds__(256) void concat_2d_jagged_kernel(ConcatParams p, long long chunks_per_row) {
  const long long total = p.out_rows * chunks_per_row;
  for (long long idx = (long long)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (long long)gridDim.x * 256) {
    const long long r = idx / chunks_per_row;
    const long long c = idx - r * chunks_per_row;
    const int b = p.is_replace ? owner(p.B, r, [&](int i) { return p.oa.at(i); })
                               : owner(p.B, r, [&](int i) { return p.oa.at(i) + p.ob.at(i); });
    const long long sa = p.oa.at(b), sb = p.ob.at(b);
    const long long la = p.oa.at(b + 1) - sa, lb = p.ob.at(b + 1) - sb;
    const long long intra = r - (p.is_replace ? sa : sa + sb);
    bool from_a;
    long long src;
    if (p.is_replace) {
      const long long keep = la - lb > 0 ? la - lb : 0;
      from_a = intra < keep;
      src = from_a ? sa + intra : sb + (intra - keep);
    } else {
      const long long np = p.n_prefix < lb ? p.n_prefix : lb;
      if (intra < np) { from_a = false; src = sb + intra; }
      else if (intra < np + la) { from_a = true; src = sa + (intra - np); }
      else { from_a = false; src = sb + (intra - la); }
    }
    CH v = zero_chunk<CH>();
    if (from_a) {
      if (p.rows_a > 0) v = ((const CH*)p.a)[clampll(src, 0, p.rows_a - 1) * chunks_per_row + c];
    } else {
      if (p.rows_b > 0) v = ((const CH*)p.b)[clampll(src, 0, p.rows_b - 1) * chunks_per_row + c];
    }
    ((CH*)p.out)[idx] = v;
  }
}

// inverse of the concatenation: a = rows [n_prefix, n_prefix + len_a) of a sample,
// b = rows [0, n_prefix) followed by rows [n_prefix + len_a, len_a + len_b)
template <typename CH>
__global__ __launch_bounds__(256) void split_2d_jagged_kernel(SplitParams p, long long chunks_per_row) {
  const long long total = (p.rows_a + p.rows_b) * chunks_per_row;
  for (long long idx = (long long)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (long long)gridDim.x * 256) {
    const long long r0 = idx / chunks_per_row;
    const long long c = idx - r0 * chunks_per_row;
    const bool to_a = r0 < p.rows_a;
    const long long r = to_a ? r0 : r0 - p.rows_a;
    const int b = to_a ? owner(p.B, r, [&](int i) { return p.oa.at(i); })
                       : owner(p.B, r, [&](int i) { return p.ob.at(i); });
    const long long sa = p.oa.at(b), sb = p.ob.at(b);
    const long long la = p.oa.at(b + 1) - sa, lb = p.ob.at(b + 1) - sb;
    const long long np = p.n_prefix < lb ? p.n_prefix : lb;
    long long src = sa + sb;
    if (to_a) {
      src += np + (r - sa);
    } else {
      const long long ib = r - sb;
      src += ib < np ? ib : ib + la;
    }
    CH v = zero_chunk<CH>();
    if (p.in_rows > 0) v = ((const CH*)p.values)[clampll(src, 0, p.in_rows - 1) * chunks_per_row + c];
    if (to_a) ((CH*)p.out_a)[r * chunks_per_row + c] = v;
    else ((CH*)p.out_b)[r * chunks_per_row + c] = v;
  }
}

}  // namespace recir_jagged
