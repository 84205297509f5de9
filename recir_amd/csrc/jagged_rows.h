// Row-gather kernels for the jagged neighbours of the attention path: packed <-> padded
// conversion and per-sample concatenation / splitting of two jagged tensors.  All four are pure
// data movement, bound by HBM.  Rows move in chunks of 16, 4, 2 or 1 bytes (the largest the row
// size and the pointers allow); a row's source is found with a binary search over the offsets (read
// on the device; they stay in L2), once per row, by one lane of the wave that then moves it.
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

// the element's bit pattern repeated over eight bytes
__device__ __forceinline__ unsigned long long pad_pattern(unsigned long long pad_bits, int elem_bytes) {
  if (elem_bytes == 1) return (pad_bits & 0xffull) * 0x0101010101010101ull;
  if (elem_bytes == 2) return (pad_bits & 0xffffull) * 0x0001000100010001ull;
  if (elem_bytes == 4) return (pad_bits & 0xffffffffull) * 0x0000000100000001ull;
  return pad_bits;
}

// chunk number c of a row filled with that pattern (a chunk may be smaller than an element: the
// chunk size divides the row size, not necessarily the element size)
template <typename CH>
__device__ __forceinline__ CH pad_chunk(unsigned long long pattern, long long c) {
  union { CH c; unsigned long long q[(sizeof(CH) + 7) / 8]; } u;
  const int shift = 8 * (int)((c * (long long)sizeof(CH)) & 7);  // 0 for chunks of 8 and 16 bytes
#pragma unroll
  for (int i = 0; i < (int)((sizeof(CH) + 7) / 8); ++i) u.q[i] = pattern >> shift;
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

// Common driver.  Looking a row's source up is a chain of dependent loads (offsets, binary search);
// done per chunk it leaves every wave waiting with one kilobyte in flight.  Here a wave takes a
// block of rows, its lanes resolve one row each (in parallel, once), and then the wave moves the
// rows: a group of G = 2^lg lanes per row (G >= chunks per row, at most 64), 64 / G rows per
// iteration, COPY_UNROLL iterations in flight; the source of a row travels from the lane that
// resolved it by a lane shuffle.
//   resolve(r)  source address of output row r, or nullptr for a filled row   (the expensive part)
//   dst_of(r)   where output row r goes                                        (arithmetic only)
//   fill(c)     chunk c of a filled row
#ifndef JAG_UNROLL
#define JAG_UNROLL 4
#endif
#ifndef JAG_ITERS
#define JAG_ITERS 8
#endif
constexpr int COPY_UNROLL = JAG_UNROLL;

__device__ __forceinline__ int rows_per_wave(int lg) {
  const int rpi = 64 >> lg;  // rows per iteration
  return rpi * JAG_ITERS < 64 ? rpi * JAG_ITERS : 64;
}

template <typename CH, typename Resolve, typename Dst, typename Fill>
__device__ __forceinline__ void gather_rows(long long rows, long long cpr, int lg, Resolve resolve, Dst dst_of, Fill fill) {
  const int lane = threadIdx.x & 63;
  const int G = 1 << lg, rpi = 64 >> lg;
  const int sub = lane >> lg, c0 = lane & (G - 1);
  const int RW = rows_per_wave(lg);
  const int iters = RW / rpi;
  const long long wave_id = (long long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const long long nwaves = (long long)gridDim.x * (blockDim.x >> 6);
  for (long long base = wave_id * RW; base < rows; base += nwaves * RW) {
    const long long r_mine = base + lane;
    const char* src_mine = (lane < RW && r_mine < rows) ? resolve(r_mine) : nullptr;
    const int src_lo = (int)(unsigned)(size_t)src_mine, src_hi = (int)(unsigned)((size_t)src_mine >> 32);
    for (int it = 0; it < iters; it += COPY_UNROLL) {
      const char* s[COPY_UNROLL];
      char* d[COPY_UNROLL];
#pragma unroll
      for (int k = 0; k < COPY_UNROLL; ++k) {
        const int j = (it + k) * rpi + sub;  // row of this lane's group inside the block
        const long long r = base + j;
        const unsigned lo = (unsigned)__shfl(src_lo, j & 63), hi = (unsigned)__shfl(src_hi, j & 63);
        s[k] = (const char*)(((size_t)hi << 32) | lo);
        d[k] = (it + k < iters && r < rows) ? dst_of(r) : nullptr;
      }
      for (long long c = c0; c < cpr; c += G) {
        CH v[COPY_UNROLL];
#pragma unroll
        for (int k = 0; k < COPY_UNROLL; ++k)
          if (d[k]) v[k] = s[k] ? ((const CH*)s[k])[c] : fill(c);
#pragma unroll
        for (int k = 0; k < COPY_UNROLL; ++k)
          if (d[k]) ((CH*)d[k])[c] = v[k];
      }
    }
  }
}

// out[b, i, :] = values[offsets[b] + i, :] for i < len_b, else the padding value
template <typename CH>
__global__ __launch_bounds__(256) void jagged_to_padded_dense_kernel(PadParams p, long long cpr, int lg) {
  const long long row_bytes = cpr * (long long)sizeof(CH);
  const unsigned long long pattern = pad_pattern(p.pad_bits, p.elem_bytes);
  gather_rows<CH>((long long)p.B * p.max_len, cpr, lg,
      [&](long long row) -> const char* {
        const int b = (int)(row / p.max_len);
        const int i = (int)(row - (long long)b * p.max_len);
        const long long s = p.off.at(b), e = p.off.at(b + 1);
        if (i < e - s && p.total_rows > 0) return p.values + clampll(s + i, 0, p.total_rows - 1) * row_bytes;
        return nullptr;
      },
      [&](long long row) { return p.out + row * row_bytes; },
      [&](long long c) { return pad_chunk<CH>(pattern, c); });
}

// out[j, :] = dense[seg(j), j - offsets[seg(j)], :] for rows inside a sequence, else 0
template <typename CH>
__global__ __launch_bounds__(256) void dense_to_jagged_kernel(UnpadParams p, long long cpr, int lg) {
  const long long row_bytes = cpr * (long long)sizeof(CH);
  gather_rows<CH>(p.total_L, cpr, lg,
      [&](long long j) -> const char* {
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
        if (valid) return p.dense + clampll((long long)seg * p.N + intra, 0, (long long)p.B * p.N - 1) * row_bytes;
        return nullptr;
      },
      [&](long long j) { return p.out + j * row_bytes; },
      [](long long) { return zero_chunk<CH>(); });
}

// per sample: [b[:n_prefix], a, b[n_prefix:]]; replace mode: [a[:len_a - len_b], b]
template <typename CH>
__global__ __launch_bounds__(256) void concat_2d_jagged_kernel(ConcatParams p, long long cpr, int lg) {
  const long long row_bytes = cpr * (long long)sizeof(CH);
  gather_rows<CH>(p.out_rows, cpr, lg,
      [&](long long r) -> const char* {
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
        if (from_a) return p.rows_a > 0 ? p.a + clampll(src, 0, p.rows_a - 1) * row_bytes : nullptr;
        return p.rows_b > 0 ? p.b + clampll(src, 0, p.rows_b - 1) * row_bytes : nullptr;
      },
      [&](long long r) { return p.out + r * row_bytes; },
      [](long long) { return zero_chunk<CH>(); });
}

// inverse of the concatenation: a = rows [n_prefix, n_prefix + len_a) of a sample,
// b = rows [0, n_prefix) followed by rows [n_prefix + len_a, len_a + len_b)
template <typename CH>
__global__ __launch_bounds__(256) void split_2d_jagged_kernel(SplitParams p, long long cpr, int lg) {
  const long long row_bytes = cpr * (long long)sizeof(CH);
  gather_rows<CH>(p.rows_a + p.rows_b, cpr, lg,
      [&](long long r0) -> const char* {
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
        return p.in_rows > 0 ? p.values + clampll(src, 0, p.in_rows - 1) * row_bytes : nullptr;
      },
      [&](long long r0) { return r0 < p.rows_a ? p.out_a + r0 * row_bytes : p.out_b + (r0 - p.rows_a) * row_bytes; },
      [](long long) { return zero_chunk<CH>(); });
}

}  // namespace recir_jagged
