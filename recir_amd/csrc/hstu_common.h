// Shared device-side definitions of the HSTU attention kernels: launch parameters, sequence
// bookkeeping (offset clamping, history cap, contextual prefix), the keep predicate and bf16 helpers.
#pragma once
#include <hip/hip_runtime.h>

#include "recir_hstu.h"

namespace recir_hstu {


typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2;

// MI355X: 8 accelerator dies (XCDs), each with its own L2; workgroup i of a launch runs on XCD i % 8.
constexpr int NUM_XCD = 8;

// Tile shape of the kernels written for head dim 128: a workgroup owns BM query rows and walks the
// keys in tiles of BN.
constexpr int BM = 128;
constexpr int BN = 64;
constexpr int HD = 128;
constexpr float kLog2e = 1.4426950408889634f;

// One unit of work of the tiled kernels: a query tile of one (sequence, head), with everything the
// workgroup needs about its sequence so that it starts with a single uniform load.
struct WorkItem {
  int s;        // first packed token of the sequence
  int n;        // sequence length
  int cap;      // history length (n - num_targets), clamped to [-1, n]
  int ctx_eff;  // keys j < ctx_eff are visible to every query
  int q0;       // first query row of the tile
  int h;        // head
  int b;        // sequence index
  int q_end;    // one past the last query row of the tile (<= n)
};

struct Params {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  const void* seq_offsets;
  const void* num_targets;
  const float* rab;
  const float* attn_scale;
  const float* q_scale;
  const float* k_scale;
  int* ws_counts;             // [NUM_XCD] length of each per-XCD work list, then [NUM_XCD] the next list position to draw
                              // (kernels whose workgroups stay and draw their items)
  struct WorkItem* ws_items;  // [NUM_XCD][items_cap]
  int items_cap;              // capacity of one per-XCD list
  int grid_slots;             // slots per XCD the launch covers (gridDim.x = NUM_XCD * grid_slots)
  int T, B, H, Dqk, Dv, N, ctx;
  int max_attn_len;    // > 0: semi-local window over the history keys
  int full_attn_size;  // > 0 (with max_attn_len > 0): rows in or after the last full_attn_size history
                       //      positions keep full causal attention
  float alpha;
  unsigned flags;
  unsigned long long* trace;  // phase-trace builds (HSTU_TRACE) only: one TRACE_WORDS record per (work item, wave); else null
};

// Phase-trace builds: the forward kernel stamps the 100 MHz counter at the phases of every work item.
// Record of (XCD x, list slot s, wave w) at trace[((x * items_cap + s) * 4 + w) * TRACE_WORDS]:
//   0 item start   1 first tile resident (query rows loaded, first barrier passed)   2 key-tile loop left
//   3 output rows stored   4..7 ticks spent in skewed trips / unclassified leading tiles / other unmasked
//   tiles / partial tiles (each with its barrier)   8 ticks in tiles this wave skipped (copies and barrier only)
//   9 tile counts, one byte each: skewed, leading, unmasked, partial, skipped   10 hardware id (XCC id << 32 | HW_ID)
//   11 shader-clock cycles of the key-tile loop
constexpr int TRACE_WORDS = 12;
#ifdef HSTU_TRACE
#define HSTU_TR(...) __VA_ARGS__
#else
#define HSTU_TR(...)
#endif

struct SeqInfo {
  int s;        // first packed token
  int n;        // length
  int cap;      // history length n - num_targets (keys j < cap are history)
  int ctx_eff;  // keys j < ctx_eff are visible to every query
  int win;      // a history key j is visible to row m when min(m, cap) - j <= win ...
  int tail0;    // ... or when min(m, cap) >= tail0 (causal mask: win is huge)
};

constexpr int WIN_ALL = 0x3fffffff;

// window and full-attention boundary of a sequence with history length cap
// (recir/ops/kjt_split_per_feature.cpp:654-668: distance window on the target-clamped ids, rows at
// or beyond cap - full_attn_size see the whole history; full_attn_size is ignored without a window)
__device__ __forceinline__ void mask_window(const struct Params& p, int cap, int& win, int& tail0);

__device__ __forceinline__ long long load_index(const void* p, int i, bool i32) {
  return i32 ? (long long)((const int*)p)[i] : ((const long long*)p)[i];
}

__device__ __forceinline__ int clamp_offset(long long x, int lo, int hi) {
  return x < lo ? lo : (x > hi ? hi : (int)x);
}

// Sequence b as the kernels see it.  Offsets are clamped into [0, T] and made non-decreasing so
// that a malformed array cannot cause an out-of-range access.
__device__ __forceinline__ SeqInfo seq_info(const Params& p, int b) {
  const bool i32 = p.flags & RECIR_HSTU_FLAG_OFFSETS_I32;
  SeqInfo si;
  si.s = clamp_offset(load_index(p.seq_offsets, b, i32), 0, p.T);
  const int e = clamp_offset(load_index(p.seq_offsets, b + 1, i32), si.s, p.T);
  si.n = e - si.s;
  long long t = p.num_targets ? load_index(p.num_targets, b, i32) : 0;
  long long cap = (long long)si.n - t;
  si.cap = cap > si.n ? si.n : (cap < -1 ? -1 : (int)cap);
  if (p.flags & RECIR_HSTU_FLAG_CTX_REFERENCE) {
    // the reference unmasks keys whose target-clamped id min(j, cap) equals 0: key 0 when cap > 0
    // (causal anyway, but outside the window of far rows under the semi-local mask), every key
    // when cap == 0, none when cap < 0
    si.ctx_eff = p.ctx > 0 ? (cap == 0 ? si.n : (cap > 0 && si.n > 0 ? 1 : 0)) : 0;
  } else {
    si.ctx_eff = p.ctx < si.n ? (p.ctx > 0 ? p.ctx : 0) : si.n;
  }
  mask_window(p, si.cap, si.win, si.tail0);
  return si;
}

__device__ __forceinline__ void mask_window(const Params& p, int cap, int& win, int& tail0) {
  win = p.max_attn_len > 0 ? p.max_attn_len : WIN_ALL;
  tail0 = (p.max_attn_len > 0 && p.full_attn_size > 0) ? cap - p.full_attn_size : 0x7fffffff;
}

__device__ __forceinline__ int end_of_sequences(const Params& p) {
  const bool i32 = p.flags & RECIR_HSTU_FLAG_OFFSETS_I32;
  return clamp_offset(load_index(p.seq_offsets, p.B, i32), 0, p.T);
}

__device__ __forceinline__ bool keep_pair(int m, int j, const SeqInfo& si) {
  const int idm = min(m, si.cap);
  return (m == j) || (j < idm && (idm - j <= si.win || idm >= si.tail0)) || (j < si.ctx_eff);
}

// The mask of a mask type other than "lower_triangular" (recir/ops/kjt_split_per_feature.cpp:650-671):
// the distance of the clamped ids counts either way round and only under a window (without one the
// diagonal is all there is); the rows of the full-attention tail see the keys whose id is below
// theirs, ids below the tail's start counting as 0.
__device__ __forceinline__ bool keep_pair_noncausal(int m, int j, const SeqInfo& si) {
  const int idm = min(m, si.cap), idj = min(j, si.cap);
  bool kp = (m == j) || (j < si.ctx_eff);
  if (si.win != WIN_ALL) {
    kp = kp || abs(idm - idj) <= si.win;
    if (si.tail0 != 0x7fffffff) {
      const int gr = idm < si.tail0 ? 0 : idm, gc = idj < si.tail0 ? 0 : idj;
      kp = kp || gr - gc > 0;
    }
  }
  return kp;
}

__device__ __forceinline__ bool keep_pair(int m, int j, const SeqInfo& si, bool noncausal) {
  return noncausal ? keep_pair_noncausal(m, j, si) : keep_pair(m, j, si);
}

__device__ __forceinline__ float bf16_bits_to_float(unsigned short b) {
  return __uint_as_float((unsigned)b << 16);
}

__device__ __forceinline__ unsigned short float_to_bf16_bits(float x) {
  f32x2 t = {x, 0.f};
  bf16x2 y = __builtin_convertvector(t, bf16x2);
  return (unsigned short)(*(unsigned*)&y & 0xffffu);
}

__device__ __forceinline__ unsigned pack_bf16x2(float lo, float hi) {
  f32x2 t = {lo, hi};
  bf16x2 y = __builtin_convertvector(t, bf16x2);
  return *(unsigned*)&y;
}

// Rows [seq_offsets[B], T) of a [T, ...] tensor := 0, shared by all workgroups of a launch.
template <int NTHREADS>
__device__ __forceinline__ void zero_tail_rows_of(const Params& p, void* tensor, size_t row_bytes) {
  const int end_all = end_of_sequences(p);
  if (end_all >= p.T) return;
  // row_bytes is a multiple of 2; use 2-byte stores only when 16-byte ones do not fit
  unsigned char* base = (unsigned char*)tensor + (size_t)end_all * row_bytes;
  const size_t total = (size_t)(p.T - end_all) * row_bytes;
  const size_t nblk = gridDim.x * (size_t)gridDim.y;
  const size_t blk = blockIdx.x + (size_t)blockIdx.y * gridDim.x;
  if ((((size_t)base) & 15) == 0 && (total & 15) == 0) {
    for (size_t i = blk * NTHREADS + threadIdx.x; i < total / 16; i += nblk * NTHREADS)
      ((uint4*)base)[i] = make_uint4(0, 0, 0, 0);
  } else {
    for (size_t i = blk * NTHREADS + threadIdx.x; i < total / 2; i += nblk * NTHREADS)
      ((unsigned short*)base)[i] = 0;
  }
}

template <int NTHREADS>
__device__ __forceinline__ void zero_tail_rows(const Params& p, size_t row_bytes) {
  zero_tail_rows_of<NTHREADS>(p, p.out, row_bytes);
}

// Element types of the generic kernels (the C ABI's dtype codes)
constexpr int ELT_BF16 = RECIR_HSTU_DTYPE_BF16, ELT_FP32 = RECIR_HSTU_DTYPE_FP32, ELT_FP16 = RECIR_HSTU_DTYPE_FP16;

template <int ELT>
__device__ __forceinline__ float load_elem(const void* base, size_t idx) {
  if (ELT == ELT_BF16) return bf16_bits_to_float(((const unsigned short*)base)[idx]);
  if (ELT == ELT_FP16) return (float)((const _Float16*)base)[idx];
  return ((const float*)base)[idx];
}

template <int ELT>
__device__ __forceinline__ void store_elem(void* base, size_t idx, float x) {
  if (ELT == ELT_BF16) ((unsigned short*)base)[idx] = float_to_bf16_bits(x);
  else if (ELT == ELT_FP16) ((_Float16*)base)[idx] = (_Float16)x;
  else ((float*)base)[idx] = x;
}

// x as the element type holds it (P and dS are rounded like that before they meet v, dout, q or k)
template <int ELT>
__device__ __forceinline__ float round_to_elem(float x) {
  if (ELT == ELT_BF16) return bf16_bits_to_float(float_to_bf16_bits(x));
  if (ELT == ELT_FP16) return (float)(_Float16)x;
  return x;
}

// Arguments of the backward kernels: the forward's inputs (f.out unused) plus the upstream
// gradient and the three gradients to write.
struct BwdParams {
  Params f;
  const void* dout;  // [T,H,Dv]
  void* dq;          // [T,H,Dqk]
  void* dk;          // [T,H,Dqk]
  void* dv;          // [T,H,Dv]
  float* drab;       // [H, 2N-1] gradient of the bias table, zeroed by the entry point, or null
  unsigned* absmax;  // with drab (tiled kernels): word 1 receives the largest |v| of the call's rows as a
                     // bf16 magnitude << 16, i.e. the bits of a float (key-tile kernel), word 2 holds the
                     // largest |per-token scale| (bits of a float); both are read by the query-tile
                     // kernel; else null
  const unsigned* dout_max;  // with drab (MFMA kernels): [H] largest |dout| of each head, bits of a float
  long long* drab_fx;        // with drab (MFMA kernels): [H, 2N-1] fixed-point sums along the diagonals
};

// Fixed-point scale of the bias-table gradient of one head: a power of two 2^sh such that `bound`
// (what the pairs of one diagonal inside one tile can add up to) stays below 2^30, and its inverse.
// A bound that is zero gives zeros, one that is not finite gives NaN for everything it scales.
__device__ __forceinline__ void drab_fx_scales(float bound, float& fx_scale, float& fx_inv) {
  const int eb = (int)((__float_as_uint(bound) >> 23) & 0xffu) - 126;  // bound < 2^eb
  const bool usable = bound > 0.f && bound < 3.0e38f;
  const int sh = min(max(30 - eb, -120), 120);
  fx_scale = usable ? __uint_as_float((unsigned)(127 + sh) << 23) : 0.f;
  fx_inv = usable ? __uint_as_float((unsigned)(127 - sh) << 23) : (bound == 0.f ? 0.f : __uint_as_float(0x7fc00000u));
}
// The bound itself: |dS| <= 1.1 |dP|, |dP| <= Dv max|dout of the head| max|v| (times the largest
// per-token scale where there is one), and a diagonal meets at most 64 pairs of a (128-row, 64-key) tile.
__device__ __forceinline__ float drab_fx_bound(const BwdParams& bp, int h, bool per_token) {
  const float dmx = __uint_as_float(bp.dout_max[h]);
  const float vmx = __uint_as_float(__hip_atomic_load(bp.absmax + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  const float rmx = per_token ? __uint_as_float(__hip_atomic_load(bp.absmax + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) : 1.0f;
  return dmx * vmx * rmx * ((float)bp.f.Dv * 1.1f * 64.0f);
}

}  // namespace recir_hstu
