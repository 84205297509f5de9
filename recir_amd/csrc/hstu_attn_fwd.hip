// HSTU jagged attention forward for gfx950 (MI355X): kernels and the C ABI declared in
// include/recir_hstu.h.
//
// Reference behaviour being replaced (paths relative to the upstream tree):
//   recir/ops/kjt_split_per_feature.cpp:602-693        per-sequence composite fallback
//   recir/ops/pallas/jagged_hstu_attention.py:378-653  packed accelerator kernel + tail zeroing
//   recir/ops/helion/jagged_hstu_attention.py:297-353  packed kernel, kv loop clamped to the q tile
//
// Kernels in this file
//   hstu_plan_kernel        (sequence, query-tile) work list, heaviest tiles first
//   hstu_fwd_tiled_d128     bf16 / fp8-qk tiled MFMA kernel, head dim 128
//   hstu_fwd_generic        any head dim, fp32 or bf16, one wave per (token, head)
//   hstu_fill_zero          out := 0 when there are no sequences
//   hstu_amax_per_head / hstu_quant_e4m3_per_head   per-head fp8 quantiser
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "recir_hstu.h"

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(16))) float f32x16;

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
  int* ws_count;   // [1] number of valid work items
  int2* ws_items;  // [max_items] (sequence, query tile)
  int T, B, H, Dqk, Dv, N, ctx;
  float alpha;
  unsigned flags;
};

struct SeqInfo {
  int s;        // first packed token
  int n;        // length
  int cap;      // history length n - num_targets (keys j < cap are history)
  int ctx_eff;  // keys j < ctx_eff are visible to every query
};

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
    // the reference unmasks keys whose target-clamped id min(j, cap) equals 0: key 0 (already
    // causal) when cap > 0, every key when cap == 0, none when cap < 0
    si.ctx_eff = (p.ctx > 0 && cap == 0) ? si.n : 0;
  } else {
    si.ctx_eff = p.ctx < si.n ? (p.ctx > 0 ? p.ctx : 0) : si.n;
  }
  return si;
}

__device__ __forceinline__ int end_of_sequences(const Params& p) {
  const bool i32 = p.flags & RECIR_HSTU_FLAG_OFFSETS_I32;
  return clamp_offset(load_index(p.seq_offsets, p.B, i32), 0, p.T);
}

__device__ __forceinline__ bool keep_pair(int m, int j, const SeqInfo& si) {
  return (m == j) || (m >= j && j < si.cap) || (j < si.ctx_eff);
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

// ---------------------------------------------------------------------------------------------
// Work list: one item per (sequence, query tile of BM rows), ordered by tile index descending so
// that the tiles with the longest causal prefix are launched first.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(64) void hstu_plan_kernel(Params p, int BM) {
  const int b = blockIdx.x;
  const SeqInfo si = seq_info(p, b);
  const int my_tiles = (si.n + BM - 1) / BM;
  for (int t = threadIdx.x; t < my_tiles; t += blockDim.x) {
    int rank = 0;
    for (int b2 = 0; b2 < p.B; ++b2) {
      const SeqInfo s2 = seq_info(p, b2);
      const int nt2 = (s2.n + BM - 1) / BM;
      rank += max(0, nt2 - 1 - t) + ((b2 < b && nt2 > t) ? 1 : 0);
    }
    p.ws_items[rank] = make_int2(b, t);
  }
  if (b == 0 && threadIdx.x == 0) {
    int total = 0;
    for (int b2 = 0; b2 < p.B; ++b2) total += (seq_info(p, b2).n + BM - 1) / BM;
    *p.ws_count = total;
  }
}

__global__ void hstu_fill_zero(unsigned short* out, size_t n2) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n2; i += stride) out[i] = 0;
}

// Rows [seq_offsets[B], T) of out := 0, shared by all workgroups of a launch.
template <int NTHREADS>
__device__ __forceinline__ void zero_tail_rows(const Params& p, size_t row_bytes) {
  const int end_all = end_of_sequences(p);
  if (end_all >= p.T) return;
  // row_bytes is a multiple of 2; use 2-byte stores only when 16-byte ones do not fit
  unsigned char* base = (unsigned char*)p.out + (size_t)end_all * row_bytes;
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

// ---------------------------------------------------------------------------------------------
// Generic kernel: one wave per (packed token, head).  Scores for 64 keys at a time are computed
// one key per lane, parked in LDS, and then each lane accumulates its share of the value columns.
// Precision ladder: operands -> fp32 scores -> SiLU in fp32 -> P rounded to the value type ->
// fp32 accumulate -> output type.
// ---------------------------------------------------------------------------------------------
template <bool BF16>
__device__ __forceinline__ float load_elem(const void* base, size_t idx) {
  if (BF16) return bf16_bits_to_float(((const unsigned short*)base)[idx]);
  return ((const float*)base)[idx];
}

constexpr int GENERIC_MAX_D = 512;

template <bool BF16>
__global__ __launch_bounds__(64) void hstu_fwd_generic(Params p) {
  __shared__ float qrow[GENERIC_MAX_D];
  __shared__ float pbuf[64];
  const int lane = threadIdx.x;
  const int r = blockIdx.x, h = blockIdx.y;
  const size_t esz = BF16 ? 2 : 4;
  zero_tail_rows<64>(p, (size_t)p.H * p.Dv * esz);
  if (r >= end_of_sequences(p)) return;

  // b = (first index whose offset exceeds r) - 1
  const bool i32 = p.flags & RECIR_HSTU_FLAG_OFFSETS_I32;
  int lo = 0, hi = p.B + 1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (load_index(p.seq_offsets, mid, i32) > (long long)r) hi = mid; else lo = mid + 1;
  }
  const int b = lo - 1;
  const size_t orow = ((size_t)r * p.H + h) * p.Dv;
  bool ok = b >= 0 && b < p.B;
  SeqInfo si = {0, 0, 0, 0};
  if (ok) {
    si = seq_info(p, b);
    ok = r >= si.s && r < si.s + si.n;
  }
  if (!ok) {  // only reachable with malformed offsets
    for (int d = lane; d < p.Dv; d += 64) {
      if (BF16) ((unsigned short*)p.out)[orow + d] = 0; else ((float*)p.out)[orow + d] = 0.f;
    }
    return;
  }
  const int m = r - si.s;
  for (int d = lane; d < p.Dqk; d += 64)
    qrow[d] = load_elem<BF16>(p.q, ((size_t)r * p.H + h) * p.Dqk + d);
  __syncthreads();

  float scale = 1.0f / (float)p.N;
  if (p.attn_scale) scale = (p.flags & RECIR_HSTU_FLAG_SCALE_PER_TOKEN) ? p.attn_scale[r] : p.attn_scale[0];
  const int rab_w = 2 * p.N - 1;

  float acc[GENERIC_MAX_D / 64];
#pragma unroll
  for (int i = 0; i < GENERIC_MAX_D / 64; ++i) acc[i] = 0.f;

  const int jend = max(m + 1, si.ctx_eff);
  for (int j0 = 0; j0 < jend; j0 += 64) {
    const int j = j0 + lane;
    float pj = 0.f;
    if (j < si.n && keep_pair(m, j, si)) {
      const size_t krow = ((size_t)(si.s + j) * p.H + h) * p.Dqk;
      float dot = 0.f;
      for (int d = 0; d < p.Dqk; ++d) dot = fmaf(qrow[d], load_elem<BF16>(p.k, krow + d), dot);
      float x = dot * p.alpha;
      if (p.rab) {
        int idx = m - j + p.N - 1;
        idx = idx < 0 ? 0 : (idx >= rab_w ? rab_w - 1 : idx);
        x += p.rab[(size_t)h * rab_w + idx];
      }
      pj = x / (1.0f + __expf(-x)) * scale;
      if (BF16) pj = bf16_bits_to_float(float_to_bf16_bits(pj));
    }
    __syncthreads();
    pbuf[lane] = pj;
    __syncthreads();
    const int cnt = min(64, si.n - j0);
    for (int jj = 0; jj < cnt; ++jj) {
      const float pv = pbuf[jj];
      if (pv == 0.f) continue;
      const size_t vrow = ((size_t)(si.s + j0 + jj) * p.H + h) * p.Dv;
#pragma unroll
      for (int i = 0; i < GENERIC_MAX_D / 64; ++i) {
        const int d = lane + 64 * i;
        if (d < p.Dv) acc[i] = fmaf(pv, load_elem<BF16>(p.v, vrow + d), acc[i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < GENERIC_MAX_D / 64; ++i) {
    const int d = lane + 64 * i;
    if (d < p.Dv) {
      if (BF16) ((unsigned short*)p.out)[orow + d] = float_to_bf16_bits(acc[i]);
      else ((float*)p.out)[orow + d] = acc[i];
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Tiled MFMA kernel, head dim 128 (qk and v), bf16 values.
//
// One workgroup (4 waves) per (sequence, query tile of BM = 128 rows, head); wave w owns query rows
// [32w, 32w+32) of the tile.  For every key tile of BN = 64 rows:
//   S^T[kv, q]  = K[kv, d] . Q^T[d, q]        v_mfma_f32_32x32x16_bf16, A = K from LDS, B = Q in VGPRs
//   P^T         = silu(alpha S^T (+rab)) masked, rounded to bf16, kept in registers: the 32x32
//                 accumulator layout (lane = query column, 8 key rows per lane half) is exactly the
//                 B-operand layout of the next contraction
//   O^T[d, q]  += V^T[d, kv] . P^T[kv, q]     A = V^T from LDS (V is transposed while it is staged)
// Neither alpha nor the 1/N scale touches P: without a bias silu(aS) = a S sigmoid(aS), so
// S sigmoid(aS) is accumulated and a * scale is applied once to the fp32 output accumulator.
//
// LDS tiles are XOR-swizzled in 16-byte chunks instead of padded:
//   Ks [BN][128]  chunk' = chunk ^ (row & 7)
//   Vts[128][BN]  chunk' = chunk ^ ((d ^ (d >> 3)) & 7), key order inside a 16-key group permuted
//                 to match the accumulator layout (kv = 16 g + 8 a + 4 half + c  ->  16 g + 8 half + 4 a + c)
// ---------------------------------------------------------------------------------------------
constexpr int BM = 128;
constexpr int BN = 64;
constexpr int HD = 128;

__device__ __forceinline__ int vt_swz(int d) { return (d ^ (d >> 3)) & 7; }

template <bool HAS_RAB, bool FP8_QK>
__global__ __launch_bounds__(256, 2) void hstu_fwd_tiled_d128(Params p) {
  __shared__ __attribute__((aligned(16))) unsigned short Ks[BN * HD];
  __shared__ __attribute__((aligned(16))) unsigned short Vts[HD * BN];
  __shared__ float rabs[HAS_RAB ? (BM + BN) : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int half = lane >> 5;

  zero_tail_rows<256>(p, (size_t)p.H * HD * 2);

  const int item = blockIdx.x / p.H;
  const int h = blockIdx.x - item * p.H;
  if (item >= *p.ws_count) return;
  const int2 it2 = p.ws_items[item];
  const SeqInfo si = seq_info(p, it2.x);
  const int q0 = it2.y * BM;
  if (q0 >= si.n) return;

  const unsigned short* __restrict__ kg = (const unsigned short*)p.k;
  const unsigned short* __restrict__ vg = (const unsigned short*)p.v;
  const size_t row_stride = (size_t)p.H * HD;

  // ---- Q fragments (B operand): lane holds row qw0 + l32, d = 16 kk + 8 half .. +7 ----
  const int qw0 = q0 + wave * 32;
  const int m = qw0 + l32;
  bf16x8 qf[8];
  {
    const bool valid = m < si.n;
    const unsigned short* qrow = (const unsigned short*)p.q + ((size_t)(si.s + (valid ? m : 0)) * p.H + h) * HD;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      uint4 t = valid ? *(const uint4*)(qrow + kk * 16 + half * 8) : make_uint4(0, 0, 0, 0);
      qf[kk] = *(bf16x8*)&t;
    }
  }

  f32x16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

  const float kLog2e = 1.4426950408889634f;
  const float c1 = HAS_RAB ? -kLog2e : -p.alpha * kLog2e;
  const int rab_w = 2 * p.N - 1;

  const int m_lo = qw0;
  const int m_hi = min(qw0 + 31, si.n - 1);
  const bool wave_has_rows = m_lo < si.n;

  const int kv_end = min(si.n, max(q0 + BM, si.ctx_eff));
  const int nkv = (kv_end + BN - 1) / BN;

  for (int it = 0; it < nkv; ++it) {
    const int k0 = it * BN;
    const int k1 = k0 + BN;
    // workgroup-uniform skip: tile holds only target keys, none on this q tile's diagonal, and no
    // contextual keys
    if (k0 >= si.cap && k1 <= q0 && k0 >= si.ctx_eff) continue;

    __syncthreads();  // all waves done reading the previous tile
    // ---- stage K: 4 passes of 16 rows, 16 threads x 16 B per row ----
    {
      const int chunk = tid & 15;
#pragma unroll
      for (int ps = 0; ps < 4; ++ps) {
        const int row = (tid >> 4) + ps * 16;
        const int j = k0 + row;
        uint4 t = make_uint4(0, 0, 0, 0);
        if (j < si.n) t = *(const uint4*)(kg + (size_t)(si.s + j) * row_stride + (size_t)h * HD + chunk * 8);
        *(uint4*)&Ks[row * HD + ((chunk ^ (row & 7)) * 8)] = t;
      }
    }
    // ---- stage V transposed: thread (g, e) loads kv rows 4g..4g+3 at d = 8e..8e+7 ----
    {
      const int g = tid >> 4, e = tid & 15;
      uint4 vr[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int j = k0 + 4 * g + c;
        vr[c] = make_uint4(0, 0, 0, 0);
        if (j < si.n) vr[c] = *(const uint4*)(vg + (size_t)(si.s + j) * row_stride + (size_t)h * HD + e * 8);
      }
      const int g16 = g >> 2, a = (g >> 1) & 1, hf = g & 1;
      const int c16 = 2 * g16 + hf;
      const unsigned* w0 = (const unsigned*)&vr[0];
      const unsigned* w1 = (const unsigned*)&vr[1];
      const unsigned* w2 = (const unsigned*)&vr[2];
      const unsigned* w3 = (const unsigned*)&vr[3];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int wi = i >> 1;
        uint2 o;
        if (i & 1) {
          o.x = (w0[wi] >> 16) | (w1[wi] & 0xffff0000u);
          o.y = (w2[wi] >> 16) | (w3[wi] & 0xffff0000u);
        } else {
          o.x = (w0[wi] & 0xffffu) | (w1[wi] << 16);
          o.y = (w2[wi] & 0xffffu) | (w3[wi] << 16);
        }
        const int d = 8 * e + i;
        *(uint2*)&Vts[d * BN + ((c16 ^ vt_swz(d)) * 8) + a * 4] = o;
      }
    }
    if (HAS_RAB) {
      // band of bias entries this (q tile, kv tile) can touch: index (m - j) + N - 1
      const int base = q0 - k0 - (BN - 1) + p.N - 1;
      if (tid < BM + BN - 1) {
        int idx = base + tid;
        idx = idx < 0 ? 0 : (idx >= rab_w ? rab_w - 1 : idx);
        rabs[tid] = p.rab[(size_t)h * rab_w + idx];
      }
    }
    __syncthreads();

    // wave-level classification of this (32 query rows) x (64 keys) block
    if (!wave_has_rows) continue;
    const bool any_kept = (k0 <= m_hi && k1 > m_lo) /* diagonal crosses */ ||
                          (k0 < si.cap && k0 <= m_hi) /* causal history */ || (k0 < si.ctx_eff);
    if (!any_kept) continue;
    const bool full = (k1 - 1 <= m_lo) && (k1 <= si.cap);  // implies k1 <= n

    // ---- S^T = K Q^T ----
    f32x16 sacc[2];
#pragma unroll
    for (int kvb = 0; kvb < 2; ++kvb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[kvb][r] = 0.f;
      const int row = kvb * 32 + l32;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const int chunk = kk * 2 + half;
        const bf16x8 a = *(const bf16x8*)&Ks[row * HD + ((chunk ^ (row & 7)) * 8)];
        sacc[kvb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], sacc[kvb], 0, 0, 0);
      }
    }

    // ---- P^T = silu(...) with the mask, packed to bf16 B operands ----
    bf16x8 pb[4];
#pragma unroll
    for (int kvb = 0; kvb < 2; ++kvb) {
      float pv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int jl = kvb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        float s = sacc[kvb][r];
        float x = s;
        if (HAS_RAB) {
          x = s * p.alpha + rabs[(m - q0) - jl + (BN - 1)];
          s = x;
        }
        const float ex = __builtin_amdgcn_exp2f(x * c1);
        const float rc = __builtin_amdgcn_rcpf(1.0f + ex);
        float pe = s * rc;
        if (!full) {
          const int j = k0 + jl;
          pe = (j < si.n && keep_pair(m, j, si)) ? pe : 0.f;
        }
        pv[r] = pe;
      }
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        unsigned w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(pv[8 * s2 + 2 * i], pv[8 * s2 + 2 * i + 1]);
        pb[kvb * 2 + s2] = *(bf16x8*)w;
      }
    }

    // ---- O^T += V^T P^T ----
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int d = db * 32 + l32;
      const int sw = vt_swz(d);
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) {
        const int c16 = s2 * 2 + half;
        const bf16x8 a = *(const bf16x8*)&Vts[d * BN + ((c16 ^ sw) * 8)];
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[s2], acc[db], 0, 0, 0);
      }
    }
  }

  // ---- epilogue: O^T accumulators -> out[s + m, h, :] ----
  if (m < si.n) {
    float oscale = 1.0f / (float)p.N;
    if (p.attn_scale)
      oscale = (p.flags & RECIR_HSTU_FLAG_SCALE_PER_TOKEN) ? p.attn_scale[si.s + m] : p.attn_scale[0];
    if (!HAS_RAB) oscale *= p.alpha;
    unsigned short* orow = (unsigned short*)p.out + ((size_t)(si.s + m) * p.H + h) * HD;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        uint2 o;
        o.x = pack_bf16x2(acc[db][4 * rq + 0] * oscale, acc[db][4 * rq + 1] * oscale);
        o.y = pack_bf16x2(acc[db][4 * rq + 2] * oscale, acc[db][4 * rq + 3] * oscale);
        *(uint2*)(orow + db * 32 + 8 * rq + 4 * half) = o;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------------
thread_local char g_err[512] = "";
thread_local const char* g_last_kernel = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail((int)e, "%s: %s", what, hipGetErrorString(e));
  return 0;
}

size_t max_items(int T, int B) { return (size_t)((T + BM - 1) / BM) + (size_t)B; }

}  // namespace

extern "C" {

int recir_hstu_abi_version(void) { return RECIR_HSTU_ABI_VERSION; }
const char* recir_hstu_last_error(void) { return g_err; }
const char* recir_hstu_last_kernel(void) { return g_last_kernel; }

size_t recir_hstu_attn_fwd_workspace_bytes(int32_t T, int32_t B, int32_t H, int32_t Dqk, int32_t Dv,
                                           int32_t dtype) {
  (void)H; (void)Dqk; (void)Dv; (void)dtype;
  if (T < 0 || B < 0) return 0;
  return 16 + sizeof(int2) * max_items(T, B);
}

int recir_hstu_attn_fwd(const void* q, const void* k, const void* v, void* out,
                        const void* seq_offsets, const void* num_targets, const float* rab,
                        const float* attn_scale, const float* q_scale, const float* k_scale,
                        int32_t T, int32_t B, int32_t H, int32_t Dqk, int32_t Dv,
                        int32_t max_seq_len, int32_t contextual_seq_len, float alpha, int32_t dtype,
                        uint32_t flags, void* workspace, size_t workspace_bytes, void* hip_stream) {
  hipStream_t stream = (hipStream_t)hip_stream;
  if (T < 0 || B < 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "negative size: T=%d B=%d", T, B);
  if (H <= 0 || Dqk <= 0 || Dv <= 0)
    return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "H, Dqk, Dv must be positive: H=%d Dqk=%d Dv=%d", H, Dqk, Dv);
  if (max_seq_len <= 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "max_seq_len must be positive, got %d", max_seq_len);
  if (contextual_seq_len < 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "contextual_seq_len must be >= 0, got %d", contextual_seq_len);
  if (dtype != RECIR_HSTU_DTYPE_BF16 && dtype != RECIR_HSTU_DTYPE_FP32 && dtype != RECIR_HSTU_DTYPE_FP8_E4M3)
    return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
  if (T == 0) return RECIR_HSTU_OK;
  if (!q || !k || !v || !out) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "q, k, v, out must be non-null");
  if (!seq_offsets) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "seq_offsets must be non-null");
  if (dtype == RECIR_HSTU_DTYPE_FP8_E4M3 && (!q_scale || !k_scale))
    return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "fp8 q/k need q_scale and k_scale");
  const unsigned variant = (flags & RECIR_HSTU_FLAG_KERNEL_MASK) >> RECIR_HSTU_FLAG_KERNEL_SHIFT;

  Params p;
  memset(&p, 0, sizeof(p));
  p.q = q; p.k = k; p.v = v; p.out = out;
  p.seq_offsets = seq_offsets; p.num_targets = num_targets;
  p.rab = rab; p.attn_scale = attn_scale; p.q_scale = q_scale; p.k_scale = k_scale;
  p.T = T; p.B = B; p.H = H; p.Dqk = Dqk; p.Dv = Dv; p.N = max_seq_len; p.ctx = contextual_seq_len;
  p.alpha = alpha; p.flags = flags;

  const size_t esz = dtype == RECIR_HSTU_DTYPE_FP32 ? 4 : 2;
  if (B == 0) {
    // a fill kernel rather than a runtime memset, so that the call can be captured in a graph
    const size_t bytes = (size_t)T * H * Dv * esz;
    hipLaunchKernelGGL(hstu_fill_zero, dim3(1024), dim3(256), 0, stream, (unsigned short*)out, bytes / 2);
    if (int rc = launch_status("hstu_fill_zero")) return rc;
    g_last_kernel = "fill_zero";
    return RECIR_HSTU_OK;
  }

  const bool tiled_ok = dtype == RECIR_HSTU_DTYPE_BF16 && Dqk == HD && Dv == HD &&
                        (((size_t)q | (size_t)k | (size_t)v | (size_t)out) & 15) == 0;
  bool use_tiled = tiled_ok;
  if (variant == 1) use_tiled = false;
  if (variant >= 2 && !tiled_ok)
    return fail(RECIR_HSTU_ERR_UNSUPPORTED, "tiled kernel needs bf16, Dqk = Dv = 128 and 16-byte aligned tensors");

  if (use_tiled) {
    const size_t need = recir_hstu_attn_fwd_workspace_bytes(T, B, H, Dqk, Dv, dtype);
    if (!workspace || workspace_bytes < need || ((size_t)workspace & 15))
      return fail(RECIR_HSTU_ERR_WORKSPACE, "workspace of %zu bytes (16-byte aligned) required, got %zu at %p", need,
                  workspace_bytes, workspace);
    p.ws_count = (int*)workspace;
    p.ws_items = (int2*)((char*)workspace + 16);
    const size_t items = max_items(T, B);
    if (items * (size_t)H > 0x7fffffffull) return fail(RECIR_HSTU_ERR_UNSUPPORTED, "grid too large");
    hipLaunchKernelGGL(hstu_plan_kernel, dim3(B), dim3(64), 0, stream, p, BM);
    if (int rc = launch_status("hstu_plan_kernel")) return rc;
    const dim3 grid((unsigned)(items * H));
    if (rab) hipLaunchKernelGGL((hstu_fwd_tiled_d128<true, false>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((hstu_fwd_tiled_d128<false, false>), grid, dim3(256), 0, stream, p);
    if (int rc = launch_status("hstu_fwd_tiled_d128")) return rc;
    g_last_kernel = rab ? "tiled_d128_bf16_rab" : "tiled_d128_bf16";
    return RECIR_HSTU_OK;
  }

  if (dtype == RECIR_HSTU_DTYPE_FP8_E4M3)
    return fail(RECIR_HSTU_ERR_UNSUPPORTED, "fp8 q/k is implemented for Dqk = Dv = 128 only");
  if (Dqk > GENERIC_MAX_D || Dv > GENERIC_MAX_D)
    return fail(RECIR_HSTU_ERR_UNSUPPORTED, "head dims above %d are not supported (Dqk=%d Dv=%d)", GENERIC_MAX_D, Dqk, Dv);
  if (H > 65535) return fail(RECIR_HSTU_ERR_UNSUPPORTED, "more than 65535 heads");
  const dim3 grid((unsigned)T, (unsigned)H);
  if (dtype == RECIR_HSTU_DTYPE_BF16) hipLaunchKernelGGL(hstu_fwd_generic<true>, grid, dim3(64), 0, stream, p);
  else hipLaunchKernelGGL(hstu_fwd_generic<false>, grid, dim3(64), 0, stream, p);
  if (int rc = launch_status("hstu_fwd_generic")) return rc;
  g_last_kernel = dtype == RECIR_HSTU_DTYPE_BF16 ? "generic_bf16" : "generic_fp32";
  return RECIR_HSTU_OK;
}

int recir_hstu_quantize_e4m3_per_head(const void* x_bf16, void* codes_u8, float* scale, int32_t T,
                                      int32_t H, int32_t D, void* hip_stream) {
  (void)x_bf16; (void)codes_u8; (void)scale; (void)T; (void)H; (void)D; (void)hip_stream;
  return fail(RECIR_HSTU_ERR_UNSUPPORTED, "fp8 quantiser not built yet");
}

}  // extern "C"
