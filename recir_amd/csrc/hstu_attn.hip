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
//   hstu_bwd_generic_dq / hstu_bwd_generic_dkv   backward, any head dim, one wave per (token, head)
//   hstu_bwd_dq_d128 / hstu_bwd_dkv_d128         backward, bf16 tiled MFMA kernels, head dim 128
//   hstu_fill_zero          out := 0 when there are no sequences
//   hstu_amax_per_head / hstu_quant_e4m3_per_head   per-head fp8 quantiser
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "recir_hstu.h"
#include "recir_jagged.h"

#include "hstu_common.h"
#include "hstu_plan.h"
#include "hstu_tiled_d128_dl.h"
#include "hstu_bwd_generic.h"
#include "hstu_mfma_any.h"
#include "hstu_bwd_d128.h"
#include "hstu_calibration.h"
#include "jagged_rows.h"
#include "ts_pos_embeddings.h"
#include "counting_sort.h"

#include <rocprim/rocprim.hpp>

using namespace recir_hstu;

namespace {

// ---------------------------------------------------------------------------------------------
// Per-head e4m3 quantiser: amax per head (bf16 magnitudes compare as integers), scale = amax / 448,
// codes = e4m3(clamp(x / scale)).  Eight elements (16 bytes) per thread; D is a multiple of 8.
// ---------------------------------------------------------------------------------------------
// head of 16-byte chunk i of a [T, H, D] bf16 tensor (D8 = D / 8 chunks per row).  The general
// form is two 64-bit divisions per chunk, which costs more than moving the chunk: shifts and masks
// when D8 and H are powers of two (d8_shift, h_mask >= 0), 32-bit arithmetic when the index fits.
__device__ __forceinline__ int quant_head(size_t i, int D8, int H, int d8_shift, int h_mask) {
  if (d8_shift >= 0) {
    const size_t row = i >> d8_shift;
    return h_mask >= 0 ? (int)(row & (size_t)h_mask) : (int)(row % (size_t)H);
  }
  if (i <= 0xffffffffull) return (int)(((unsigned)i / (unsigned)D8) % (unsigned)H);
  return (int)((i / (size_t)D8) % (size_t)H);
}

__global__ void hstu_quant_clear(unsigned* amax_bits, int H) {
  for (int h = threadIdx.x; h < H; h += blockDim.x) amax_bits[h] = 0u;
}

// Per-head maximum magnitude.  The maxima of a block are gathered in LDS (integer max on the bf16
// magnitude bits) and only then merged into the H global words: one global atomic per element chunk
// would queue millions of them on H addresses.
constexpr int QUANT_LDS_HEADS = 4096;
#ifndef QUANT_AMAX_BLOCKS
#define QUANT_AMAX_BLOCKS 1024
#endif
// Chunks of the rows a quantiser launch looks at: all T rows, or only those below the end of the
// sequences (seq_end points at seq_offsets[B], read on the device): rows after it are padding whose
// contents (possibly Inf or NaN) must not reach a head's scale.
__device__ __forceinline__ size_t quant_valid_chunks(size_t n8, const void* seq_end, int i32, int T, int H, int D8) {
  if (!seq_end) return n8;
  const long long e = i32 ? (long long)*(const int*)seq_end : *(const long long*)seq_end;
  const size_t rows = (size_t)(e < 0 ? 0 : (e > T ? T : e));
  const size_t v = rows * (size_t)H * (size_t)D8;
  return v < n8 ? v : n8;
}

__global__ __launch_bounds__(256) void hstu_quant_amax(const u32x4* x, unsigned* amax_bits, unsigned* partial, size_t n8_all, int H, int D8, int d8_shift, int h_mask,
                                                       const void* seq_end, int i32, int T) {
  __shared__ unsigned lmax[QUANT_LDS_HEADS];
  const size_t n8 = quant_valid_chunks(n8_all, seq_end, i32, T, H, D8);
  const bool in_lds = H <= QUANT_LDS_HEADS;
  if (in_lds) {
    for (int h = threadIdx.x; h < H; h += blockDim.x) lmax[h] = 0u;
    __syncthreads();
  }
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  // When the grid stride is a multiple of the chunks of one token (D8 * H), a thread meets the same
  // head in every iteration: it keeps one running maximum and merges it once.
  const bool fixed_head = stride % ((size_t)D8 * H) == 0;
  constexpr int U = 4;  // loads in flight per thread
  const size_t first = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  unsigned run = 0;
  for (size_t i0 = first; i0 < n8; i0 += stride * U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t i = i0 + u * stride;
      v[u] = i < n8 ? x[i] : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t i = i0 + u * stride;
      unsigned mx = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        mx = max(mx, (v[u][j] << 16) & 0x7fffffffu);
        mx = max(mx, v[u][j] & 0x7fff0000u);
      }
      if (fixed_head) {
        run = max(run, mx);
      } else if (i < n8) {
        const int h = quant_head(i, D8, H, d8_shift, h_mask);
        if (in_lds) atomicMax(&lmax[h], mx);
        else atomicMax(&amax_bits[h], mx);
      }
    }
  }
  if (fixed_head && first < n8) {
    const int h = quant_head(first, D8, H, d8_shift, h_mask);
    if (in_lds) atomicMax(&lmax[h], run);
    else atomicMax(&amax_bits[h], run);
  }
  if (in_lds) {
    __syncthreads();
    // with a scratch table every block leaves its maxima for the finalising kernel; otherwise H
    // global atomics per block (a thousand blocks on H addresses: about 12 us of queueing)
    for (int h = threadIdx.x; h < H; h += blockDim.x) {
      if (partial) partial[(size_t)blockIdx.x * H + h] = lmax[h];
      else if (lmax[h]) atomicMax(&amax_bits[h], lmax[h]);
    }
  }
}

__global__ __launch_bounds__(1024) void hstu_quant_finalize(float* scale, const unsigned* partial, int blocks, int H) {
  __shared__ unsigned red[QUANT_LDS_HEADS];
  if (partial) {  // H <= QUANT_LDS_HEADS on this path
    for (int h = threadIdx.x; h < H; h += blockDim.x) red[h] = 0u;
    __syncthreads();
    const int n = blocks * H;
    for (int i = threadIdx.x; i < n; i += blockDim.x) atomicMax(&red[i % H], partial[i]);
    __syncthreads();
  }
  for (int h = threadIdx.x; h < H; h += blockDim.x) {
    const unsigned bits = partial ? red[h] : ((unsigned*)scale)[h];
    scale[h] = fmaxf(__uint_as_float(bits), 1e-12f) / 448.0f;
  }
}

__global__ __launch_bounds__(256) void hstu_quant_encode(const u32x4* x, u32x2* codes, const float* scale, size_t n8, int H, int D8, int d8_shift, int h_mask,
                                                         const void* seq_end, int i32, int T) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const size_t valid = quant_valid_chunks(n8, seq_end, i32, T, H, D8);
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += stride) {
    if (i >= valid) { codes[i] = u32x2{0u, 0u}; continue; }  // padding rows: zero codes
    const u32x4 v = x[i];
    const float sc = scale[quant_head(i, D8, H, d8_shift, h_mask)];
    float y[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      y[2 * j] = __uint_as_float(v[j] << 16) / sc;
      y[2 * j + 1] = __uint_as_float(v[j] & 0xffff0000u) / sc;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) y[j] = fminf(fmaxf(y[j], -448.0f), 448.0f);
    u32x2 o;
    int w = 0;
    w = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], w, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], w, true);
    o.x = (unsigned)w;
    w = 0;
    w = __builtin_amdgcn_cvt_pk_fp8_f32(y[4], y[5], w, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(y[6], y[7], w, true);
    o.y = (unsigned)w;
    codes[i] = o;
  }
}

__global__ __launch_bounds__(256) void hstu_calibration_copy(u32x4* dst, const u32x4* src, size_t n16) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

// n2 two-byte words := 0: 16-byte stores for the aligned middle, two-byte stores for what is left at
// either end
__global__ void hstu_fill_zero(unsigned short* out, size_t n2) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const size_t first = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t head = (size_t)((16 - ((size_t)out & 15)) & 15) / 2;  // words before the first 16-byte boundary
  if (head > n2) head = n2;
  const size_t n16 = (n2 - head) / 8;
  u32x4* mid = (u32x4*)(out + head);
  for (size_t i = first; i < n16; i += stride) mid[i] = u32x4{0u, 0u, 0u, 0u};
  const size_t tail0 = head + n16 * 8;
  for (size_t i = first; i < head; i += stride) out[i] = 0;
  for (size_t i = tail0 + first; i < n2; i += stride) out[i] = 0;
}

// ---------------------------------------------------------------------------------------------
// Generic kernel: one wave per (packed token, head).  Scores for 64 keys at a time are computed
// one key per lane, parked in LDS, and then each lane accumulates its share of the value columns.
// Precision ladder: operands -> fp32 scores -> SiLU in fp32 -> P rounded to the value type ->
// fp32 accumulate -> output type.
// ---------------------------------------------------------------------------------------------
constexpr int GENERIC_MAX_D = 512;

template <int ELT>
__global__ __launch_bounds__(64) void hstu_fwd_generic(Params p) {
  __shared__ float qrow[GENERIC_MAX_D];
  __shared__ float pbuf[64];
  const int lane = threadIdx.x;
  const int r = blockIdx.x, h = blockIdx.y;
  const size_t esz = ELT == ELT_FP32 ? 4 : 2;
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
      store_elem<ELT>(p.out, orow + d, 0.f);
    }
    return;
  }
  const int m = r - si.s;
  for (int d = lane; d < p.Dqk; d += 64)
    qrow[d] = load_elem<ELT>(p.q, ((size_t)r * p.H + h) * p.Dqk + d);
  __syncthreads();

  float scale = 1.0f / (float)p.N;
  if (p.attn_scale) scale = (p.flags & RECIR_HSTU_FLAG_SCALE_PER_TOKEN) ? p.attn_scale[r] : p.attn_scale[0];
  const int rab_w = 2 * p.N - 1;

  float acc[GENERIC_MAX_D / 64];
#pragma unroll
  for (int i = 0; i < GENERIC_MAX_D / 64; ++i) acc[i] = 0.f;

  const bool noncausal = p.flags & RECIR_HSTU_FLAG_MASK_NONCAUSAL;  // then keys after the query count too
  const int jend = noncausal ? si.n : max(m + 1, si.ctx_eff);
  for (int j0 = 0; j0 < jend; j0 += 64) {
    const int j = j0 + lane;
    float pj = 0.f;
    if (j < si.n && keep_pair(m, j, si, noncausal)) {
      const size_t krow = ((size_t)(si.s + j) * p.H + h) * p.Dqk;
      float dot = 0.f;
      for (int d = 0; d < p.Dqk; ++d) dot = fmaf(qrow[d], load_elem<ELT>(p.k, krow + d), dot);
      float x = dot * p.alpha;
      if (p.rab) {
        const int idx = m - j + p.N - 1;  // outside the table (sequence longer than max_seq_len): no bias
        if (idx >= 0 && idx < rab_w) x += p.rab[(size_t)h * rab_w + idx];
      }
      pj = x / (1.0f + __expf(-x)) * scale;
      pj = round_to_elem<ELT>(pj);
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
        if (d < p.Dv) acc[i] = fmaf(pv, load_elem<ELT>(p.v, vrow + d), acc[i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < GENERIC_MAX_D / 64; ++i) {
    const int d = lane + 64 * i;
    if (d < p.Dv) {
      store_elem<ELT>(p.out, orow + d, acc[i]);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------------
thread_local char g_err[512] = "";
thread_local const char* g_last_kernel = "";
#ifdef HSTU_TRACE
unsigned long long* g_trace_buffer = nullptr;  // device memory of the next forward launches' phase records
size_t g_trace_words = 0;
#endif

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

// Do the tensors one call streams (n_qk of [T, H, Dqk] with qk_bytes per element, n_v of [T, H, Dv] in
// bf16) exceed the 256 MB last-level cache?
bool tensors_exceed_llc(int T, int H, int Dqk, int Dv, int qk_bytes, int n_each) {
  const size_t bytes = (size_t)T * H * ((size_t)Dqk * qk_bytes + (size_t)Dv * 2) * n_each;
  return bytes > ((size_t)256 << 20);
}

#ifndef BWD_GROUP_TENSORS
#define BWD_GROUP_TENSORS 1000000  // backward: grouped lists only on request until measured
#endif
// upper bound on the (sequence, query tile, head) items of a call
size_t max_items(int T, int B, int H) { return ((size_t)((T + BM - 1) / BM) + (size_t)B) * (size_t)H; }
constexpr size_t WS_HEADER = 64;

template <bool SEMI, bool HAS_RAB>
void launch_bwd_tiled_as(dim3 grid, dim3 grid_k, hipStream_t stream, const BwdParams& bk, const BwdParams& bq) {
  const bool per_token = bk.f.attn_scale && (bk.f.flags & RECIR_HSTU_FLAG_SCALE_PER_TOKEN);
  if (per_token) hipLaunchKernelGGL((hstu_bwd_dkv_d128<SEMI, HAS_RAB, true>), grid_k, dim3(256), 0, stream, bk);
  else hipLaunchKernelGGL((hstu_bwd_dkv_d128<SEMI, HAS_RAB, false>), grid_k, dim3(256), 0, stream, bk);
  if constexpr (HAS_RAB) {
    if (bq.drab) {  // the query-tile kernel also sums dS along the diagonals
      if (per_token) hipLaunchKernelGGL((hstu_bwd_dq_d128<SEMI, true, true, true>), grid, dim3(256), 0, stream, bq);
      else hipLaunchKernelGGL((hstu_bwd_dq_d128<SEMI, true, false, true>), grid, dim3(256), 0, stream, bq);
      return;
    }
  }
  if (per_token) hipLaunchKernelGGL((hstu_bwd_dq_d128<SEMI, HAS_RAB, true>), grid, dim3(256), 0, stream, bq);
  else hipLaunchKernelGGL((hstu_bwd_dq_d128<SEMI, HAS_RAB, false>), grid, dim3(256), 0, stream, bq);
}
void launch_bwd_tiled(bool semi, bool has_rab, dim3 grid, dim3 grid_k, hipStream_t stream, const BwdParams& bk, const BwdParams& bq) {
  if (semi) {
    if (has_rab) launch_bwd_tiled_as<true, true>(grid, grid_k, stream, bk, bq);
    else launch_bwd_tiled_as<true, false>(grid, grid_k, stream, bk, bq);
  } else {
    if (has_rab) launch_bwd_tiled_as<false, true>(grid, grid_k, stream, bk, bq);
    else launch_bwd_tiled_as<false, false>(grid, grid_k, stream, bk, bq);
  }
}

// Padded head dim of the general MFMA kernels for a call, 0 when they do not take it: the larger head
// dim at most 256 (fp32: 128, its tiles are twice as wide).
int mfma_any_padded_dim(int Dqk, int Dv, int dtype) {
  const bool f32 = dtype == RECIR_HSTU_DTYPE_FP32;
  if (dtype != RECIR_HSTU_DTYPE_BF16 && dtype != RECIR_HSTU_DTYPE_FP16 && !f32) return 0;
  const int d = Dqk > Dv ? Dqk : Dv;
  if (d < 1 || d > (f32 ? 128 : 256)) return 0;
  return d <= 32 ? 32 : (d <= 64 ? 64 : (d <= 128 ? 128 : 256));
}
// Rows of Dqk and of Dv elements are multiples of 16 bytes (with 16-byte aligned tensors every row then
// starts at such a multiple, and the general MFMA kernels move rows in 16-byte pieces).
bool rows_are_16_byte_multiples(int Dqk, int Dv, int dtype) {
  const int per_chunk = dtype == RECIR_HSTU_DTYPE_FP32 ? 4 : 8;
  return Dqk % per_chunk == 0 && Dv % per_chunk == 0;
}
// "mfma_bf16_d64", "bwd_mfma_fp32_d32_elems", ...: "_elems" where the rows are aligned to the element only
const char* mfma_any_name(bool bwd, int dtype, int dp, bool aligned) {
  static thread_local char name[48];
  const char* t = dtype == RECIR_HSTU_DTYPE_FP16 ? "fp16" : (dtype == RECIR_HSTU_DTYPE_FP32 ? "fp32" : "bf16");
  snprintf(name, sizeof(name), "%smfma_%s_d%d%s", bwd ? "bwd_" : "", t, dp, aligned ? "" : "_elems");
  return name;
}

template <bool FP8>
void launch_dl(bool has_rab, bool semi, dim3 grid, hipStream_t stream, const Params& p) {
  if (semi) {
    if (has_rab) hipLaunchKernelGGL((hstu_fwd_tiled_d128_dl<true, FP8, true>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((hstu_fwd_tiled_d128_dl<false, FP8, true>), grid, dim3(256), 0, stream, p);
  } else {
    if (has_rab) hipLaunchKernelGGL((hstu_fwd_tiled_d128_dl<true, FP8, false>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((hstu_fwd_tiled_d128_dl<false, FP8, false>), grid, dim3(256), 0, stream, p);
  }
}

}  // namespace

extern "C" {

int recir_hstu_abi_version(void) { return RECIR_HSTU_ABI_VERSION; }
const char* recir_hstu_last_error(void) { return g_err; }
const char* recir_hstu_last_kernel(void) { return g_last_kernel; }

size_t recir_hstu_attn_fwd_workspace_bytes(int32_t T, int32_t B, int32_t H, int32_t Dqk, int32_t Dv,
                                           int32_t dtype) {
  (void)Dqk; (void)Dv; (void)dtype;
  if (T < 0 || B < 0 || H <= 0) return 0;
  // list lengths + NUM_XCD work lists, each able to hold every item of the call
  return WS_HEADER + sizeof(WorkItem) * max_items(T, B, H) * NUM_XCD;
}

int recir_hstu_attn_fwd(const void* q, const void* k, const void* v, void* out,
                        const void* seq_offsets, const void* num_targets, const float* rab,
                        const float* attn_scale, const float* q_scale, const float* k_scale,
                        int32_t T, int32_t B, int32_t H, int32_t Dqk, int32_t Dv,
                        int32_t max_seq_len, int32_t contextual_seq_len, int32_t max_attn_len,
                        int32_t full_attn_size, float alpha, int32_t dtype, uint32_t flags,
                        void* workspace, size_t workspace_bytes, void* hip_stream) {
  hipStream_t stream = (hipStream_t)hip_stream;
  if (T < 0 || B < 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "negative size: T=%d B=%d", T, B);
  if (max_attn_len < 0 || full_attn_size < 0)
    return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "max_attn_len and full_attn_size must be >= 0, got %d and %d",
                max_attn_len, full_attn_size);
  if (H <= 0 || Dqk <= 0 || Dv <= 0)
    return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "H, Dqk, Dv must be positive: H=%d Dqk=%d Dv=%d", H, Dqk, Dv);
  if (max_seq_len <= 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "max_seq_len must be positive, got %d", max_seq_len);
  if (contextual_seq_len < 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "contextual_seq_len must be >= 0, got %d", contextual_seq_len);
  if (dtype != RECIR_HSTU_DTYPE_BF16 && dtype != RECIR_HSTU_DTYPE_FP32 && dtype != RECIR_HSTU_DTYPE_FP8_E4M3 &&
      dtype != RECIR_HSTU_DTYPE_FP16)
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
  p.max_attn_len = max_attn_len; p.full_attn_size = full_attn_size;
  const bool semi = max_attn_len > 0;

  const size_t esz = dtype == RECIR_HSTU_DTYPE_FP32 ? 4 : 2;
  if (B == 0) {
    // a fill kernel rather than a runtime memset, so that the call can be captured in a graph
    const size_t bytes = (size_t)T * H * Dv * esz;
    hipLaunchKernelGGL(hstu_fill_zero, dim3(1024), dim3(256), 0, stream, (unsigned short*)out, bytes / 2);
    if (int rc = launch_status("hstu_fill_zero")) return rc;
    g_last_kernel = "fill_zero";
    return RECIR_HSTU_OK;
  }

  const bool fp8 = dtype == RECIR_HSTU_DTYPE_FP8_E4M3;
  const bool f16 = dtype == RECIR_HSTU_DTYPE_FP16;
  const bool noncausal = (flags & RECIR_HSTU_FLAG_MASK_NONCAUSAL) != 0;
  const bool aligned = (((size_t)q | (size_t)k | (size_t)v | (size_t)out) & 15) == 0;
  // The kernels written for head dim 128 keep a bias divided by the score multiplier in their
  // accumulators: not possible with alpha = 0 (the scores are then the bias alone).
  const bool bias_needs_other = rab && !std::isnormal(1.0f / alpha);
  const bool d128_ok = (dtype == RECIR_HSTU_DTYPE_BF16 || fp8) && Dqk == HD && Dv == HD && aligned && !noncausal && !bias_needs_other;
  // the MFMA kernels for other head dims, fp16 and the remaining masks (hstu_mfma_any.h)
  const int any_dp = mfma_any_padded_dim(Dqk, Dv, dtype);
  const bool elem_aligned = (((size_t)q | (size_t)k | (size_t)v | (size_t)out) & (esz - 1)) == 0;
  const bool any_ok = any_dp != 0 && elem_aligned;
  const bool any_aligned = aligned && rows_are_16_byte_multiples(Dqk, Dv, dtype);
  if (variant > 3) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "unknown kernel selector %u", variant);
  if (variant == 3 && !d128_ok)
    return fail(RECIR_HSTU_ERR_UNSUPPORTED,
                "the head-dim-128 kernel needs bf16 or fp8 q/k, Dqk = Dv = 128, 16-byte aligned tensors, the causal or "
                "semi-local mask and alpha != 0 with a bias");
  if (variant == 2 && !any_ok)
    return fail(RECIR_HSTU_ERR_UNSUPPORTED,
                "the general MFMA kernel needs bf16, fp16 or fp32 and head dims up to 256 (fp32: 128)");
  if (fp8 && !d128_ok)
    return fail(RECIR_HSTU_ERR_UNSUPPORTED,
                "fp8 q/k is implemented for Dqk = Dv = 128, 16-byte aligned tensors, the causal or semi-local mask (and alpha != 0 with a bias)");
  if (fp8 && (variant == 1 || variant == 2)) return fail(RECIR_HSTU_ERR_UNSUPPORTED, "fp8 q/k runs on the head-dim-128 kernel only");
  const bool use_tiled = d128_ok && (variant == 0 || variant == 3);
  const bool use_any = !use_tiled && any_ok && variant != 1;

  if (use_tiled || use_any) {
    const size_t need = recir_hstu_attn_fwd_workspace_bytes(T, B, H, Dqk, Dv, dtype);
    if (!workspace || workspace_bytes < need || ((size_t)workspace & 15))
      return fail(RECIR_HSTU_ERR_WORKSPACE, "workspace of %zu bytes (16-byte aligned) required, got %zu at %p", need,
                  workspace_bytes, workspace);
    const size_t items = max_items(T, B, H);
    p.ws_counts = (int*)workspace;
    p.ws_items = (WorkItem*)((char*)workspace + WS_HEADER);
    p.items_cap = (int)items;
    const int bm = BM;
    int plan_mode = PLAN_SHIFT_ODD | PLAN_PAIR_CU;  // (two workgroups per CU)
    // q, k, v and out beyond the last-level cache: lists ordered by groups of pairs (hstu_plan.h)
    if ((flags & RECIR_HSTU_FLAG_GROUPED_LISTS) || tensors_exceed_llc(T, H, Dqk, Dv, fp8 ? 1 : 2, 2)) plan_mode |= PLAN_GROUP;
    // slots per XCD the launch covers: an even share of the items plus the imbalance the dealing of
    // whole (sequence, head) pairs can leave (about one sequence's worth of tiles); longer lists,
    // possible only with sequences above max_seq_len, are walked by the workgroups' stride loop
    const size_t per_seq = (size_t)(max_seq_len + bm - 1) / bm;
    const size_t items_bm = ((size_t)((T + bm - 1) / bm) + (size_t)B) * (size_t)H;
    size_t slots = (items_bm + NUM_XCD - 1) / NUM_XCD + 2 * per_seq + 1;
    if (slots > items_bm) slots = items_bm;
    if (slots < 1) slots = 1;
    if (items > 0x7fffffffull || slots * NUM_XCD > 0x7fffffffull) return fail(RECIR_HSTU_ERR_UNSUPPORTED, "grid too large");
    p.grid_slots = (int)slots;
    if (!(flags & RECIR_HSTU_FLAG_REUSE_PLAN)) {
      if (B <= PLAN_MAX_B && (size_t)B * H <= PLAN_MAX_PAIRS)
        hipLaunchKernelGGL(hstu_plan_kernel, dim3(1), dim3(PLAN_THREADS), 0, stream, p, bm, plan_mode);
      else
        hipLaunchKernelGGL(hstu_plan_kernel_general, dim3(((size_t)B * H + 255) / 256), dim3(256), 0, stream, p, bm, plan_mode);
      if (int rc = launch_status("hstu_plan_kernel")) return rc;
    }
#ifdef HSTU_TRACE
    if (g_trace_buffer) {
      if (g_trace_words < items * NUM_XCD * 4 * TRACE_WORDS)
        return fail(RECIR_HSTU_ERR_WORKSPACE, "trace buffer of %zu words, %zu needed", g_trace_words, items * NUM_XCD * 4 * TRACE_WORDS);
      p.trace = g_trace_buffer;
    }
#endif
    const dim3 grid((unsigned)(slots * NUM_XCD));
    if (use_any) {
      if (!launch_mfma_any_fwd(dtype, any_dp, any_aligned, grid, stream, p))
        return fail(RECIR_HSTU_ERR_UNSUPPORTED, "no general MFMA kernel for dtype %d, padded head dim %d", dtype, any_dp);
      g_last_kernel = mfma_any_name(false, dtype, any_dp, any_aligned);
    } else if (fp8) {
      launch_dl<true>(rab != nullptr, semi, grid, stream, p);
      g_last_kernel = rab ? "tiled_d128_fp8qk_rab" : "tiled_d128_fp8qk";
    } else {
      launch_dl<false>(rab != nullptr, semi, grid, stream, p);
      g_last_kernel = rab ? "tiled_d128_bf16_rab" : "tiled_d128_bf16";
    }
    if (int rc = launch_status("hstu_fwd_tiled_d128")) return rc;
    return RECIR_HSTU_OK;
  }

  if (flags & RECIR_HSTU_FLAG_TILED_ONLY)
    return fail(RECIR_HSTU_ERR_UNSUPPORTED,
                "only the generic kernel covers this call (the MFMA kernels take head dims up to 256, fp32: 128): dtype=%d Dqk=%d "
                "Dv=%d", dtype, Dqk, Dv);
  if (Dqk > GENERIC_MAX_D || Dv > GENERIC_MAX_D)
    return fail(RECIR_HSTU_ERR_UNSUPPORTED, "head dims above %d are not supported (Dqk=%d Dv=%d)", GENERIC_MAX_D, Dqk, Dv);
  if (H > 65535) return fail(RECIR_HSTU_ERR_UNSUPPORTED, "more than 65535 heads");
  const dim3 grid((unsigned)T, (unsigned)H);
  if (dtype == RECIR_HSTU_DTYPE_BF16) hipLaunchKernelGGL(hstu_fwd_generic<ELT_BF16>, grid, dim3(64), 0, stream, p);
  else if (f16) hipLaunchKernelGGL(hstu_fwd_generic<ELT_FP16>, grid, dim3(64), 0, stream, p);
  else hipLaunchKernelGGL(hstu_fwd_generic<ELT_FP32>, grid, dim3(64), 0, stream, p);
  if (int rc = launch_status("hstu_fwd_generic")) return rc;
  g_last_kernel = dtype == RECIR_HSTU_DTYPE_BF16 ? "generic_bf16" : (f16 ? "generic_fp16" : "generic_fp32");
  return RECIR_HSTU_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------
// Forward entry point that allocates nothing: the work lists live in a device array of the
// library image instead of a caller-provided workspace.
// ---------------------------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[RECIR_HSTU_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int NOALLOC_MAX_DEVICES = 64;
// Device address of `scratch` on each GPU.  In host code the array's name is only a handle for the
// runtime; the address a kernel can use comes from hipGetSymbolAddress, once per device, with that
// device current (every GPU holds its own copy of the array at its own address).
std::atomic<void*> g_scratch_ptr[NOALLOC_MAX_DEVICES];
std::mutex g_scratch_mutex;

int scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail((int)e, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES)
    return fail(RECIR_HSTU_ERR_UNSUPPORTED, "device index %d outside the %d the library keeps scratch addresses for", dev,
                NOALLOC_MAX_DEVICES);
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!ptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!ptr) {
      e = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !ptr)
        return fail(e != hipSuccess ? (int)e : RECIR_HSTU_ERR_WORKSPACE, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                    hipGetErrorString(e));
      g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return 0;
}
// Largest magnitude of x[rows, H, D] (rows = min(seq_offsets[B], T)), per head into per_head[H] or over all
// heads into *all, as the bits of a float merged with an integer maximum (the bits of non-negative floats
// order like integers; a NaN's are above every finite value's).  A wave keeps one head and walks its share
// of the rows, so that it ends with one atomic.
template <int ELT>
__global__ __launch_bounds__(256) void hstu_rows_absmax(const void* x, unsigned* per_head, unsigned* all, int H, int D, const void* seq_end,
                                                        int i32, int T) {
  const long long e = i32 ? (long long)*(const int*)seq_end : *(const long long*)seq_end;
  const int rows = (int)(e < 0 ? 0 : (e > T ? T : e));
  const int lane = threadIdx.x & 63;
  const int wid = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6), nwaves = (int)((gridDim.x * blockDim.x) >> 6);
  const int slots = nwaves / H;  // (the launch has at least H waves)
  const int h = wid % H, slot = wid / H;
  if (slot >= slots) return;
  unsigned mx = 0;
  constexpr int U = 4;  // rows in flight per wave
  for (int r0 = slot; r0 < rows; r0 += slots * U) {
    for (int d = lane; d < D; d += 64) {
      float f[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int r = r0 + u * slots;
        f[u] = r < rows ? load_elem<ELT>(x, ((size_t)r * H + h) * D + d) : 0.f;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) mx = max(mx, __float_as_uint(f[u]) & 0x7fffffffu);
    }
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) mx = max(mx, (unsigned)__shfl_xor((int)mx, d, 64));
  if (lane == 0 && mx) atomicMax(per_head ? per_head + h : all, mx);
}
static void launch_rows_absmax(int dtype, const void* x, unsigned* per_head, unsigned* all, int H, int D, const void* seq_end, int i32,
                               int T, hipStream_t stream) {
  if (dtype == RECIR_HSTU_DTYPE_BF16 && D % 8 == 0 && ((size_t)x & 15) == 0) {
    // the quantiser's pass over 16-byte pieces; for the maximum over all heads a token's H rows count as one
    const int h_eff = per_head ? H : 1, d8 = per_head ? D / 8 : H * (D / 8);
    const size_t n8 = (size_t)T * H * (D / 8);
    const unsigned blocks = (unsigned)((n8 + 255) / 256 < 256 ? (n8 + 255) / 256 : 256);  // (each ends with h_eff global atomics)
    hipLaunchKernelGGL(hstu_quant_amax, dim3(blocks ? blocks : 1), dim3(256), 0, stream, (const u32x4*)x, per_head ? per_head : all, (unsigned*)nullptr, n8,
                       h_eff, d8, -1, (h_eff & (h_eff - 1)) == 0 ? h_eff - 1 : -1, seq_end, i32, T);
    return;
  }
  // 2048 waves or a multiple of H above that
  const unsigned waves = (unsigned)(((2048 + H - 1) / H) * H), blocks = (waves + 3) / 4;
  if (dtype == RECIR_HSTU_DTYPE_FP32) hipLaunchKernelGGL(hstu_rows_absmax<ELT_FP32>, dim3(blocks), dim3(256), 0, stream, x, per_head, all, H, D, seq_end, i32, T);
  else if (dtype == RECIR_HSTU_DTYPE_FP16) hipLaunchKernelGGL(hstu_rows_absmax<ELT_FP16>, dim3(blocks), dim3(256), 0, stream, x, per_head, all, H, D, seq_end, i32, T);
  else hipLaunchKernelGGL(hstu_rows_absmax<ELT_BF16>, dim3(blocks), dim3(256), 0, stream, x, per_head, all, H, D, seq_end, i32, T);
}

}  // namespace

extern "C" {

int recir_hstu_attn_fwd_noalloc(const void* q, const void* k, const void* v, void* out,
                                const void* seq_offsets, const void* num_targets, const float* rab,
                                const float* attn_scale, const float* q_scale, const float* k_scale,
                                int32_t T, int32_t B, int32_t H, int32_t Dqk, int32_t Dv,
                                int32_t max_seq_len, int32_t contextual_seq_len,
                                int32_t max_attn_len, int32_t full_attn_size, float alpha,
                                int32_t dtype, uint32_t flags, void* hip_stream) {
  if (flags & RECIR_HSTU_FLAG_REUSE_PLAN)
    return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT,
                "RECIR_HSTU_FLAG_REUSE_PLAN is not available without a caller-owned workspace: the built-in scratch is "
                "shared by every call on the GPU");
  const size_t need = recir_hstu_attn_fwd_workspace_bytes(T, B, H, Dqk, Dv, dtype);
  if (need > (size_t)RECIR_HSTU_NOALLOC_SCRATCH_BYTES)
    return fail(RECIR_HSTU_ERR_WORKSPACE,
                "work lists of %zu bytes (T=%d B=%d H=%d) exceed the built-in scratch of %zu bytes; use recir_hstu_attn_fwd "
                "with a workspace", need, T, B, H, (size_t)RECIR_HSTU_NOALLOC_SCRATCH_BYTES);
  void* ptr = nullptr;
  if (int rc = scratch_of_current_device(&ptr)) return rc;
  // The plan kernel writes every list length and every item the attention kernel reads, so
  // nothing left in the array by an earlier call is seen: no clearing needed.
  return recir_hstu_attn_fwd(q, k, v, out, seq_offsets, num_targets, rab, attn_scale, q_scale, k_scale, T, B, H, Dqk, Dv,
                             max_seq_len, contextual_seq_len, max_attn_len, full_attn_size, alpha, dtype, flags, ptr,
                             (size_t)RECIR_HSTU_NOALLOC_SCRATCH_BYTES, hip_stream);
}

constexpr size_t BWD_WS_TAIL = 256;  // behind the two lists: the largest |v| and |per-token scale| of the call (see drab)
size_t recir_hstu_attn_bwd_workspace_bytes(int32_t T, int32_t B, int32_t H, int32_t Dqk, int32_t Dv,
                                           int32_t dtype) {
  // two work lists: query tiles for dQ, key tiles for dK/dV
  return 2 * ((recir_hstu_attn_fwd_workspace_bytes(T, B, H, Dqk, Dv, dtype) + 255) & ~(size_t)255) + BWD_WS_TAIL;
}

// behind that, with drab: [H] largest |dout| per head, then the [H, 2N-1] fixed-point table
static size_t drab_head_words_bytes(int32_t H) { return (((size_t)H * 4) + 255) & ~(size_t)255; }
size_t recir_hstu_attn_bwd_rab_grad_workspace_bytes(int32_t H, int32_t max_seq_len) {
  if (H <= 0 || max_seq_len <= 0) return 0;
  return drab_head_words_bytes(H) + (size_t)H * (2 * (size_t)max_seq_len - 1) * sizeof(long long);
}

int recir_hstu_attn_bwd(const void* dout, const void* q, const void* k, const void* v, void* dq,
                        void* dk, void* dv, float* drab, const void* seq_offsets, const void* num_targets,
                        const float* rab, const float* attn_scale, int32_t T, int32_t B, int32_t H,
                        int32_t Dqk, int32_t Dv, int32_t max_seq_len, int32_t contextual_seq_len,
                        int32_t max_attn_len, int32_t full_attn_size, float alpha, int32_t dtype,
                        uint32_t flags, void* workspace, size_t workspace_bytes, void* hip_stream) {
  hipStream_t stream = (hipStream_t)hip_stream;
  if (T < 0 || B < 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "negative size: T=%d B=%d", T, B);
  if (max_attn_len < 0 || full_attn_size < 0)
    return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "max_attn_len and full_attn_size must be >= 0, got %d and %d",
                max_attn_len, full_attn_size);
  if (H <= 0 || Dqk <= 0 || Dv <= 0)
    return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "H, Dqk, Dv must be positive: H=%d Dqk=%d Dv=%d", H, Dqk, Dv);
  if (max_seq_len <= 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "max_seq_len must be positive, got %d", max_seq_len);
  if (contextual_seq_len < 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "contextual_seq_len must be >= 0, got %d", contextual_seq_len);
  if (dtype != RECIR_HSTU_DTYPE_BF16 && dtype != RECIR_HSTU_DTYPE_FP32 && dtype != RECIR_HSTU_DTYPE_FP16)
    return fail(dtype == RECIR_HSTU_DTYPE_FP8_E4M3 ? RECIR_HSTU_ERR_UNSUPPORTED : RECIR_HSTU_ERR_INVALID_ARGUMENT,
                "backward supports bf16, fp16 and fp32 tensors, got dtype %d", dtype);
  if (drab && !rab) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "drab (the gradient of rab) needs rab");
  // drab is written in full whatever follows: by the last kernel of the MFMA path, and on every other
  // path as zeros first, to which the generic kernel adds
  auto zero_drab = [&]() -> int {
    if (!drab) return 0;
    const size_t n = (size_t)H * (2 * (size_t)max_seq_len - 1);
    hipLaunchKernelGGL(hstu_fill_zero, dim3(64), dim3(256), 0, stream, (unsigned short*)drab, n * 2);
    return launch_status("hstu_fill_zero");
  };
  if (T == 0) return zero_drab();
  if (!dout || !q || !k || !v || !dq || !dk || !dv)
    return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "dout, q, k, v, dq, dk, dv must be non-null");
  if (!seq_offsets) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "seq_offsets must be non-null");

  BwdParams bp;
  memset(&bp, 0, sizeof(bp));
  Params& p = bp.f;
  p.q = q; p.k = k; p.v = v;
  p.seq_offsets = seq_offsets; p.num_targets = num_targets;
  p.rab = rab; p.attn_scale = attn_scale;
  p.T = T; p.B = B; p.H = H; p.Dqk = Dqk; p.Dv = Dv; p.N = max_seq_len; p.ctx = contextual_seq_len;
  p.alpha = alpha; p.flags = flags;
  p.max_attn_len = max_attn_len; p.full_attn_size = full_attn_size;
  const bool semi = max_attn_len > 0;
  bp.dout = dout; bp.dq = dq; bp.dk = dk; bp.dv = dv; bp.drab = drab; bp.absmax = nullptr;

  const bool bf16 = dtype == RECIR_HSTU_DTYPE_BF16;
  const size_t esz = dtype == RECIR_HSTU_DTYPE_FP32 ? 4 : 2;
  if (B == 0) {
    if (int rc = zero_drab()) return rc;
    void* outs[3] = {dq, dk, dv};
    const int dims[3] = {Dqk, Dqk, Dv};
    for (int i = 0; i < 3; ++i) {
      const size_t bytes = (size_t)T * H * dims[i] * esz;
      hipLaunchKernelGGL(hstu_fill_zero, dim3(1024), dim3(256), 0, stream, (unsigned short*)outs[i], bytes / 2);
      if (int rc = launch_status("hstu_fill_zero")) return rc;
    }
    g_last_kernel = "fill_zero";
    return RECIR_HSTU_OK;
  }
  if (Dqk > BWD_GENERIC_MAX_D || Dv > BWD_GENERIC_MAX_D)
    return fail(RECIR_HSTU_ERR_UNSUPPORTED, "head dims above %d are not supported (Dqk=%d Dv=%d)", BWD_GENERIC_MAX_D, Dqk, Dv);
  if ((unsigned)H > 65535u) return fail(RECIR_HSTU_ERR_UNSUPPORTED, "more than 65535 heads");
  const unsigned variant = (flags & RECIR_HSTU_FLAG_KERNEL_MASK) >> RECIR_HSTU_FLAG_KERNEL_SHIFT;
  const bool f16 = dtype == RECIR_HSTU_DTYPE_FP16;
  const bool noncausal = (flags & RECIR_HSTU_FLAG_MASK_NONCAUSAL) != 0;
  const bool aligned = (((size_t)dout | (size_t)q | (size_t)k | (size_t)v | (size_t)dq | (size_t)dk | (size_t)dv) & 15) == 0;
  // the kernels written for head dim 128 start their score accumulators from bias / alpha: a bias
  // with alpha = 0 (scores that are the bias alone) is not theirs, as in the forward
  const bool bias_needs_other = rab && !std::isnormal(1.0f / alpha);
  const bool d128_ok = bf16 && Dqk == HD && Dv == HD && aligned && !noncausal && !bias_needs_other;
  // the general MFMA kernels (hstu_mfma_any.h)
  const int any_dp = mfma_any_padded_dim(Dqk, Dv, dtype);
  const bool elem_aligned = (((size_t)dout | (size_t)q | (size_t)k | (size_t)v | (size_t)dq | (size_t)dk | (size_t)dv) & (esz - 1)) == 0;
  const bool any_ok = any_dp != 0 && elem_aligned;
  const bool any_aligned = aligned && rows_are_16_byte_multiples(Dqk, Dv, dtype);
  if (variant > 3) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "unknown kernel selector %u", variant);
  if (variant == 3 && !d128_ok)
    return fail(RECIR_HSTU_ERR_UNSUPPORTED,
                "the head-dim-128 backward needs bf16, Dqk = Dv = 128, 16-byte aligned tensors, the causal or semi-local mask "
                "and alpha != 0 with a bias");
  if (variant == 2 && !any_ok)
    return fail(RECIR_HSTU_ERR_UNSUPPORTED,
                "the general MFMA backward needs bf16, fp16 or fp32 and head dims up to 256 (fp32: 128)");
  const bool use_tiled = d128_ok && (variant == 0 || variant == 3);
  const bool use_any = !use_tiled && any_ok && variant != 1;
  if (use_tiled || use_any) {
    const size_t half_ws = (recir_hstu_attn_fwd_workspace_bytes(T, B, H, Dqk, Dv, dtype) + 255) & ~(size_t)255;
    if (!workspace || workspace_bytes < 2 * half_ws + BWD_WS_TAIL || ((size_t)workspace & 15))
      return fail(RECIR_HSTU_ERR_WORKSPACE, "workspace of %zu bytes (16-byte aligned) required, got %zu at %p",
                  2 * half_ws + BWD_WS_TAIL, workspace_bytes, workspace);
    const size_t items = max_items(T, B, H);
    const size_t per_seq = (size_t)(max_seq_len + BWD_BM - 1) / BWD_BM;
    const size_t items_bm = ((size_t)((T + BWD_BM - 1) / BWD_BM) + (size_t)B) * (size_t)H;
    size_t slots = (items_bm + NUM_XCD - 1) / NUM_XCD + 2 * per_seq + 1;
    if (slots > items_bm) slots = items_bm;
    if (slots < 1) slots = 1;
    if (items > 0x7fffffffull || slots * NUM_XCD > 0x7fffffffull) return fail(RECIR_HSTU_ERR_UNSUPPORTED, "grid too large");
    // two work lists: query tiles (heaviest = last tile of a sequence) and key tiles (heaviest = first)
    BwdParams bq = bp, bk = bp;
    bq.f.ws_counts = (int*)workspace;
    bq.f.ws_items = (WorkItem*)((char*)workspace + WS_HEADER);
    bk.f.ws_counts = (int*)((char*)workspace + half_ws);
    bk.f.ws_items = (WorkItem*)((char*)workspace + half_ws + WS_HEADER);
    bq.f.items_cap = bk.f.items_cap = (int)items;
    bq.f.grid_slots = (int)slots;
    // the key-tile kernel's workgroups (one per CU) stay and draw further items from the lists' counters
    const size_t kslots = slots < (size_t)BWD_DKV_WG_PER_XCD ? slots : (size_t)BWD_DKV_WG_PER_XCD;
    bk.f.grid_slots = (int)(use_any ? slots : kslots);
    if (!(flags & RECIR_HSTU_FLAG_REUSE_PLAN)) {
      if (B <= PLAN_MAX_B && (size_t)B * H <= PLAN_MAX_PAIRS) {
        // q, k, v, dout and the three gradients beyond the last-level cache: lists ordered by groups of pairs
        const int grp = ((flags & RECIR_HSTU_FLAG_GROUPED_LISTS) || tensors_exceed_llc(T, H, Dqk, Dv, 2, BWD_GROUP_TENSORS)) ? PLAN_GROUP : 0;
        hipLaunchKernelGGL(hstu_plan_pair_kernel, dim3(2), dim3(PLAN_THREADS), 0, stream, bq.f, PLAN_SHIFT_ODD | PLAN_PAIR_CU | grp, bk.f, PLAN_REVERSE | grp, BWD_BM);
        if (int rc = launch_status("hstu_plan_pair_kernel")) return rc;
      } else {
        for (int rev = 0; rev < 2; ++rev) {
          const Params& pp = rev ? bk.f : bq.f;
          hipLaunchKernelGGL(hstu_plan_kernel_general, dim3(((size_t)B * H + 255) / 256), dim3(256), 0, stream, pp, BWD_BM, rev ? PLAN_REVERSE : PLAN_SHIFT_ODD);
          if (int rc = launch_status("hstu_plan_kernel")) return rc;
        }
      }
    }
    const bool per_token = attn_scale && (flags & RECIR_HSTU_FLAG_SCALE_PER_TOKEN);
    if (use_any) {
      if (drab) {
        // The dQ pass sums dS along the diagonals as fixed-point integers (a band in LDS, a 64-bit table per
        // head), as the kernels written for head dim 128 do below; the maxima that give a head its scale
        // come from a pass over dout and one over v (any element type, any head dim).
        const size_t base = 2 * half_ws + BWD_WS_TAIL;
        const size_t need = base + recir_hstu_attn_bwd_rab_grad_workspace_bytes(H, max_seq_len);
        if (workspace_bytes < need)
          return fail(RECIR_HSTU_ERR_WORKSPACE,
                      "with drab the workspace must hold recir_hstu_attn_bwd_workspace_bytes + "
                      "recir_hstu_attn_bwd_rab_grad_workspace_bytes = %zu bytes, got %zu", need, workspace_bytes);
        unsigned* am = (unsigned*)((char*)workspace + 2 * half_ws);
        unsigned* dmax = (unsigned*)((char*)workspace + base);
        long long* tab = (long long*)((char*)workspace + base + drab_head_words_bytes(H));
        hipLaunchKernelGGL(hstu_drab_prepare, dim3(128), dim3(256), 0, stream, am, dmax, H, tab, (size_t)H * (2 * (size_t)max_seq_len - 1));
        if (int rc = launch_status("hstu_drab_prepare")) return rc;
        const int i32 = (flags & RECIR_HSTU_FLAG_OFFSETS_I32) ? 1 : 0;
        const void* seq_end = (const char*)seq_offsets + (size_t)B * (i32 ? 4 : 8);
        launch_rows_absmax(dtype, dout, dmax, nullptr, H, Dv, seq_end, i32, T, stream);
        launch_rows_absmax(dtype, v, nullptr, am + 1, H, Dv, seq_end, i32, T, stream);
        if (per_token) hipLaunchKernelGGL(hstu_scale_absmax, dim3(64), dim3(256), 0, stream, attn_scale, seq_end, i32, T, am + 2);
        if (int rc = launch_status("hstu_rows_absmax")) return rc;
        bq.absmax = bk.absmax = am;
        bq.dout_max = dmax;
        bq.drab_fx = tab;
      }
      const dim3 grid((unsigned)(slots * NUM_XCD));
      if (!launch_mfma_any_bwd(dtype, any_dp, any_aligned, grid, grid, stream, bq, bk))
        return fail(RECIR_HSTU_ERR_UNSUPPORTED, "no general MFMA backward for dtype %d, padded head dim %d", dtype, any_dp);
      if (int rc = launch_status("hstu_mfma_any (backward)")) return rc;
      if (drab) {
        hipLaunchKernelGGL(hstu_drab_finalize, dim3(256), dim3(256), 0, stream, bq, per_token ? 1 : 0);
        if (int rc = launch_status("hstu_drab_finalize")) return rc;
      }
      g_last_kernel = mfma_any_name(true, dtype, any_dp, any_aligned);
      return RECIR_HSTU_OK;
    }
    if (drab) {
      // The query-tile kernel sums dS along the diagonals as fixed-point integers, in LDS (float LDS
      // atomics run one lane at a time) and then in a 64-bit table per head (integer additions commute:
      // the gradient does not depend on the order of the workgroups).  The scale of a head comes from a
      // bound on |dS|: the head's largest |dout| (a pass over dout, here), the call's largest |v| (the
      // key-tile kernel, which runs first and holds every v row once, leaves it in word 1) and, with a
      // per-token output scale, its largest magnitude (word 2).
      const size_t base = 2 * half_ws + BWD_WS_TAIL;
      const size_t need = base + recir_hstu_attn_bwd_rab_grad_workspace_bytes(H, max_seq_len);
      if (workspace_bytes < need)
        return fail(RECIR_HSTU_ERR_WORKSPACE,
                    "with drab the workspace must hold recir_hstu_attn_bwd_workspace_bytes + "
                    "recir_hstu_attn_bwd_rab_grad_workspace_bytes = %zu bytes, got %zu", need, workspace_bytes);
      unsigned* am = (unsigned*)((char*)workspace + 2 * half_ws);
      unsigned* dmax = (unsigned*)((char*)workspace + base);
      long long* tab = (long long*)((char*)workspace + base + drab_head_words_bytes(H));
      const size_t tab_words = (size_t)H * (2 * (size_t)max_seq_len - 1);
      hipLaunchKernelGGL(hstu_drab_prepare, dim3(128), dim3(256), 0, stream, am, dmax, H, tab, tab_words);
      if (int rc = launch_status("hstu_drab_prepare")) return rc;
      const int i32 = (flags & RECIR_HSTU_FLAG_OFFSETS_I32) ? 1 : 0;
      const void* seq_end = (const char*)seq_offsets + (size_t)B * (i32 ? 4 : 8);
      const size_t n8 = (size_t)T * H * (HD / 8);
      const unsigned blocks = (unsigned)((n8 + 255) / 256 < 256 ? (n8 + 255) / 256 : 256);  // (each ends with H global atomics)
      const int h_mask = (H & (H - 1)) == 0 ? H - 1 : -1;
      hipLaunchKernelGGL(hstu_quant_amax, dim3(blocks), dim3(256), 0, stream, (const u32x4*)dout, dmax, (unsigned*)nullptr, n8, H, HD / 8, 4,
                         h_mask, seq_end, i32, T);
      if (per_token) hipLaunchKernelGGL(hstu_scale_absmax, dim3(64), dim3(256), 0, stream, attn_scale, seq_end, i32, T, am + 2);
      if (int rc = launch_status("hstu_quant_amax")) return rc;
      bq.absmax = bk.absmax = am;
      bq.dout_max = dmax;
      bq.drab_fx = tab;
    }
    const dim3 grid((unsigned)(slots * NUM_XCD)), grid_k((unsigned)(kslots * NUM_XCD));
    launch_bwd_tiled(semi, rab != nullptr, grid, grid_k, stream, bk, bq);
    if (int rc = launch_status("hstu_bwd_d128")) return rc;
    if (drab) {
      hipLaunchKernelGGL(hstu_drab_finalize, dim3(256), dim3(256), 0, stream, bq, per_token ? 1 : 0);
      if (int rc = launch_status("hstu_drab_finalize")) return rc;
    }
    g_last_kernel = rab ? "bwd_tiled_d128_bf16_rab" : "bwd_tiled_d128_bf16";
    return RECIR_HSTU_OK;
  }
  if (flags & RECIR_HSTU_FLAG_TILED_ONLY)
    return fail(RECIR_HSTU_ERR_UNSUPPORTED,
                "only the generic kernels cover this call (the MFMA kernels take head dims up to 256, fp32: 128): dtype=%d Dqk=%d "
                "Dv=%d", dtype, Dqk, Dv);
  if (int rc = zero_drab()) return rc;
  const dim3 grid((unsigned)T, (unsigned)H);
  if (bf16) {
    hipLaunchKernelGGL(hstu_bwd_generic_dq<ELT_BF16>, grid, dim3(64), 0, stream, bp);
    if (int rc = launch_status("hstu_bwd_generic_dq")) return rc;
    hipLaunchKernelGGL(hstu_bwd_generic_dkv<ELT_BF16>, grid, dim3(64), 0, stream, bp);
  } else if (f16) {
    hipLaunchKernelGGL(hstu_bwd_generic_dq<ELT_FP16>, grid, dim3(64), 0, stream, bp);
    if (int rc = launch_status("hstu_bwd_generic_dq")) return rc;
    hipLaunchKernelGGL(hstu_bwd_generic_dkv<ELT_FP16>, grid, dim3(64), 0, stream, bp);
  } else {
    hipLaunchKernelGGL(hstu_bwd_generic_dq<ELT_FP32>, grid, dim3(64), 0, stream, bp);
    if (int rc = launch_status("hstu_bwd_generic_dq")) return rc;
    hipLaunchKernelGGL(hstu_bwd_generic_dkv<ELT_FP32>, grid, dim3(64), 0, stream, bp);
  }
  if (int rc = launch_status("hstu_bwd_generic_dkv")) return rc;
  g_last_kernel = bf16 ? "bwd_generic_bf16" : (f16 ? "bwd_generic_fp16" : "bwd_generic_fp32");
  return RECIR_HSTU_OK;
}

#ifdef HSTU_TRACE
// Phase-trace builds only (a second library, never the one the operators load): device buffer that
// the next forward launches of the direct-to-LDS tiled kernel fill with one record of TRACE_WORDS
// 64-bit words per (XCD, list slot, wave); null switches the records off.
int recir_hstu_trace_buffer(void* device_words, size_t words) {
  g_trace_buffer = (unsigned long long*)device_words;
  g_trace_words = words;
  return RECIR_HSTU_OK;
}
int recir_hstu_trace_words_per_record(void) { return TRACE_WORDS; }
#endif

int recir_hstu_calibration_copy(void* dst, const void* src, size_t bytes, void* hip_stream) {
  if (!dst || !src || (bytes & 15) || (((size_t)dst | (size_t)src) & 15))
    return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "calibration copy needs 16-byte aligned pointers and size");
  if (bytes == 0) return RECIR_HSTU_OK;
  hipLaunchKernelGGL(hstu_calibration_copy, dim3(4096), dim3(256), 0, (hipStream_t)hip_stream, (u32x4*)dst,
                     (const u32x4*)src, bytes / 16);
  return launch_status("hstu_calibration_copy");
}

}  // extern "C"

namespace {
template <int KIND>
int launch_calibration(int pieces, unsigned grid, hipStream_t stream, const CalParams& c) {
  const dim3 g(grid), b(256);
  switch (pieces) {
    case 0: hipLaunchKernelGGL((hstu_calibration_loop<KIND, 0>), g, b, 0, stream, c); return 0;
    case CAL_NO_SILU: hipLaunchKernelGGL((hstu_calibration_loop<KIND, CAL_NO_SILU>), g, b, 0, stream, c); return 0;
    case CAL_NO_LDS_READS: hipLaunchKernelGGL((hstu_calibration_loop<KIND, CAL_NO_LDS_READS>), g, b, 0, stream, c); return 0;
    case CAL_NO_COPIES | CAL_NO_BARRIER:
      hipLaunchKernelGGL((hstu_calibration_loop<KIND, CAL_NO_COPIES | CAL_NO_BARRIER>), g, b, 0, stream, c); return 0;
    case CAL_NO_LDS_READS | CAL_NO_COPIES | CAL_NO_BARRIER:
      hipLaunchKernelGGL((hstu_calibration_loop<KIND, CAL_NO_LDS_READS | CAL_NO_COPIES | CAL_NO_BARRIER>), g, b, 0, stream, c); return 0;
    default: return -1;
  }
}
}  // namespace

extern "C" {

int recir_hstu_calibration_mfma_loop(int32_t kind, int32_t pieces, const void* k, const void* v, const void* q, size_t rows,
                                     int32_t sequences, int32_t tiles, int32_t workgroups, float alpha, uint64_t* stats,
                                     float* sink, void* hip_stream) {
  if (kind < 0 || kind > 3) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "calibration kind must be 0, 1, 2 or 3, got %d", kind);
  if (!k || !v || !q || !stats || !sink) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "calibration buffers must be non-null");
  if ((((size_t)k | (size_t)v | (size_t)q) & 15) || ((size_t)stats & 7))
    return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "calibration buffers must be 16-byte aligned");
  if (sequences <= 0 || workgroups <= 0 || tiles <= 0 || (tiles & 1))
    return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "sequences, workgroups and an even number of tiles must be positive");
  const size_t seq_tiles = rows / BN / (size_t)sequences;
  if (seq_tiles < 2 || rows < (size_t)BM) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "the buffers must hold at least two key tiles of 64 rows per sequence");
  if (seq_tiles > 0x7fffffffull) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "buffers too large");
  CalParams c;
  c.k = (const char*)k; c.v = (const char*)v; c.q = (const char*)q;
  c.sink = sink; c.stats = (unsigned long long*)stats;
  c.tiles = tiles; c.seq_tiles = (int)seq_tiles; c.sequences = sequences;
  c.neg_c = -alpha * kLog2e;
  hipStream_t stream = (hipStream_t)hip_stream;
  int rc = 0;
  if (kind == 0) {
    if (pieces != 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "the MFMA-only loop has no pieces to remove");
    hipLaunchKernelGGL((hstu_calibration_loop<0, 0>), dim3((unsigned)workgroups), dim3(256), 0, stream, c);
  } else if (kind == 1) {
    rc = launch_calibration<1>(pieces, (unsigned)workgroups, stream, c);
  } else if (kind == 2) {
    rc = launch_calibration<2>(pieces, (unsigned)workgroups, stream, c);
  } else {
    const dim3 g((unsigned)workgroups), b(256);
    if (pieces == 0) hipLaunchKernelGGL((hstu_calibration_loop64<0>), g, b, 0, stream, c);
    else if (pieces == CAL_NO_LDS_READS) hipLaunchKernelGGL((hstu_calibration_loop64<CAL_NO_LDS_READS>), g, b, 0, stream, c);
    else rc = -1;
  }
  if (rc) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "pieces %d is not one of the built combinations (0, 1, 2, 12, 14)", pieces);
  return launch_status("hstu_calibration_loop");
}

int recir_hstu_quantize_e4m3_per_head(const void* x_bf16, void* codes_u8, float* scale, int32_t T,
                                      int32_t H, int32_t D, void* hip_stream) {
  return recir_hstu_quantize_e4m3_per_head_rows(x_bf16, codes_u8, scale, T, H, D, nullptr, 0, 0, hip_stream);
}

int recir_hstu_quantize_e4m3_per_head_rows(const void* x_bf16, void* codes_u8, float* scale, int32_t T,
                                           int32_t H, int32_t D, const void* seq_offsets, int32_t B,
                                           uint32_t flags, void* hip_stream) {
  hipStream_t stream = (hipStream_t)hip_stream;
  if (B < 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "negative batch size %d", B);
  const int i32 = (flags & RECIR_HSTU_FLAG_OFFSETS_I32) ? 1 : 0;
  const void* seq_end = seq_offsets ? (const void*)((const char*)seq_offsets + (size_t)B * (i32 ? 4 : 8)) : nullptr;
  if (T < 0 || H <= 0 || D <= 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "bad sizes: T=%d H=%d D=%d", T, H, D);
  if (!scale) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "scale must be non-null");
  if (D % 8 != 0) return fail(RECIR_HSTU_ERR_UNSUPPORTED, "D must be a multiple of 8, got %d", D);
  if (T > 0 && (!x_bf16 || !codes_u8)) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "x and codes must be non-null");
  if ((((size_t)x_bf16) & 15) || (((size_t)codes_u8) & 7))
    return fail(RECIR_HSTU_ERR_UNSUPPORTED, "x must be 16-byte and codes 8-byte aligned");
  const size_t n8 = (size_t)T * H * (D / 8);
  const unsigned blocks = (unsigned)((n8 + 255) / 256 < 4096 ? (n8 + 255) / 256 : 4096);
  const unsigned amax_blocks = blocks < QUANT_AMAX_BLOCKS ? blocks : QUANT_AMAX_BLOCKS;  // each block ends with H global atomics on H addresses
  const int D8 = D / 8;
  int d8_shift = -1, h_mask = -1;
  if ((D8 & (D8 - 1)) == 0) { d8_shift = 0; while ((1 << d8_shift) < D8) ++d8_shift; }
  if ((H & (H - 1)) == 0) h_mask = H - 1;
  // the codes buffer doubles as the table of per-block maxima (it is written only afterwards)
  unsigned* partial = nullptr;
  if (H <= QUANT_LDS_HEADS && n8 > 0 && (size_t)T * H * D >= (size_t)amax_blocks * H * 4 && (((size_t)codes_u8) & 3) == 0)
    partial = (unsigned*)codes_u8;
  if (!partial) {
    hipLaunchKernelGGL(hstu_quant_clear, dim3(1), dim3(256), 0, stream, (unsigned*)scale, H);
    if (int rc = launch_status("hstu_quant_clear")) return rc;
  }
  if (n8 > 0) {
    hipLaunchKernelGGL(hstu_quant_amax, dim3(amax_blocks), dim3(256), 0, stream, (const u32x4*)x_bf16, (unsigned*)scale, partial, n8, H, D / 8, d8_shift, h_mask, seq_end, i32, T);
    if (int rc = launch_status("hstu_quant_amax")) return rc;
  }
  hipLaunchKernelGGL(hstu_quant_finalize, dim3(1), dim3(1024), 0, stream, scale, (const unsigned*)partial, (int)amax_blocks, H);
  if (int rc = launch_status("hstu_quant_finalize")) return rc;
  if (n8 > 0) {
    hipLaunchKernelGGL(hstu_quant_encode, dim3(blocks), dim3(256), 0, stream, (const u32x4*)x_bf16, (u32x2*)codes_u8, scale, n8, H, D / 8, d8_shift, h_mask, seq_end, i32, T);
    if (int rc = launch_status("hstu_quant_encode")) return rc;
  }
  return RECIR_HSTU_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------
// Jagged neighbours (row gathers)
// ---------------------------------------------------------------------------------------------
namespace {

// largest chunk (16, 4, 2, 1 bytes) that divides the row size and keeps every pointer aligned
int chunk_bytes(int64_t row_bytes, std::initializer_list<const void*> ptrs) {
  size_t bits = (size_t)row_bytes;
  for (const void* q : ptrs) bits |= (size_t)q;
  if ((bits & 15) == 0) return 16;
  if ((bits & 3) == 0) return 4;
  if ((bits & 1) == 0) return 2;
  return 1;
}

unsigned row_grid(long long chunks) {
  const long long blocks = (chunks + 255) / 256;
  return (unsigned)(blocks < 1 ? 1 : (blocks > 16384 ? 16384 : blocks));
}

int check_rows(int64_t row_bytes, int32_t B) {
  if (row_bytes <= 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "row_bytes must be positive, got %lld", (long long)row_bytes);
  if (B < 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "negative batch size %d", B);
  return 0;
}

// lanes per row group (log2): the smallest power of two that covers the chunks of a row, at most 64
static int group_log2(long long cpr) {
  int lg = 0;
  while (lg < 6 && (1ll << lg) < cpr) ++lg;
  return lg;
}
// blocks of four waves, one block of rows (JAG_ITERS iterations of 64 >> lg rows, at most 64 rows) per wave
static unsigned gather_grid(long long rows, int lg) {
  const long long rpi = 64 >> lg;
  const long long per_wave = rpi * JAG_ITERS < 64 ? rpi * JAG_ITERS : 64;
  long long blocks = ((rows + per_wave - 1) / per_wave + 3) / 4;
  if (blocks < 1) blocks = 1;
  if (blocks > 65536) blocks = 65536;
  return (unsigned)blocks;
}

#define RECIR_DISPATCH_CHUNK(cb, KERNEL, rows, stream, params, cpr)                                \
  do {                                                                                            \
    const int lg_ = group_log2(cpr);                                                              \
    const unsigned grid_ = gather_grid(rows, lg_);                                                \
    if (cb == 16) hipLaunchKernelGGL((KERNEL<uint4>), dim3(grid_), dim3(256), 0, stream, params, cpr, lg_);          \
    else if (cb == 4) hipLaunchKernelGGL((KERNEL<unsigned>), dim3(grid_), dim3(256), 0, stream, params, cpr, lg_);   \
    else if (cb == 2) hipLaunchKernelGGL((KERNEL<unsigned short>), dim3(grid_), dim3(256), 0, stream, params, cpr, lg_); \
    else hipLaunchKernelGGL((KERNEL<unsigned char>), dim3(grid_), dim3(256), 0, stream, params, cpr, lg_);           \
  } while (0)

}  // namespace

extern "C" {

int recir_jagged_to_padded_dense(const void* values, void* out, const void* offsets,
                                 int64_t total_rows, int32_t B, int32_t max_len, int64_t row_bytes,
                                 int32_t elem_bytes, uint64_t pad_bits, uint32_t flags,
                                 void* hip_stream) {
  using namespace recir_jagged;
  if (int rc = check_rows(row_bytes, B)) return rc;
  if (max_len < 0 || total_rows < 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "negative size");
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8)
    return fail(RECIR_HSTU_ERR_UNSUPPORTED, "padding element of %d bytes (1, 2, 4 or 8 supported)", elem_bytes);
  if (row_bytes % elem_bytes) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "row_bytes is not a multiple of elem_bytes");
  if (B == 0 || max_len == 0) return RECIR_HSTU_OK;
  if (!out || !offsets || (total_rows > 0 && !values)) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "null pointer");
  const int cb = chunk_bytes(row_bytes, {values, out});
  PadParams p{(const char*)values, (char*)out, {offsets, 0, (int)(flags & RECIR_HSTU_FLAG_OFFSETS_I32)},
              total_rows, B, max_len, pad_bits, elem_bytes};
  const long long cpr = row_bytes / cb;
  RECIR_DISPATCH_CHUNK(cb, jagged_to_padded_dense_kernel, (long long)B * max_len, (hipStream_t)hip_stream, p, cpr);
  return launch_status("jagged_to_padded_dense_kernel");
}

int recir_dense_to_jagged(const void* dense, void* out, const void* offsets, int64_t total_L,
                          int32_t B, int32_t N, int64_t row_bytes, uint32_t flags, void* hip_stream) {
  using namespace recir_jagged;
  if (int rc = check_rows(row_bytes, B)) return rc;
  if (N < 0 || total_L < 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "negative size");
  if (total_L == 0) return RECIR_HSTU_OK;
  if (!out) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "null pointer");
  if (B == 0 || N == 0) {  // nothing to gather from: zeros
    if (row_bytes & 1) return fail(RECIR_HSTU_ERR_UNSUPPORTED, "odd row size with an empty dense input");
    hipLaunchKernelGGL(hstu_fill_zero, dim3(1024), dim3(256), 0, (hipStream_t)hip_stream, (unsigned short*)out,
                       (size_t)(total_L * row_bytes) / 2);
    return launch_status("hstu_fill_zero");
  }
  if (!dense || !offsets) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "null pointer");
  const int cb = chunk_bytes(row_bytes, {dense, out});
  UnpadParams p{(const char*)dense, (char*)out, {offsets, 0, (int)(flags & RECIR_HSTU_FLAG_OFFSETS_I32)}, total_L, B, N};
  const long long cpr = row_bytes / cb;
  RECIR_DISPATCH_CHUNK(cb, dense_to_jagged_kernel, total_L, (hipStream_t)hip_stream, p, cpr);
  return launch_status("dense_to_jagged_kernel");
}

int recir_concat_2d_jagged(const void* values_a, const void* values_b, void* out,
                           const void* offsets_a, const void* offsets_b, int32_t B,
                           int32_t dense_len_a, int32_t dense_len_b, int64_t rows_a, int64_t rows_b,
                           int64_t row_bytes, int32_t is_replace, int32_t n_prefix_from_right,
                           uint32_t flags, void* hip_stream) {
  using namespace recir_jagged;
  if (int rc = check_rows(row_bytes, B)) return rc;
  // same argument rules as the reference (kjt_split_per_feature.cpp:108-121)
  if (!offsets_a && !offsets_b) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "at least one input must be jagged");
  if (n_prefix_from_right < 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "n_prefix_from_right must be non-negative, got %d", n_prefix_from_right);
  if (is_replace && n_prefix_from_right != 0)
    return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "n_prefix_from_right is not supported when is_replace is true");
  if (n_prefix_from_right != 0 && (!offsets_a || !offsets_b))
    return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "n_prefix_from_right is only supported for two jagged inputs");
  if (rows_a < 0 || rows_b < 0 || dense_len_a < 0 || dense_len_b < 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "negative size");
  const long long out_rows = is_replace ? rows_a : rows_a + rows_b;
  if (out_rows == 0 || B == 0) return RECIR_HSTU_OK;
  if (!out || (rows_a > 0 && !values_a) || (rows_b > 0 && !values_b)) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "null pointer");
  const int i32 = (int)(flags & RECIR_HSTU_FLAG_OFFSETS_I32);
  const int cb = chunk_bytes(row_bytes, {values_a, values_b, out});
  ConcatParams p{(const char*)values_a, (const char*)values_b, (char*)out, {offsets_a, dense_len_a, i32},
                 {offsets_b, dense_len_b, i32}, rows_a, rows_b, out_rows, B, is_replace, n_prefix_from_right};
  const long long cpr = row_bytes / cb;
  RECIR_DISPATCH_CHUNK(cb, concat_2d_jagged_kernel, out_rows, (hipStream_t)hip_stream, p, cpr);
  return launch_status("concat_2d_jagged_kernel");
}

int recir_split_2d_jagged(const void* values, void* out_a, void* out_b, const void* offsets_a,
                          const void* offsets_b, int32_t B, int32_t dense_len_a, int32_t dense_len_b,
                          int64_t rows_a, int64_t rows_b, int64_t row_bytes,
                          int32_t n_prefix_to_right, uint32_t flags, void* hip_stream) {
  using namespace recir_jagged;
  if (int rc = check_rows(row_bytes, B)) return rc;
  if (n_prefix_to_right < 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "n_prefix_to_right must be non-negative, got %d", n_prefix_to_right);
  if (rows_a < 0 || rows_b < 0 || dense_len_a < 0 || dense_len_b < 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "negative size");
  if (rows_a + rows_b == 0 || B == 0) return RECIR_HSTU_OK;
  if (!values || (rows_a > 0 && !out_a) || (rows_b > 0 && !out_b)) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "null pointer");
  const int i32 = (int)(flags & RECIR_HSTU_FLAG_OFFSETS_I32);
  const int cb = chunk_bytes(row_bytes, {values, out_a, out_b});
  SplitParams p{(const char*)values, (char*)out_a, (char*)out_b, {offsets_a, dense_len_a, i32},
                {offsets_b, dense_len_b, i32}, rows_a, rows_b, rows_a + rows_b, B, n_prefix_to_right};
  const long long cpr = row_bytes / cb;
  RECIR_DISPATCH_CHUNK(cb, split_2d_jagged_kernel, rows_a + rows_b, (hipStream_t)hip_stream, p, cpr);
  return launch_status("split_2d_jagged_kernel");
}

}  // extern "C"

namespace {
size_t sort_temp_bytes(int64_t L) {
  size_t bytes = 0;
  (void)rocprim::radix_sort_pairs(nullptr, bytes, (const int*)nullptr, (int*)nullptr, (const int*)nullptr, (int*)nullptr,
                                  (size_t)(L > 0 ? L : 1), 0, 12);
  return bytes;
}
size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
}  // namespace

extern "C" {

// chunks (one per wave) and tokens per chunk of the counting sort
static void csort_chunks(int64_t L, int& NW, int& CW) {
#ifndef CSORT_CHUNK
#define CSORT_CHUNK 512
#endif
  long long nw = (L + CSORT_CHUNK - 1) / CSORT_CHUNK;
  nw = nw < 1 ? 1 : (nw > recir_jagged::CSORT_MAX_CHUNKS ? recir_jagged::CSORT_MAX_CHUNKS : nw);
  long long cw = ((L + nw - 1) / nw + 63) / 64 * 64;
  if (cw < 64) cw = 64;
  CW = (int)cw;
  NW = (int)((L + cw - 1) / cw);
  if (NW < 1) NW = 1;
}
static int bucket_keys(int32_t TS) { return TS < 2049 ? TS : 2049; }

size_t recir_add_timestamp_position_embeddings_workspace_bytes(int64_t L, int32_t P, int32_t TS) {
  if (L < 0 || P < 0 || TS < 0) return 0;
  // unsorted position rows, unsorted buckets, identity permutation, sort scratch (the larger of the
  // counting sort's tables and the general sort's)
  size_t scratch = sort_temp_bytes(L);
  if (P <= recir_jagged::CSORT_MAX_K) {
    int NW, CW;
    csort_chunks(L, NW, CW);
    const size_t keys = (size_t)P + (size_t)bucket_keys(TS);
    const size_t tables = align256((size_t)NW * keys * 4) + align256(keys * 4) + 512;
    if (tables > scratch) scratch = tables;
  }
  return 3 * align256((size_t)L * 4) + align256(scratch);
}

int recir_add_timestamp_position_embeddings(
    const void* seq, void* out, const void* seq_offsets, const void* pos_emb, const void* ts_emb,
    const void* timestamps, const void* seq_lengths, const void* num_targets, int32_t* sorted_pos,
    int32_t* pos_order, int32_t* sorted_ts, int32_t* ts_order, int64_t L, int32_t B, int32_t D,
    int32_t P, int32_t TS, int32_t Tmax, int32_t max_contextual_seq_len, int32_t interleave_targets,
    int32_t time_bucket_log, int32_t seq_dtype, int32_t table_dtype, int32_t timestamps_float,
    uint32_t flags, void* workspace, size_t workspace_bytes, void* hip_stream) {
  using namespace recir_jagged;
  hipStream_t stream = (hipStream_t)hip_stream;
  if (L < 0 || B < 0 || D <= 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "bad sizes: L=%lld B=%d D=%d", (long long)L, B, D);
  if (L > 0x7fffffffll) return fail(RECIR_HSTU_ERR_UNSUPPORTED, "more than 2^31 - 1 tokens");
  // same shape rules as the reference (kjt_split_per_feature.cpp:320-347)
  if (TS < 2049) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "timestamp embeddings must contain 2049 buckets, got %d", TS);
  if (P <= 0 || Tmax <= 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "position table and timestamps must be non-empty");
  if (max_contextual_seq_len < 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "max_contextual_seq_len must be >= 0");
  for (int dt : {seq_dtype, table_dtype})
    if (dt != RECIR_HSTU_DTYPE_BF16 && dt != RECIR_HSTU_DTYPE_FP32)
      return fail(RECIR_HSTU_ERR_UNSUPPORTED, "embeddings must be bf16 or fp32, got dtype %d", dt);
  if (L == 0) return RECIR_HSTU_OK;
  if (B == 0) return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "tokens without sequences");
  if (!seq || !out || !seq_offsets || !pos_emb || !ts_emb || !timestamps || !seq_lengths || !sorted_pos || !pos_order ||
      !sorted_ts || !ts_order)
    return fail(RECIR_HSTU_ERR_INVALID_ARGUMENT, "null pointer");
  const size_t need = recir_add_timestamp_position_embeddings_workspace_bytes(L, P, TS);
  if (!workspace || workspace_bytes < need || ((size_t)workspace & 255))
    return fail(RECIR_HSTU_ERR_WORKSPACE, "workspace of %zu bytes (256-byte aligned) required, got %zu at %p", need,
                workspace_bytes, workspace);
  const size_t seg = align256((size_t)L * 4);
  TsPosParams p;
  memset(&p, 0, sizeof(p));
  p.seq = seq; p.out = out; p.offsets = seq_offsets; p.pos_emb = pos_emb; p.ts_emb = ts_emb;
  p.timestamps = timestamps; p.seq_lengths = seq_lengths; p.num_targets = num_targets;
  p.pos_idx = (int*)workspace; p.ts_idx = (int*)((char*)workspace + seg); p.iota = (int*)((char*)workspace + 2 * seg);
  p.L = L; p.B = B; p.D = D; p.P = P; p.TS = TS; p.Tmax = Tmax; p.max_ctx = max_contextual_seq_len;
  p.interleave = interleave_targets != 0; p.use_log = time_bucket_log != 0;
  p.seq_bf16 = seq_dtype == RECIR_HSTU_DTYPE_BF16; p.tab_bf16 = table_dtype == RECIR_HSTU_DTYPE_BF16;
  p.ts_is_float = timestamps_float != 0; p.i32 = (int)(flags & RECIR_HSTU_FLAG_OFFSETS_I32);
  {
    // elements per lane and access: 8 (both types two bytes wide) or 4 when the row length and the
    // alignment of all four tensors allow 16-byte accesses, else 1
    const bool aligned = ((((size_t)seq | (size_t)out | (size_t)pos_emb | (size_t)ts_emb) & 15) == 0);
    const int wide = (p.seq_bf16 && p.tab_bf16) ? 8 : 4;
    const int E = (aligned && D % wide == 0) ? wide : 1;
    const int lg = group_log2(D / E);
    const long long rpi = 64 >> lg;
    const long long per_wave = rpi * 8 < 64 ? rpi * 8 : 64;
    long long blocks = ((L + per_wave - 1) / per_wave + 3) / 4;
    if (blocks > 65536) blocks = 65536;
    const dim3 grid((unsigned)blocks), block(256);
#define RECIR_TS_POS_LAUNCH(EE)                                                                              \
    do {                                                                                                     \
      if (p.seq_bf16 && p.tab_bf16) hipLaunchKernelGGL((ts_pos_embeddings_kernel<EE, true, true>), grid, block, 0, stream, p, lg);   \
      else if (p.seq_bf16) hipLaunchKernelGGL((ts_pos_embeddings_kernel<EE, true, false>), grid, block, 0, stream, p, lg);           \
      else if (p.tab_bf16) hipLaunchKernelGGL((ts_pos_embeddings_kernel<EE, false, true>), grid, block, 0, stream, p, lg);           \
      else hipLaunchKernelGGL((ts_pos_embeddings_kernel<EE, false, false>), grid, block, 0, stream, p, lg);                         \
    } while (0)
    if (E == 8) RECIR_TS_POS_LAUNCH(8);
    else if (E == 4) RECIR_TS_POS_LAUNCH(4);
    else RECIR_TS_POS_LAUNCH(1);
#undef RECIR_TS_POS_LAUNCH
  }
  if (int rc = launch_status("ts_pos_embeddings_kernel")) return rc;
  void* temp = (char*)workspace + 3 * seg;
  if (P <= CSORT_MAX_K) {
    // both lists in three launches (stable counting sort: position rows < P, buckets <= 2048)
    CsortParams c;
    memset(&c, 0, sizeof(c));
    csort_chunks(L, c.NW, c.CW);
    c.L = L;
    const int kp = P, kt = bucket_keys(TS);
    c.kmax = kp > kt ? kp : kt;
    char* t = (char*)temp;
    int* counts = (int*)t;
    t += align256((size_t)c.NW * ((size_t)kp + kt) * 4);
    int* starts = (int*)t;
    auto bits_of = [](int k) { int b = 0; while ((1 << b) < k) ++b; return b; };
    c.list[0] = {p.pos_idx, sorted_pos, pos_order, counts, starts, kp, bits_of(kp)};
    c.list[1] = {p.ts_idx, sorted_ts, ts_order, counts + (size_t)c.NW * kp, starts + kp, kt, bits_of(kt)};
    // LDS: one histogram per wave, and in the scatter kernel one more table for the block
    int wpb = 65536 / (c.kmax * 4) - 1;
    wpb = wpb < 1 ? 1 : (wpb > 4 ? 4 : wpb);
    const dim3 grid((unsigned)((c.NW + wpb - 1) / wpb), 2), block((unsigned)(wpb * 64));
    hipLaunchKernelGGL(csort_count, grid, block, (size_t)wpb * c.kmax * 4, stream, c);
    if (int rc = launch_status("csort_count")) return rc;
    hipLaunchKernelGGL(csort_scan, dim3((unsigned)((c.kmax + 255) / 256), 2), dim3(256), 0, stream, c);
    if (int rc = launch_status("csort_scan")) return rc;
    hipLaunchKernelGGL(csort_scatter, grid, block, (size_t)(wpb + 1) * c.kmax * 4, stream, c);
    if (int rc = launch_status("csort_scatter")) return rc;
    return RECIR_HSTU_OK;
  }
  size_t temp_bytes = sort_temp_bytes(L);
  // position rows fit 31 bits, buckets 12 (0..2048)
  hipError_t e = rocprim::radix_sort_pairs(temp, temp_bytes, (const int*)p.pos_idx, (int*)sorted_pos, (const int*)p.iota,
                                           (int*)pos_order, (size_t)L, 0, 31, stream);
  if (e != hipSuccess) return fail((int)e, "sort of the position rows: %s", hipGetErrorString(e));
  e = rocprim::radix_sort_pairs(temp, temp_bytes, (const int*)p.ts_idx, (int*)sorted_ts, (const int*)p.iota, (int*)ts_order,
                                (size_t)L, 0, 12, stream);
  if (e != hipSuccess) return fail((int)e, "sort of the timestamp buckets: %s", hipGetErrorString(e));
  return RECIR_HSTU_OK;
}

}  // extern "C"
