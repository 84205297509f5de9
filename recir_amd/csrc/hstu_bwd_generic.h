// Generic backward kernels of the HSTU attention: any head dim up to 512, fp32 or bf16 tensors,
// fp32 arithmetic, one wave per (token, head).  They cover what the tiled MFMA kernels do not
// (fp32, other head dims, score bias, per-token output scale).
//
// Gradient formulas (recir/ops/helion/jagged_hstu_attention.py:16-27), per head and sequence:
//   S = alpha Q K^T (+ rab)     P = silu(S) scale keep        O = P V
//   dP = dO V^T                 dV = P^T dO
//   dS = dP keep scale silu'(S), silu'(x) = sig(x) (1 + x (1 - sig(x)))
//   dQ = alpha dS K             dK = alpha dS^T Q
// Two kernels, as in the reference (dQ walks the keys of a query row, dK/dV walk the queries of a
// key row), so that every output row has exactly one writer and no atomics are needed.
#pragma once
#include "hstu_common.h"

namespace recir_hstu {

constexpr int BWD_GENERIC_MAX_D = 512;

// (b, m) of packed row r, or b = -1 when r belongs to no sequence
__device__ __forceinline__ int find_sequence(const Params& p, int r, SeqInfo& si) {
  const bool i32 = p.flags & RECIR_HSTU_FLAG_OFFSETS_I32;
  int lo = 0, hi = p.B + 1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (load_index(p.seq_offsets, mid, i32) > (long long)r) hi = mid; else lo = mid + 1;
  }
  const int b = lo - 1;
  if (b < 0 || b >= p.B) return -1;
  si = seq_info(p, b);
  if (r < si.s || r >= si.s + si.n) return -1;
  return b;
}

__device__ __forceinline__ float score_bias(const Params& p, int h, int m, int j) {
  if (!p.rab) return 0.f;
  const int rab_w = 2 * p.N - 1;
  // a pair outside the table (possible only in a sequence longer than max_seq_len) has no bias
  const int idx = m - j + p.N - 1;
  return (idx >= 0 && idx < rab_w) ? p.rab[(size_t)h * rab_w + idx] : 0.f;
}

// dQ[r] = alpha * sum_j dS(m, j) K[j]
template <int ELT>
__global__ __launch_bounds__(64) void hstu_bwd_generic_dq(BwdParams bp) {
  const Params& p = bp.f;
  __shared__ float qrow[BWD_GENERIC_MAX_D];
  __shared__ float grow[BWD_GENERIC_MAX_D];
  __shared__ float dsbuf[64];
  const int lane = threadIdx.x;
  const int r = blockIdx.x, h = blockIdx.y;
  const size_t esz = ELT == ELT_FP32 ? 4 : 2;
  zero_tail_rows_of<64>(p, bp.dq, (size_t)p.H * p.Dqk * esz);
  if (r >= end_of_sequences(p)) return;
  SeqInfo si = {0, 0, 0, 0};
  const size_t qoff = ((size_t)r * p.H + h) * p.Dqk;
  const size_t goff = ((size_t)r * p.H + h) * p.Dv;
  if (find_sequence(p, r, si) < 0) {  // only reachable with malformed offsets
    for (int d = lane; d < p.Dqk; d += 64) store_elem<ELT>(bp.dq, qoff + d, 0.f);
    return;
  }
  const int m = r - si.s;
  for (int d = lane; d < p.Dqk; d += 64) qrow[d] = load_elem<ELT>(p.q, qoff + d);
  for (int d = lane; d < p.Dv; d += 64) grow[d] = load_elem<ELT>(bp.dout, goff + d);
  __syncthreads();
  float scale = 1.0f / (float)p.N;
  if (p.attn_scale) scale = (p.flags & RECIR_HSTU_FLAG_SCALE_PER_TOKEN) ? p.attn_scale[r] : p.attn_scale[0];

  float acc[BWD_GENERIC_MAX_D / 64];
#pragma unroll
  for (int i = 0; i < BWD_GENERIC_MAX_D / 64; ++i) acc[i] = 0.f;
  const bool noncausal = p.flags & RECIR_HSTU_FLAG_MASK_NONCAUSAL;  // then keys after the query count too
  const int jend = noncausal ? si.n : max(m + 1, si.ctx_eff);
  for (int j0 = 0; j0 < jend; j0 += 64) {
    const int j = j0 + lane;
    float ds = 0.f;
    if (j < si.n && keep_pair(m, j, si, noncausal)) {
      const size_t krow = ((size_t)(si.s + j) * p.H + h) * p.Dqk;
      const size_t vrow = ((size_t)(si.s + j) * p.H + h) * p.Dv;
      float dot = 0.f, dp = 0.f;
      for (int d = 0; d < p.Dqk; ++d) dot = fmaf(qrow[d], load_elem<ELT>(p.k, krow + d), dot);
      for (int d = 0; d < p.Dv; ++d) dp = fmaf(grow[d], load_elem<ELT>(p.v, vrow + d), dp);
      const float x = dot * p.alpha + score_bias(p, h, m, j);
      const float sig = 1.0f / (1.0f + __expf(-x));
      ds = dp * scale * sig * (1.0f + x * (1.0f - sig));
      if (bp.drab) {  // d score / d rab = 1: the pair's dS goes to its diagonal's column
        const int rab_w = 2 * p.N - 1, idx = m - j + p.N - 1;
        if (idx >= 0 && idx < rab_w) unsafeAtomicAdd(&bp.drab[(size_t)h * rab_w + idx], ds);
      }
    }
    __syncthreads();
    dsbuf[lane] = ds;
    __syncthreads();
    const int cnt = min(64, si.n - j0);
    for (int jj = 0; jj < cnt; ++jj) {
      const float w = dsbuf[jj];
      if (w == 0.f) continue;
      const size_t krow = ((size_t)(si.s + j0 + jj) * p.H + h) * p.Dqk;
#pragma unroll
      for (int i = 0; i < BWD_GENERIC_MAX_D / 64; ++i) {
        const int d = lane + 64 * i;
        if (d < p.Dqk) acc[i] = fmaf(w, load_elem<ELT>(p.k, krow + d), acc[i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < BWD_GENERIC_MAX_D / 64; ++i) {
    const int d = lane + 64 * i;
    if (d < p.Dqk) store_elem<ELT>(bp.dq, qoff + d, acc[i] * p.alpha);
  }
}

// dK[r] = alpha * sum_m dS(m, j) Q[m],  dV[r] = sum_m P(m, j) dO[m]   for key row j = r - s
template <int ELT>
__global__ __launch_bounds__(64) void hstu_bwd_generic_dkv(BwdParams bp) {
  const Params& p = bp.f;
  __shared__ float krow_s[BWD_GENERIC_MAX_D];
  __shared__ float vrow_s[BWD_GENERIC_MAX_D];
  __shared__ float pbuf[64];
  __shared__ float dsbuf[64];
  const int lane = threadIdx.x;
  const int r = blockIdx.x, h = blockIdx.y;
  const size_t esz = ELT == ELT_FP32 ? 4 : 2;
  zero_tail_rows_of<64>(p, bp.dk, (size_t)p.H * p.Dqk * esz);
  zero_tail_rows_of<64>(p, bp.dv, (size_t)p.H * p.Dv * esz);
  if (r >= end_of_sequences(p)) return;
  SeqInfo si = {0, 0, 0, 0};
  const size_t koff = ((size_t)r * p.H + h) * p.Dqk;
  const size_t voff = ((size_t)r * p.H + h) * p.Dv;
  if (find_sequence(p, r, si) < 0) {
    for (int d = lane; d < p.Dqk; d += 64) store_elem<ELT>(bp.dk, koff + d, 0.f);
    for (int d = lane; d < p.Dv; d += 64) store_elem<ELT>(bp.dv, voff + d, 0.f);
    return;
  }
  const int j = r - si.s;
  for (int d = lane; d < p.Dqk; d += 64) krow_s[d] = load_elem<ELT>(p.k, koff + d);
  for (int d = lane; d < p.Dv; d += 64) vrow_s[d] = load_elem<ELT>(p.v, voff + d);
  __syncthreads();

  float acck[BWD_GENERIC_MAX_D / 64], accv[BWD_GENERIC_MAX_D / 64];
#pragma unroll
  for (int i = 0; i < BWD_GENERIC_MAX_D / 64; ++i) acck[i] = accv[i] = 0.f;
  // queries that see key j: all of them for a contextual key, m >= j for a history key, m == j else
  // (every query is tried under a mask type other than the causal one)
  const bool noncausal = p.flags & RECIR_HSTU_FLAG_MASK_NONCAUSAL;
  const bool ctx_key = j < si.ctx_eff || noncausal;
  const int mbeg = ctx_key ? 0 : j;
  const int mend = (ctx_key || j < si.cap) ? si.n : j + 1;
  for (int m0 = mbeg; m0 < mend; m0 += 64) {
    const int m = m0 + lane;
    float pw = 0.f, ds = 0.f;
    if (m < mend && keep_pair(m, j, si, noncausal)) {
      const size_t qrow = ((size_t)(si.s + m) * p.H + h) * p.Dqk;
      const size_t grow = ((size_t)(si.s + m) * p.H + h) * p.Dv;
      float dot = 0.f, dp = 0.f;
      for (int d = 0; d < p.Dqk; ++d) dot = fmaf(krow_s[d], load_elem<ELT>(p.q, qrow + d), dot);
      for (int d = 0; d < p.Dv; ++d) dp = fmaf(vrow_s[d], load_elem<ELT>(bp.dout, grow + d), dp);
      float scale = 1.0f / (float)p.N;
      if (p.attn_scale) scale = (p.flags & RECIR_HSTU_FLAG_SCALE_PER_TOKEN) ? p.attn_scale[si.s + m] : p.attn_scale[0];
      const float x = dot * p.alpha + score_bias(p, h, m, j);
      const float sig = 1.0f / (1.0f + __expf(-x));
      pw = x * sig * scale;
      ds = dp * scale * sig * (1.0f + x * (1.0f - sig));
    }
    __syncthreads();
    pbuf[lane] = pw;
    dsbuf[lane] = ds;
    __syncthreads();
    const int cnt = min(64, mend - m0);
    for (int mm = 0; mm < cnt; ++mm) {
      const float w = pbuf[mm], u = dsbuf[mm];
      if (w == 0.f && u == 0.f) continue;
      const size_t qrow = ((size_t)(si.s + m0 + mm) * p.H + h) * p.Dqk;
      const size_t grow = ((size_t)(si.s + m0 + mm) * p.H + h) * p.Dv;
#pragma unroll
      for (int i = 0; i < BWD_GENERIC_MAX_D / 64; ++i) {
        const int d = lane + 64 * i;
        if (d < p.Dqk) acck[i] = fmaf(u, load_elem<ELT>(p.q, qrow + d), acck[i]);
        if (d < p.Dv) accv[i] = fmaf(w, load_elem<ELT>(bp.dout, grow + d), accv[i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < BWD_GENERIC_MAX_D / 64; ++i) {
    const int d = lane + 64 * i;
    if (d < p.Dqk) store_elem<ELT>(bp.dk, koff + d, acck[i] * p.alpha);
    if (d < p.Dv) store_elem<ELT>(bp.dv, voff + d, accv[i]);
  }
}

}  // namespace recir_hstu
