// Tiled MFMA kernel of the HSTU attention forward, head dim 128 (qk and v), bf16 values.
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
// Pipeline: the K/V rows of tile i+1 are fetched from global memory into registers before the
// contractions of tile i start and are written to the other LDS buffer after them, so one barrier
// per tile suffices and the global latency hides behind the MFMA work.
//
// LDS tiles are XOR-swizzled in 16-byte chunks instead of padded:
//   Ks [BN][128]  chunk' = chunk ^ (row & 7)
//   Vts[128][BN]  chunk' = chunk ^ ((d ^ (d >> 3)) & 7), key order inside a 16-key group permuted
//                 to match the accumulator layout (kv = 16 g + 8 a + 4 half + c  ->  16 g + 8 half + 4 a + c)
#pragma once
#include <type_traits>

#include "hstu_common.h"

namespace recir_hstu {

constexpr int BM = 128;
constexpr int BN = 64;
constexpr int HD = 128;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ int vt_swz(int d) { return (d ^ (d >> 3)) & 7; }

// One thread's share of a staged K/V tile (kept as named members, not arrays, so that it lives in
// registers whatever the control flow around it looks like).


struct TileRegs {
  u32x4 k0, k1, k2, k3;
  u32x4 v0, v1, v2, v3;
  float rab;
};

template <bool HAS_RAB>
__global__ __launch_bounds__(256, 2) void hstu_fwd_tiled_d128(Params p) {
  __shared__ __attribute__((aligned(16))) unsigned short Ks[2][BN * HD];
  __shared__ __attribute__((aligned(16))) unsigned short Vts[2][HD * BN];
  __shared__ float rabs[2][HAS_RAB ? (BM + BN) : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int half = lane >> 5;

  zero_tail_rows<256>(p, (size_t)p.H * HD * 2);

  // Work list of the XCD this workgroup runs on.  Normally one item per workgroup; the stride loop
  // only matters when a list is longer than the launch assumed (sequences above max_seq_len).
  const int xcd = blockIdx.x % NUM_XCD;
  const int list_len = p.ws_counts[xcd];
  const WorkItem* __restrict__ list = p.ws_items + (size_t)xcd * p.items_cap;
  for (int slot = blockIdx.x / NUM_XCD; slot < list_len; slot += p.grid_slots) {
  const WorkItem wi = list[slot];
  SeqInfo si;
  si.s = wi.s; si.n = wi.n; si.cap = wi.cap; si.ctx_eff = wi.ctx_eff;
  const int q0 = wi.q0;
  const int h = wi.h;

  const size_t row_stride = (size_t)p.H * HD;
  const unsigned short* __restrict__ kg = (const unsigned short*)p.k + (size_t)si.s * row_stride + (size_t)h * HD;
  const unsigned short* __restrict__ vg = (const unsigned short*)p.v + (size_t)si.s * row_stride + (size_t)h * HD;
  const int rab_w = 2 * p.N - 1;
  const float* __restrict__ rabg = HAS_RAB ? p.rab + (size_t)h * rab_w : nullptr;

  // ---- Q fragments (B operand): lane holds row qw0 + l32, d = 16 kk + 8 half .. +7 ----
  // q enters the products as stored (no rescaling, hence no rounding of its own): the score
  // accumulator holds S' = q . k, S' sigmoid(alpha S') is accumulated and alpha goes into the output scale.
  const int qw0 = q0 + wave * 32;
  const int m = qw0 + l32;
  bf16x8 qf[8];
  {
    const bool valid = m < si.n;
    const unsigned short* qrow = (const unsigned short*)p.q + ((size_t)(si.s + (valid ? m : 0)) * p.H + h) * HD;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const u32x4 zero4 = {0u, 0u, 0u, 0u};
      const u32x4 t = valid ? *(const u32x4*)(qrow + kk * 16 + half * 8) : zero4;
      qf[kk] = __builtin_bit_cast(bf16x8, t);
    }
  }
  // accumulator value S' = q . k (+ bias / alpha); sigmoid(alpha S') = 1 / (1 + exp2(neg_c S'))
  const float neg_c = -(p.alpha * kLog2e);
  const float bias_mul = HAS_RAB ? 1.0f / p.alpha : 0.f;

  f32x16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;


  const int m_lo = qw0;
  const int m_hi = min(qw0 + 31, si.n - 1);
  const bool wave_has_rows = m_lo < si.n;

  // key tiles [0, nkv) minus the run [skip_a, skip_b) that holds only target keys off this query
  // tile's diagonal (and no contextual key)
  const int kv_end = min(si.n, max(q0 + BM, si.ctx_eff));
  const int nkv = (kv_end + BN - 1) / BN;
  const int cap0 = si.cap > 0 ? si.cap : 0;
  const int skip_a = (max(cap0, si.ctx_eff) + BN - 1) / BN;
  const int skip_b = q0 / BN;
  const bool has_skip = skip_a < skip_b;

  // staging roles of this thread
  const int k_chunk = tid & 15, k_row0 = tid >> 4;        // K: rows k_row0 + 16 ps, 16-byte chunk
  const int v_g = tid >> 4, v_e = tid & 15;               // V: rows 4 v_g .. +3, d = 8 v_e .. +7
  const int v_c16 = 2 * (v_g >> 2) + (v_g & 1), v_a = (v_g >> 1) & 1;

  // Global addresses are (uniform tile base) + (per-thread 32-bit byte offset): no 64-bit vector
  // arithmetic and no multiplies inside the loop.  Rows at or past the end of the sequence (last,
  // partial tile only) re-read the sequence's last row; the mask zeroes their contribution.
  const unsigned row_bytes = (unsigned)row_stride * 2u;
  const unsigned k_off0 = (unsigned)k_row0 * row_bytes + (unsigned)k_chunk * 16u;
  const unsigned v_off0 = (unsigned)(4 * v_g) * row_bytes + (unsigned)v_e * 16u;
  const char* __restrict__ kgb = (const char*)kg;
  const char* __restrict__ vgb = (const char*)vg;

  auto load_tile = [&](int it, TileRegs& tr) __attribute__((always_inline)) {
    const int k0 = it * BN;
    const char* kt = kgb + (size_t)k0 * row_bytes;
    const char* vt = vgb + (size_t)k0 * row_bytes;
    unsigned ko0 = k_off0, ko1 = k_off0 + 16 * row_bytes, ko2 = k_off0 + 32 * row_bytes, ko3 = k_off0 + 48 * row_bytes;
    unsigned vo0 = v_off0, vo1 = v_off0 + row_bytes, vo2 = v_off0 + 2 * row_bytes, vo3 = v_off0 + 3 * row_bytes;
    if (k0 + BN > si.n) {
      asm volatile("" ::: "memory");   // keep this a branch: the multiplies below must stay off the steady-state path
      const int last = si.n - 1 - k0;  // >= 0: a tile is only visited when k0 < n
      const unsigned kc = (unsigned)k_chunk * 16u, vc = (unsigned)v_e * 16u;
      ko0 = (unsigned)min(k_row0, last) * row_bytes + kc;
      ko1 = (unsigned)min(k_row0 + 16, last) * row_bytes + kc;
      ko2 = (unsigned)min(k_row0 + 32, last) * row_bytes + kc;
      ko3 = (unsigned)min(k_row0 + 48, last) * row_bytes + kc;
      vo0 = (unsigned)min(4 * v_g, last) * row_bytes + vc;
      vo1 = (unsigned)min(4 * v_g + 1, last) * row_bytes + vc;
      vo2 = (unsigned)min(4 * v_g + 2, last) * row_bytes + vc;
      vo3 = (unsigned)min(4 * v_g + 3, last) * row_bytes + vc;
    }
    tr.k0 = *(const u32x4*)(kt + ko0);
    tr.k1 = *(const u32x4*)(kt + ko1);
    tr.k2 = *(const u32x4*)(kt + ko2);
    tr.k3 = *(const u32x4*)(kt + ko3);
    tr.v0 = *(const u32x4*)(vt + vo0);
    tr.v1 = *(const u32x4*)(vt + vo1);
    tr.v2 = *(const u32x4*)(vt + vo2);
    tr.v3 = *(const u32x4*)(vt + vo3);
    if (HAS_RAB) {
      // band of bias entries this (q tile, kv tile) can touch: index (m - j) + N - 1
      int idx = q0 - k0 - (BN - 1) + p.N - 1 + tid;
      idx = idx < 0 ? 0 : (idx >= rab_w ? rab_w - 1 : idx);
      tr.rab = (tid < BM + BN - 1) ? rabg[idx] * bias_mul : 0.f;
    }
  };

  // LDS byte addresses of this thread's staging stores (buffer 0); the swizzled K chunk does not
  // depend on the pass because 16 ps leaves row & 7 unchanged; for V^T the swizzle of row
  // d = 8 v_e + i is (i ^ v_e) & 7, so the chunk is (v_c16 ^ (v_e & 7)) ^ i.
  const unsigned ks_st = (unsigned)k_row0 * (HD * 2) + (unsigned)((k_chunk ^ (k_row0 & 7)) * 16);
  const unsigned vt_cx = (unsigned)((v_c16 ^ (v_e & 7)) * 16);
  const unsigned vt_st = (unsigned)(8 * v_e) * (BN * 2) + (unsigned)v_a * 8u;

  auto store_tile = [&](int buf, const TileRegs& tr) __attribute__((always_inline)) {
    char* kb = (char*)&Ks[buf][0] + ks_st;
    *(u32x4*)(kb) = tr.k0;
    *(u32x4*)(kb + 16 * HD * 2) = tr.k1;
    *(u32x4*)(kb + 32 * HD * 2) = tr.k2;
    *(u32x4*)(kb + 48 * HD * 2) = tr.k3;
    char* vb = (char*)&Vts[buf][0] + vt_st;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const unsigned w0 = tr.v0[i >> 1], w1 = tr.v1[i >> 1], w2 = tr.v2[i >> 1], w3 = tr.v3[i >> 1];
      u32x2 o;
      if (i & 1) {
        o.x = (w0 >> 16) | (w1 & 0xffff0000u);
        o.y = (w2 >> 16) | (w3 & 0xffff0000u);
      } else {
        o.x = (w0 & 0xffffu) | (w1 << 16);
        o.y = (w2 & 0xffffu) | (w3 << 16);
      }
      *(u32x2*)(vb + i * (BN * 2) + (vt_cx ^ (unsigned)(i * 16))) = o;
    }
    if (HAS_RAB) {
      if (tid < BM + BN - 1) rabs[buf][tid] = tr.rab;
    }
  };

  // LDS byte offsets of this lane's MFMA A-operand reads.  K: row = 32 kvb + l32, chunk 2 kk + half;
  // the swizzle touches only the low 3 chunk bits, so kk and kk + 4 differ by a constant 128 bytes
  // and kvb by a constant 32 rows.  V^T: row d = 32 db + l32 has swizzle
  // (l32 ^ (4 db + (l32 >> 3))) & 7 = vt_swz(l32) ^ 4 (db & 1): odd db flips chunk bit 2 (64 bytes).
  // Both chunk indices are (constant) ^ (lane part), so every read address is one per-lane base
  // XOR a compile-time constant in address bits 5..6.
  const unsigned ks_rd = (unsigned)l32 * (HD * 2) + (unsigned)((half ^ (l32 & 7)) * 16);
  const unsigned vt_rd = (unsigned)l32 * (BN * 2) + (unsigned)((half ^ vt_swz(l32)) * 16);

  // silu + mask + bf16 packing of one 32 x 32 score block (accumulator layout) into two B operands
  auto silu_pack = [&](auto masked_tag, const f32x16& sv, int k0, int kvb, int buf, bf16x8& o0,
                       bf16x8& o1) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    f32x16 pv;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int jl = kvb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
      float s = sv[r];
      if (HAS_RAB) s += rabs[buf][(m - q0) - jl + (BN - 1)];  // bias staged divided by alpha
      const float t = s * neg_c;  // -x log2(e); P is kept as t sigmoid(x), its factor -1 / log2(e) goes on the output
      float pe = t * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
      if (MASKED) {
        const int j = k0 + jl;
        // branch-free keep(m, j) & (j < n)
        const bool kp = ((m == j) | ((m >= j) & (j < si.cap)) | (j < si.ctx_eff)) & (j < si.n);
        pe = kp ? pe : 0.f;
      }
      pv[r] = pe;
    }
    u32x4 w0, w1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w0[i] = pack_bf16x2(pv[2 * i], pv[2 * i + 1]);
      w1[i] = pack_bf16x2(pv[8 + 2 * i], pv[8 + 2 * i + 1]);
    }
    o0 = __builtin_bit_cast(bf16x8, w0);
    o1 = __builtin_bit_cast(bf16x8, w1);
  };

  // One (32 query rows) x (64 keys) block of this wave.  The code is laid out in four stages of
  // eight MFMAs; the VALU work of one stage is independent of that stage's MFMAs, and the
  // scheduling fences keep the two streams interleaved so the matrix pipe runs in the shadow of
  // the SiLU arithmetic:
  //   0: S0 = K[0:32] Q^T          |  -
  //   A: S1 = K[32:64] Q^T         |  P0 = silu(S0)
  //   B: O += V^T[:, 0:32] P0      |  P1 = silu(S1)
  //   C: O += V^T[:, 32:64] P1     |  (caller: register -> LDS staging of the next tile)
  auto tile_body = [&](auto masked_tag, int k0, int buf) __attribute__((always_inline)) {
    const char* kb = (const char*)&Ks[buf][0];
    const char* vb = (const char*)&Vts[buf][0];
    const f32x16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    auto k_frag = [&](int kvb, int kk) __attribute__((always_inline)) {
      return *(const bf16x8*)(kb + kvb * 32 * HD * 2 + (ks_rd ^ (unsigned)((kk & 3) * 32)) + (kk >> 2) * 128);
    };
    auto v_frag = [&](int db, int s2) __attribute__((always_inline)) {
      return *(const bf16x8*)(vb + db * 32 * BN * 2 + (vt_rd ^ (unsigned)((s2 * 32) ^ ((db & 1) * 64))));
    };
    f32x16 s0, s1;
    bf16x8 pb0, pb1, pb2, pb3;
    // stage 0
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k_frag(0, kk), qf[kk], kk == 0 ? zero : s0, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    // stage A
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k_frag(1, kk), qf[kk], kk == 0 ? zero : s1, 0, 0, 0);
    silu_pack(masked_tag, s0, k0, 0, buf, pb0, pb1);
    // MFMAs issue in pairs: the second of a back-to-back pair costs less issue time than a
    // lone one, and the pair's 64 pipe cycles cover the VALU batch that follows
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);   // 2 MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 10, 0);  // 10 VALU
      __builtin_amdgcn_sched_group_barrier(0x400, 8, 0);   // 8 transcendental
    }
    __builtin_amdgcn_sched_barrier(0);
    // stage B
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v_frag(db, 0), pb0, acc[db], 0, 0, 0);
      acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v_frag(db, 1), pb1, acc[db], 0, 0, 0);
    }
    silu_pack(masked_tag, s1, k0, 1, buf, pb2, pb3);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 10, 0);
      __builtin_amdgcn_sched_group_barrier(0x400, 8, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    // stage C
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v_frag(db, 2), pb2, acc[db], 0, 0, 0);
      acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v_frag(db, 3), pb3, acc[db], 0, 0, 0);
    }
  };

  auto compute_tile = [&](int it, int buf) __attribute__((always_inline)) {
    const int k0 = it * BN;
    const int k1 = k0 + BN;
    // wave-level classification of this (32 query rows) x (64 keys) block
    if (!wave_has_rows) return;
    const bool any_kept = (k0 <= m_hi && k1 > m_lo) /* diagonal crosses */ ||
                          (k0 < si.cap && k0 <= m_hi) /* causal history */ || (k0 < si.ctx_eff);
    if (!any_kept) return;
    const bool full = (k1 - 1 <= m_lo) && (k1 <= si.cap);  // implies k1 <= n
    if (full) tile_body(std::false_type{}, k0, buf);
    else tile_body(std::true_type{}, k0, buf);
  };

  auto next_tile = [&](int it) { return (has_skip && it + 1 == skip_a) ? skip_b : it + 1; };

  TileRegs tr;
  int it = (has_skip && skip_a == 0) ? skip_b : 0;
  int buf = 0;
  if (it < nkv) {
    load_tile(it, tr);
    store_tile(0, tr);
    __syncthreads();
    int nxt = next_tile(it);
    if (nxt < nkv) load_tile(nxt, tr);
    while (true) {
      compute_tile(it, buf);
      if (nxt >= nkv) break;
      store_tile(buf ^ 1, tr);
      __syncthreads();
      it = nxt;
      buf ^= 1;
      nxt = next_tile(it);
      if (nxt < nkv) load_tile(nxt, tr);
    }
  }

  // ---- epilogue: O^T accumulators -> out[s + m, h, :] ----
  if (m < si.n) {
    float oscale = 1.0f / (float)p.N;
    if (p.attn_scale)
      oscale = (p.flags & RECIR_HSTU_FLAG_SCALE_PER_TOKEN) ? p.attn_scale[si.s + m] : p.attn_scale[0];
    oscale *= -1.0f / kLog2e;
    unsigned short* orow = (unsigned short*)p.out + ((size_t)(si.s + m) * p.H + h) * HD;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        u32x2 o;
        o.x = pack_bf16x2(acc[db][4 * rq + 0] * oscale, acc[db][4 * rq + 1] * oscale);
        o.y = pack_bf16x2(acc[db][4 * rq + 2] * oscale, acc[db][4 * rq + 3] * oscale);
        *(u32x2*)(orow + db * 32 + 8 * rq + 4 * half) = o;
      }
    }
  }
  __syncthreads();  // LDS buffers are reused by the next item
  }  // work items
}

}  // namespace recir_hstu
