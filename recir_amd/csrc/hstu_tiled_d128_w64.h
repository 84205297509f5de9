// Tiled MFMA kernel of the HSTU attention forward, head dim 128, 64 query rows per wave.
//
// One workgroup (4 waves, one per SIMD, up to 512 registers each) per (sequence, head, query tile of
// 256 rows); wave w owns query rows [64 w, 64 w + 64) as two 32-row blocks.  Every K and V^T fragment
// read from LDS feeds two MFMAs (one per row block), which halves the LDS traffic per FLOP of the
// 32-rows-per-wave kernels -- LDS bandwidth (128 B/clk per CU) is what bounds those.
//
// Per key tile of 64 rows, for both row blocks:
//   S^T = K Q^T               v_mfma_f32_32x32x16_bf16 (fp8: v_mfma_scale_f32_32x32x64_f8f6f4)
//   P^T = silu(S^T (+rab)) masked, bf16, in registers (accumulator layout = B-operand layout)
//   O^T += V^T P^T            A = V^T via ds_read_b64_tr_b16 from the row-major V tile
//
// K/V tiles travel HBM -> LDS with global_load_lds_dwordx4 into a ring of four stages (128 KB); the
// copies of tile i + 3 are issued at the start of tile i, so a copy has three tile times to land.
// The copies are issued from inline assembly with explicit vmcnt waits: the ring slot is a run-time
// value and the compiler would otherwise serialise every LDS read behind all copies in flight.
// One barrier per tile: it publishes tile i (all waves have waited for their own copies) and
// retires tile i - 1, whose slot the new copies overwrite.
//
// LDS layouts, swizzles, the SiLU formulation and the mask handling are those of
// hstu_tiled_d128_dl.h.
#pragma once
#include <type_traits>

#include "hstu_common.h"
#include "hstu_tiled_d128_dl.h"

namespace recir_hstu {

#ifndef W64_ABL
#define W64_ABL 0   // debug builds only: bit mask of parts to leave out (timing experiments)
#endif
constexpr int BM2 = 256;     // query rows per workgroup
constexpr int W64_STAGES = 4;
constexpr bool W64_Q_IN_ACC = false;
constexpr int W64_DIST = 3;  // tiles of prefetch distance

// one global -> LDS copy of 64 lanes x 16 bytes; lds_addr is wave-uniform
__device__ __forceinline__ void dma16(const void* gbase, unsigned voff, unsigned lds_addr) {
  if (W64_ABL & 8) return;
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_addr), "v"(voff), "s"(gbase) : "memory");
}
__device__ __forceinline__ void dma4(const void* gbase, unsigned voff, unsigned lds_addr) {
  if (W64_ABL & 8) return;
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds_addr), "v"(voff), "s"(gbase) : "memory");
}

template <bool HAS_RAB, bool FP8>
__global__ __launch_bounds__(256, 1) void hstu_fwd_tiled_d128_w64(Params p) {
  __shared__ __attribute__((aligned(1024))) unsigned short Kring[W64_STAGES][BN * HD];
  __shared__ __attribute__((aligned(1024))) unsigned short Vring[W64_STAGES][BN * HD];
  constexpr int RAB_BAND = 512;  // >= BM2 + BN - 1, one dword per lane of 8 copy instructions
  __shared__ __attribute__((aligned(1024))) float rab_ring[W64_STAGES][HAS_RAB ? RAB_BAND : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int half = lane >> 5;

  zero_tail_rows<256>(p, (size_t)p.H * HD * 2);

  // ---- per-lane constants of the LDS access patterns (see hstu_tiled_d128_dl.h) ----
  const unsigned ks_rd = (unsigned)l32 * (HD * 2) + (unsigned)((half ^ (l32 & 7)) * 16);
  const int tr_s = lane & 15, tr_r = tr_s >> 2, tr_c = tr_s & 3, tr_dgrp = (lane >> 4) & 1;
  const unsigned vt_base = (unsigned)(4 * half + tr_r) * (HD * 2) + (unsigned)((tr_dgrp ^ (tr_r & 1)) * 32) + (unsigned)tr_c * 8u;
  const unsigned vt_rd_e = vt_base + (unsigned)((tr_r >> 1) * 64);
  const unsigned vt_rd_o = vt_base - (unsigned)((tr_r >> 1) * 64);
  const int ld_row = lane >> 4, ld_chunk = lane & 15;
  const unsigned k8_rd = (unsigned)l32 * 128u + (unsigned)(((2 * half) ^ (l32 & 7)) * 16);
  const int ld8_row = lane >> 3, ld8_chunk = lane & 7;
  // copies per wave per tile (vmcnt bookkeeping): K 4 (fp8: 2) + V 4 (+ 2 for the bias band)
  constexpr int DMA_PER_TILE = (FP8 ? 2 : 4) + 4 + (HAS_RAB ? 2 : 0);

  const unsigned k_lds0 = (unsigned)(size_t)&Kring[0][0];
  const unsigned v_lds0 = (unsigned)(size_t)&Vring[0][0];
  const unsigned r_lds0 = (unsigned)(size_t)&rab_ring[0][0];

#ifdef HSTU_TRACE
  const bool trace_on = (int)blockIdx.x == g_trace_block;
  int trace_it = 0;
#endif
  const int xcd = blockIdx.x % NUM_XCD;
  const int list_len = p.ws_counts[xcd];
  const WorkItem* __restrict__ list = p.ws_items + (size_t)xcd * p.items_cap;
  for (int slot = blockIdx.x / NUM_XCD; slot < list_len; slot += p.grid_slots) {
    HSTU_ITEM_STAMP(0);
    const WorkItem wi = list[slot];
    SeqInfo si;
    si.s = wi.s; si.n = wi.n; si.cap = wi.cap; si.ctx_eff = wi.ctx_eff;
    const int q0 = wi.q0;
    const int h = wi.h;

    const unsigned row_bytes = (unsigned)p.H * HD * 2u;
    const unsigned krow_bytes = FP8 ? (unsigned)p.H * HD : row_bytes;
    const char* __restrict__ kgb = (const char*)p.k + ((size_t)si.s * p.H + h) * (FP8 ? HD : HD * 2);
    const char* __restrict__ vgb = (const char*)p.v + ((size_t)si.s * p.H + h) * (HD * 2);
    const int rab_w = 2 * p.N - 1;
    const float* __restrict__ rabg = HAS_RAB ? p.rab + (size_t)h * rab_w : nullptr;

    const unsigned k_off_e = (unsigned)ld_row * krow_bytes + (unsigned)((ld_chunk ^ ld_row) * 16);
    const unsigned k_off_o = (unsigned)ld_row * krow_bytes + (unsigned)((ld_chunk ^ (4 + ld_row)) * 16);
    const unsigned v_off = (unsigned)ld_row * row_bytes + (unsigned)((ld_chunk ^ (2 * ld_row)) * 16);
    const unsigned k8_off = (unsigned)ld8_row * krow_bytes + (unsigned)((ld8_chunk ^ ld8_row) * 16);

    const int qw0 = q0 + wave * 64;
    const int ma = qw0 + l32;   // this lane's query row in block a; block b is ma + 32
    const int m_lo = qw0;
    const int m_hi = min(qw0 + 63, si.n - 1);
    const bool wave_has_rows = m_lo < si.n;

    const int kv_end = min(si.n, max(q0 + BM2, si.ctx_eff));
    const int nkv = (kv_end + BN - 1) / BN;
    const int cap0 = si.cap > 0 ? si.cap : 0;
    const int skip_a = (max(cap0, si.ctx_eff) + BN - 1) / BN;
    const int skip_b = q0 / BN;
    const bool has_skip = skip_a < skip_b;
    auto next_tile = [&](int it) { return (has_skip && it + 1 == skip_a) ? skip_b : it + 1; };

    // Copies of one tile into ring slot st: exactly DMA_PER_TILE instructions per wave.  Rows at or
    // past the end of the sequence (last, partial tile only) re-read the sequence's last row.
    auto issue_tile = [&](int it, int st) __attribute__((always_inline)) {
      const int k0 = it * BN;
      const char* kt = kgb + (size_t)k0 * krow_bytes;
      const char* vt = vgb + (size_t)k0 * row_bytes;
      const bool whole = k0 + BN <= si.n;
      const int last = si.n - 1 - k0;
      const unsigned kl = k_lds0 + (unsigned)st * (BN * HD * 2);
      const unsigned vl = v_lds0 + (unsigned)st * (BN * HD * 2);
#pragma unroll
      for (int ps = 0; ps < 4; ++ps) {
        const int r0 = 4 * (4 * wave + ps);
        unsigned ko = (ps & 1) ? k_off_o : k_off_e;
        unsigned vo = v_off;
        const char* kr = kt + (size_t)r0 * krow_bytes;
        const char* vr = vt + (size_t)r0 * row_bytes;
        if (!whole) {
          asm volatile("" ::: "memory");
          const int row = min(r0 + ld_row, last);
          ko = (unsigned)row * krow_bytes + (unsigned)((ld_chunk ^ ((r0 + ld_row) & 7)) * 16);
          vo = (unsigned)row * row_bytes + (unsigned)((ld_chunk ^ (2 * ld_row)) * 16);
          kr = kt;
          vr = vt;
        }
        if (!FP8) dma16(kr, ko, kl + (unsigned)r0 * (HD * 2));
        dma16(vr, vo, vl + (unsigned)r0 * (HD * 2));
      }
      if (FP8) {
#pragma unroll
        for (int ps = 0; ps < 2; ++ps) {
          const int r0 = 8 * (2 * wave + ps);
          unsigned ko = k8_off;
          const char* kr = kt + (size_t)r0 * krow_bytes;
          if (!whole) {
            asm volatile("" ::: "memory");
            ko = (unsigned)min(r0 + ld8_row, last) * krow_bytes + (unsigned)((ld8_chunk ^ ld8_row) * 16);
            kr = kt;
          }
          dma16(kr, ko, kl + (unsigned)r0 * 128u);
        }
      }
      if (HAS_RAB) {
        // bias band of this (q tile, kv tile): entry i holds rab[(q0 - k0 - (BN - 1) + N - 1) + i]
#pragma unroll
        for (int ps = 0; ps < 2; ++ps) {
          const int i = (2 * wave + ps) * 64 + lane;
          int idx = q0 - k0 - (BN - 1) + p.N - 1 + i;
          idx = idx < 0 ? 0 : (idx >= rab_w ? rab_w - 1 : idx);
          dma4(rabg, (unsigned)idx * 4u, r_lds0 + (unsigned)st * (RAB_BAND * 4) + (unsigned)(2 * wave + ps) * 256u);
        }
      }
    };

    // ---- prologue: the first W64_DIST tiles go in flight before anything is waited for ----
    int it = (has_skip && skip_a == 0) ? skip_b : 0;
    int it_issue = it;     // next tile to issue
    int issued = 0;        // tiles issued and not yet consumed
    int st_issue = 0;      // ring slot of the next issue
#pragma unroll
    for (int d = 0; d < W64_DIST; ++d) {
      if (it_issue < nkv) {
        issue_tile(it_issue, st_issue);
        it_issue = next_tile(it_issue);
        st_issue = (st_issue + 1) & (W64_STAGES - 1);
        ++issued;
      }
    }

    // ---- Q fragments (B operands) of both row blocks ----
    bf16x8 qf[2][FP8 ? 1 : 8];
    i32x8 q8[2][FP8 ? 2 : 1];
    float s_mul = 1.0f;
    if constexpr (FP8) s_mul = p.alpha * p.q_scale[h] * p.k_scale[h] * kLog2e;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int m = ma + 32 * qb;
      const bool valid = m < si.n;
      const u32x4 zero4 = {0u, 0u, 0u, 0u};
      if constexpr (FP8) {
        const char* qrow = (const char*)p.q + ((size_t)(si.s + (valid ? m : 0)) * p.H + h) * HD;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const u32x4 lo = valid ? *(const u32x4*)(qrow + 64 * st + 32 * half) : zero4;
          const u32x4 hi = valid ? *(const u32x4*)(qrow + 64 * st + 32 * half + 16) : zero4;
          q8[qb][st] = (i32x8){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        }
      } else {
        const unsigned short* qrow = (const unsigned short*)p.q + ((size_t)(si.s + (valid ? m : 0)) * p.H + h) * HD;
        const float qmul = p.alpha * kLog2e;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const u32x4 t = valid ? *(const u32x4*)(qrow + kk * 16 + half * 8) : zero4;
          u32x4 sc;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            sc[i] = pack_bf16x2(__uint_as_float(t[i] << 16) * qmul, __uint_as_float(t[i] & 0xffff0000u) * qmul);
          qf[qb][kk] = __builtin_bit_cast(bf16x8, sc);
          // Q is only ever an MFMA operand from here on: park it in the accumulation register file
          if (W64_Q_IN_ACC) asm volatile("" : "+a"(qf[qb][kk]));
        }
      }
    }
    // the q loads above are ordinary vector loads issued after the first copies: once their data
    // has been used, everything issued before them has landed as well.  Make that explicit so the
    // counting below starts from a known state.
    HSTU_ITEM_STAMP(1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    HSTU_ITEM_STAMP(2);
#ifdef HSTU_TRACE
    const long long trace_c2 = clock64();
#endif

    f32x16 acc[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[qb][i][r] = 0.f;
    // the output accumulators are only ever MFMA operands until the epilogue: start them out in
    // the accumulation register file
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int db = 0; db < 4; ++db) asm volatile("" : "+a"(acc[qb][db]));

    // silu + mask + bf16 packing of one 32 x 32 score block into two B operands
    auto silu_pack = [&](auto masked_tag, const f32x16& sv, int m, int k0, int kvb, const float* rabt,
                         bf16x8& o0, bf16x8& o1) __attribute__((always_inline)) {
      constexpr bool MASKED = decltype(masked_tag)::value;
      f32x16 pv;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int jl = kvb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        float s = sv[r];
        if (FP8) s *= s_mul;
        if (HAS_RAB) s = fmaf(rabt[(m - q0) - jl + (BN - 1)], kLog2e, s);
        const float ex = __builtin_amdgcn_exp2f(-s);
        float pe = s * __builtin_amdgcn_rcpf(1.0f + ex);
        if (MASKED) {
          const int j = k0 + jl;
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

    // One (64 query rows) x (64 keys) block of this wave: eight groups of four fragments, each
    // fragment feeding both row blocks (8 MFMAs per group); fragments are fetched one group ahead.
    //   groups 0,1: S0 (K rows 0..31)    groups 2,3: S1 (K rows 32..63)   | P0 = silu(S0) over 2,3
    //   groups 4,5: O += V^T[:, 0:32] P0                                  | P1 = silu(S1) over 4,5
    //   groups 6,7: O += V^T[:, 32:64] P1
    auto tile_body = [&](auto masked_tag, int k0, int st) __attribute__((always_inline)) {
      const char* kb = (const char*)&Kring[0][0] + st * (BN * HD * 2);
      const char* vb = (const char*)&Vring[0][0] + st * (BN * HD * 2);
      const float* rabt = &rab_ring[0][0] + (HAS_RAB ? st * RAB_BAND : 0);
      const f32x16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      auto k_frag = [&](int kvb, int kk) __attribute__((always_inline)) {
        return *(const bf16x8*)(kb + kvb * 32 * HD * 2 + (ks_rd ^ (unsigned)((kk & 3) * 32)) + (kk >> 2) * 128);
      };
      auto v_frag = [&](int db, int s2) __attribute__((always_inline)) {
        const char* a = vb + ((db & 1) ? vt_rd_o : vt_rd_e) + db * 64 + s2 * 16 * HD * 2;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)a);
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(a + 8 * HD * 2));
        const i16x8 both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        return __builtin_bit_cast(bf16x8, both);
      };
      f32x16 s0[2], s1[2];
      bf16x8 pb[2][4];
      auto load_group = [&](int g, bf16x8 (&f)[4]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (g < 4) f[i] = k_frag(g >> 1, (g & 1) * 4 + i);
          else f[i] = v_frag(((g & 1) * 2) + (i >> 1), ((g - 4) >> 1) * 2 + (i & 1));
        }
      };
      auto mfma_group = [&](int g, const bf16x8 (&f)[4]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) {
            if (g < 2) {
              const int kk = FP8 ? 0 : g * 4 + i;
              s0[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i], qf[qb][kk], (g * 4 + i) == 0 ? zero : s0[qb], 0, 0, 0);
            } else if (g < 4) {
              const int kk = FP8 ? 0 : (g - 2) * 4 + i;
              s1[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i], qf[qb][kk], ((g - 2) * 4 + i) == 0 ? zero : s1[qb], 0, 0, 0);
            } else {
              const int db = ((g & 1) * 2) + (i >> 1);
              const int s2 = ((g - 4) >> 1) * 2 + (i & 1);
              acc[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i], pb[qb][s2], acc[qb][db], 0, 0, 0);
            }
          }
        }
      };
      bf16x8 fa[4], fb[4];
      if constexpr (FP8) {
        auto k8_frag = [&](int kvb, int st8) __attribute__((always_inline)) {
          const char* a = kb + kvb * 32 * 128;
          const u32x4 lo = *(const u32x4*)(a + (k8_rd ^ (unsigned)((4 * st8) * 16)));
          const u32x4 hi = *(const u32x4*)(a + (k8_rd ^ (unsigned)((4 * st8 + 1) * 16)));
          return (i32x8){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        };
        const i32x8 ka0 = k8_frag(0, 0), ka1 = k8_frag(0, 1);
        const i32x8 kb0 = k8_frag(1, 0), kb1 = k8_frag(1, 1);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          s0[qb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ka0, q8[qb][0], zero, 0, 0, 0, 0x7f7f7f7f, 0, 0x7f7f7f7f);
          s0[qb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ka1, q8[qb][1], s0[qb], 0, 0, 0, 0x7f7f7f7f, 0, 0x7f7f7f7f);
        }
        __builtin_amdgcn_sched_barrier(0);
        load_group(4, fa);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          s1[qb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(kb0, q8[qb][0], zero, 0, 0, 0, 0x7f7f7f7f, 0, 0x7f7f7f7f);
          s1[qb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(kb1, q8[qb][1], s1[qb], 0, 0, 0, 0x7f7f7f7f, 0, 0x7f7f7f7f);
        }
        silu_pack(masked_tag, s0[0], ma, k0, 0, rabt, pb[0][0], pb[0][1]);
        silu_pack(masked_tag, s0[1], ma + 32, k0, 0, rabt, pb[1][0], pb[1][1]);
      } else {
        load_group(0, fa);
        load_group(1, fb);
        mfma_group(0, fa);
        __builtin_amdgcn_sched_barrier(0);
        load_group(2, fa);
        mfma_group(1, fb);
        __builtin_amdgcn_sched_barrier(0);
        // groups 2 and 3 with silu(S0), one row block per group so that few SiLU chains are live at once
        load_group(3, fb);
        mfma_group(2, fa);
        silu_pack(masked_tag, s0[0], ma, k0, 0, rabt, pb[0][0], pb[0][1]);
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);   // 2 MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 14, 0);  // 14 VALU (incl. the reads of the score registers)
          __builtin_amdgcn_sched_group_barrier(0x400, 8, 0);   // 8 transcendental
        }
        __builtin_amdgcn_sched_barrier(0);
        load_group(4, fa);
        mfma_group(3, fb);
        silu_pack(masked_tag, s0[1], ma + 32, k0, 0, rabt, pb[1][0], pb[1][1]);
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 14, 0);
          __builtin_amdgcn_sched_group_barrier(0x400, 8, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      // groups 4 and 5 with silu(S1)
      load_group(5, fb);
      mfma_group(4, fa);
      silu_pack(masked_tag, s1[0], ma, k0, 1, rabt, pb[0][2], pb[0][3]);
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 14, 0);
        __builtin_amdgcn_sched_group_barrier(0x400, 8, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      load_group(6, fa);
      mfma_group(5, fb);
      silu_pack(masked_tag, s1[1], ma + 32, k0, 1, rabt, pb[1][2], pb[1][3]);
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 14, 0);
        __builtin_amdgcn_sched_group_barrier(0x400, 8, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      load_group(7, fb);
      mfma_group(6, fa);
      __builtin_amdgcn_sched_barrier(0);
      mfma_group(7, fb);
    };

    // bf16 path: one (64 query rows) x (64 keys) block as 64 slots of one MFMA each, in program
    // order (a scheduling barrier closes every slot), with the LDS reads and the SiLU work of
    // other blocks placed into the slots by hand:
    //   slots  0..7   S0a = K[0:32] Qa^T     8..15  S0b = K[0:32] Qb^T      (a, b: the two row blocks)
    //   slots 16..23  S1a = K[32:64] Qa^T   24..31  S1b = K[32:64] Qb^T
    //   slots 32..39  Oa += V^T[:, 0:32] P0a    40..47  Ob += V^T[:, 0:32] P0b
    //   slots 48..55  Oa += V^T[:, 32:64] P1a   56..63  Ob += V^T[:, 32:64] P1b
    // Each fragment is read once and feeds both row blocks: buffer FA holds K[0:32] (slots 0..15),
    // then V^T[:, 0:32] (32..47); FB holds K[32:64] (16..31), then V^T[:, 32:64] (48..63).
    // The 32 SiLU units (two scores each, in the order S0a S0b S1a S1b) are spread over slots
    // 10..55, which keeps every unit after the MFMA chain that produces its scores and before the
    // MFMA that consumes its packed result.
    auto tile_body_slots = [&](auto masked_tag, int k0, int st) __attribute__((always_inline)) {
      constexpr bool MASKED = decltype(masked_tag)::value;
      const char* kb = (const char*)&Kring[0][0] + st * (BN * HD * 2);
      const char* vb = (const char*)&Vring[0][0] + st * (BN * HD * 2);
      const float* rabt = &rab_ring[0][0] + (HAS_RAB ? st * RAB_BAND : 0);
      const f32x16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      auto k_frag = [&](int kvb, int kk) __attribute__((always_inline)) {
        return *(const bf16x8*)(kb + kvb * 32 * HD * 2 + (ks_rd ^ (unsigned)((kk & 3) * 32)) + (kk >> 2) * 128);
      };
      auto v_frag = [&](int db, int s2) __attribute__((always_inline)) {
        const char* a = vb + ((db & 1) ? vt_rd_o : vt_rd_e) + db * 64 + s2 * 16 * HD * 2;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)a);
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(a + 8 * HD * 2));
        const i16x8 both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        return __builtin_bit_cast(bf16x8, both);
      };
      f32x16 sc[4];        // S0a S0b S1a S1b
      unsigned pw[4][8];   // packed P of the same four blocks: words 0..3 = keys 0..15, 4..7 = keys 16..31 of the block
      bf16x8 FA[8], FB[8];
      auto silu_unit = [&](int u) __attribute__((always_inline)) {
        const int blk = u >> 3, e = u & 7;
        const int qb = blk & 1, kvb = blk >> 1;
        const int m = ma + 32 * qb;
        float pe[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int r = 2 * e + t;
          const int jl = kvb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          float sv = sc[blk][r];
          if (HAS_RAB) sv = fmaf(rabt[(m - q0) - jl + (BN - 1)], kLog2e, sv);
          const float ex = __builtin_amdgcn_exp2f(-sv);
          float pv = sv * __builtin_amdgcn_rcpf(1.0f + ex);
          if (MASKED) {
            const int j = k0 + jl;
            const bool kp = ((m == j) | ((m >= j) & (j < si.cap)) | (j < si.ctx_eff)) & (j < si.n);
            pv = kp ? pv : 0.f;
          }
          pe[t] = pv;
        }
        pw[blk][e] = pack_bf16x2(pe[0], pe[1]);
        if (W64_ABL & 1) pw[blk][e] = 0x3f803f80u;
      };
      auto p_frag = [&](int blk, int s2l) __attribute__((always_inline)) {
        const u32x4 w = {pw[blk][4 * s2l + 0], pw[blk][4 * s2l + 1], pw[blk][4 * s2l + 2], pw[blk][4 * s2l + 3]};
        return __builtin_bit_cast(bf16x8, w);
      };
      constexpr int U_FIRST = 10, U_LAST = 56, U_SPAN = U_LAST - U_FIRST;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) FA[kk] = (W64_ABL & 2) ? qf[1][kk] : k_frag(0, kk);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < 64; ++s) {
        // LDS reads of later slots
        if (W64_ABL & 2) {
          if (s < 8) FB[s] = qf[0][s];
        } else if (s < 8) {
          FB[s] = k_frag(1, s);
        } else if (s >= 16 && s < 32) {
          if (((s - 16) & 1) == 0) { const int f = (s - 16) >> 1; FA[f] = v_frag(f >> 1, f & 1); }
        } else if (s >= 32 && s < 48) {
          if (((s - 32) & 1) == 0) { const int f = (s - 32) >> 1; FB[f] = v_frag(f >> 1, 2 + (f & 1)); }
        }
        // the MFMA of this slot
        if (s < 32) {
          const int blk = s >> 3, kk = s & 7;
          const int qb = blk & 1, kvb = blk >> 1;
          sc[blk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kvb ? FB[kk] : FA[kk], qf[qb][kk], kk == 0 ? zero : sc[blk], 0, 0, 0);
        } else {
          const int i = s & 7, qb = (s >> 3) & 1, kvb = (s - 32) >> 4;
          const int db = i >> 1, s2l = i & 1;
          acc[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kvb ? FB[i] : FA[i], p_frag(2 * kvb + qb, s2l), acc[qb][db], 0, 0, 0);
        }
        // SiLU units of this slot
        if (s >= U_FIRST && s < U_LAST) {
          const int u0 = ((s - U_FIRST) * 32) / U_SPAN, u1 = ((s + 1 - U_FIRST) * 32) / U_SPAN;
#pragma unroll
          for (int u = u0; u < u1; ++u) silu_unit(u);
        }
        __builtin_amdgcn_sched_barrier(0);
        if ((W64_ABL & 1) && s == 63) asm volatile("" ::"a"(sc[0]), "a"(sc[1]), "a"(sc[2]), "a"(sc[3]));
      }
    };

    auto compute_tile = [&](int itc, int st) __attribute__((always_inline)) {
      const int k0 = itc * BN;
      const int k1 = k0 + BN;
      const bool any_kept = wave_has_rows && ((k0 <= m_hi && k1 > m_lo) || (k0 < si.cap && k0 <= m_hi) ||
                                              (k0 < si.ctx_eff));
      if (!any_kept) return;
      const bool full = (k1 - 1 <= m_lo) && (k1 <= si.cap);
      if constexpr (FP8) {
        if (full) tile_body(std::false_type{}, k0, st);
        else tile_body(std::true_type{}, k0, st);
      } else {
        if (full) tile_body_slots(std::false_type{}, k0, st);
        else tile_body_slots(std::true_type{}, k0, st);
      }
    };

    // ---- main loop: wait for tile `it`, publish it, refill the ring, compute ----
    int st = 0;
    while (it < nkv) {
      HSTU_STAMP(0);
      // this wave's copies of tile `it` have landed when at most (issued - 1) tiles are in flight
      if (issued >= 3) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * DMA_PER_TILE) : "memory");
      else if (issued == 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA_PER_TILE) : "memory");
      else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      HSTU_STAMP(1);
      if (!(W64_ABL & 16)) __syncthreads();  // tile `it` visible to all waves; tile it - 1 no longer read by anyone
      HSTU_STAMP(2);
      --issued;
      if (it_issue < nkv) {
        issue_tile(it_issue, st_issue);
        it_issue = next_tile(it_issue);
        st_issue = (st_issue + 1) & (W64_STAGES - 1);
        ++issued;
      }
      HSTU_STAMP(3);
      compute_tile(it, st);
      HSTU_STAMP(7);
#ifdef HSTU_TRACE
      ++trace_it;
#endif
      it = next_tile(it);
      st = (st + 1) & (W64_STAGES - 1);
    }

    HSTU_ITEM_STAMP(3);
#ifdef HSTU_TRACE
    const long long trace_c3 = clock64();
#endif
    // ---- epilogue ----
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int db = 0; db < 4; ++db) asm volatile("" : "+a"(acc[qb][db]));
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int m = ma + 32 * qb;
      if (m < si.n) {
        float oscale = 1.0f / (float)p.N;
        if (p.attn_scale)
          oscale = (p.flags & RECIR_HSTU_FLAG_SCALE_PER_TOKEN) ? p.attn_scale[si.s + m] : p.attn_scale[0];
        oscale *= 1.0f / kLog2e;
        unsigned short* orow = (unsigned short*)p.out + ((size_t)(si.s + m) * p.H + h) * HD;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
#pragma unroll
          for (int rq = 0; rq < 4; ++rq) {
            u32x2 o;
            o.x = pack_bf16x2(acc[qb][db][4 * rq + 0] * oscale, acc[qb][db][4 * rq + 1] * oscale);
            o.y = pack_bf16x2(acc[qb][db][4 * rq + 2] * oscale, acc[qb][db][4 * rq + 3] * oscale);
            *(u32x2*)(orow + db * 32 + 8 * rq + 4 * half) = o;
          }
        }
      }
    }
#ifdef HSTU_TRACE
    if (lane == 0 && blockIdx.x < 4096 && slot == (int)(blockIdx.x / NUM_XCD))
      g_item_trace[(blockIdx.x * 4 + wave) * 8 + 4] = (unsigned long long)(trace_c3 - trace_c2);
#endif
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // known state for the next item's copy counting
    HSTU_ITEM_STAMP(5);
    if (lane == 0) {
#ifdef HSTU_TRACE
      if (blockIdx.x < 4096 && slot == (int)(blockIdx.x / NUM_XCD)) {
        unsigned hwid;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hwid));
        unsigned xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        g_item_trace[(blockIdx.x * 4 + wave) * 8 + 6] = ((unsigned long long)xcc << 32) | hwid;
        g_item_trace[(blockIdx.x * 4 + wave) * 8 + 7] = (unsigned long long)nkv;
      }
#endif
    }
    __syncthreads();                                   // ring slots are reused by the next item
  }  // work items
}

}  // namespace recir_hstu
