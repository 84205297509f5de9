// Calibration loops: what the chip sustains on the instruction mix of the attention forward, measured
// by kernels that have none of its bookkeeping (no work items, no masks, no epilogue).  They price
// the real kernel: `MFMA only` is the ceiling any bf16 MFMA kernel meets on this chip under its power
// limit, the two tile loops are the forward's inner loop as a stand-alone program.
//
//   kind 0  MFMA only: v_mfma_f32_32x32x16_bf16 back to back, four independent accumulators per wave,
//           operands in registers (loaded once from the k and q buffers)
//   kind 1  tile loop, plain arrangement: per 32-row x 64-key wave tile 32 MFMAs (S0, S1, then P.V),
//           SiLU of the 32 scores a lane holds as 16 units in slots 9..24, 48 LDS fragment reads with
//           the kernel's swizzled addresses, 8 global -> LDS copies of the next tile, one barrier
//   kind 2  tile loop, skewed by one tile: every slot carries an MFMA and one score's SiLU stage
//           (second half of P.V of tile i - 1 | S1 of tile i | S0 of tile i + 1 | first half of P.V of
//           tile i), half-tile copies
//   kind 3  the skewed loop with 64 query rows per wave and one wave per SIMD (see hstu_calibration_loop64)
// `pieces` removes parts of kinds 1, 2 and 3 (bit 0: no SiLU, bit 1: no LDS fragment reads, bit 2: no
// copies, bit 3: no barrier); the results are then meaningless, only the time counts.
//
// Every workgroup (256 threads, two per CU) walks `tiles` key tiles of "its" (sequence, head) of the k
// and v buffers, laid out [rows, 4 heads, 128] bf16 like the operator's tensors; the caller chooses
// what the buffers hold (random values, zeros): the clock the chip grants depends on it.
// Wave 0 of every workgroup records the shader-clock and the constant-rate (100 MHz) counter around
// its loop, so that the caller sees both the cycles and the clock.
#pragma once
#include <type_traits>

#include "hstu_common.h"
#include "hstu_tiled_d128_dl.h"  // copy16, tile constants, LDS pointer types

namespace recir_hstu {

struct CalParams {
  const char* k;       // [rows, 4, 128] bf16
  const char* v;       // [rows, 4, 128] bf16
  const char* q;       // [>= 128, 4, 128] bf16: the query rows every workgroup holds
  float* sink;         // [grid * 256] keeps the arithmetic alive
  unsigned long long* stats;  // [grid][4]: shader-clock cycles and 100 MHz ticks of wave 0's loop, its start and end on the 100 MHz counter
  int tiles;           // key tiles per workgroup (even)
  int seq_tiles;       // key tiles of one pretended sequence in the buffers (rows / 64 / sequences)
  int sequences;       // pretended sequences in the buffers
  float neg_c;         // the SiLU multiplier, -alpha log2(e)
};

constexpr int CAL_NO_SILU = 1, CAL_NO_LDS_READS = 2, CAL_NO_COPIES = 4, CAL_NO_BARRIER = 8;

template <int KIND, int PIECES>
__global__ __launch_bounds__(256, 2) void hstu_calibration_loop(CalParams c) {
  constexpr bool SILU = !(PIECES & CAL_NO_SILU), LDSR = !(PIECES & CAL_NO_LDS_READS);
  constexpr bool COPY = !(PIECES & CAL_NO_COPIES), BAR = !(PIECES & CAL_NO_BARRIER);
  __shared__ __attribute__((aligned(1024))) unsigned short Ks0[BN * HD];
  __shared__ __attribute__((aligned(1024))) unsigned short Ks1[BN * HD];
  __shared__ __attribute__((aligned(1024))) unsigned short Vs0[BN * HD];
  __shared__ __attribute__((aligned(1024))) unsigned short Vs1[BN * HD];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, half = lane >> 5;
  constexpr unsigned row_bytes = 4 * HD * 2;
  const int seq = (int)(blockIdx.x % (unsigned)c.sequences), h = (int)((blockIdx.x / (unsigned)c.sequences) & 3);
  const char* kgb = c.k + ((size_t)seq * c.seq_tiles * BN * 4 + h) * (HD * 2);
  const char* vgb = c.v + ((size_t)seq * c.seq_tiles * BN * 4 + h) * (HD * 2);

  // the forward kernel's LDS access patterns (64-bank swizzles)
  const unsigned ks_rd = (unsigned)l32 * (HD * 2) + (unsigned)((half ^ (l32 & 15)) * 16);
  const int tr_s = lane & 15, tr_r = tr_s >> 2, tr_c = tr_s & 3, tr_dgrp = (lane >> 4) & 1;
  const unsigned vt_rd = (unsigned)(4 * half + tr_r) * (HD * 2) + (unsigned)tr_r * 64u + (unsigned)tr_dgrp * 32u + (unsigned)tr_c * 8u;
  const int ld_row = lane >> 4, ld_chunk = lane & 15;
  const unsigned k_off = (unsigned)ld_row * row_bytes + (unsigned)((ld_chunk ^ ld_row) * 16);
  const unsigned v_off = (unsigned)ld_row * row_bytes + (unsigned)((ld_chunk ^ (4 * ld_row)) * 16);

  // query fragments (B operand) and, for the builds without LDS reads, stand-in A fragments
  bf16x8 qf[8], kfr[8];
  {
    const unsigned short* qrow = (const unsigned short*)c.q + ((size_t)(wave * 32 + l32) * 4 + h) * HD;
    const unsigned short* krow = (const unsigned short*)kgb + (size_t)(wave * 32 + l32) * 4 * HD;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      qf[kk] = __builtin_bit_cast(bf16x8, *(const u32x4*)(qrow + kk * 16 + half * 8));
      kfr[kk] = __builtin_bit_cast(bf16x8, *(const u32x4*)(krow + kk * 16 + half * 8));
    }
  }
  f32x16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  const f32x16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const float neg_c = c.neg_c;

  // copy instruction `part` (0..7) of tile `it` into LDS stage `stage`: K (even part) or V (odd) rows 16 wave + 4 (part >> 1) ..
  auto copy_part = [&](int it, int stage, int part) __attribute__((always_inline)) {
    if constexpr (!COPY) return;
    const int k0 = (it % c.seq_tiles) * BN;
    const int ps = part >> 1;
    const int r0 = 4 * (4 * wave + ps);
    unsigned short* Kd = stage ? Ks1 : Ks0;
    unsigned short* Vd = stage ? Vs1 : Vs0;
    if (!(part & 1)) copy16(kgb + (size_t)(k0 + r0) * row_bytes, k_off ^ (unsigned)(64 * (ps & 3)), (unsigned)(size_t)&Kd[r0 * HD]);
    else copy16(vgb + (size_t)(k0 + r0) * row_bytes, v_off, (unsigned)(size_t)&Vd[r0 * HD]);
  };
  // the skewed loop's half-tile copies of trip i (stage BUF = i & 1): parts 0, 1 K rows 0..31 of tile i + 2 (stage BUF);
  // 2, 3 K rows 32..63 of tile i + 1 (other stage); 4, 5 V rows 0..31 of tile i + 1 (other stage); 6, 7 V rows 32..63
  // of tile i (stage BUF); this wave moves rows 8 wave + 4 (part & 1) .. + 3 of the half tile
  auto skew_copy = [&](int i, int BUF, int part) __attribute__((always_inline)) {
    if constexpr (!COPY) return;
    const int idx = part & 1, sel = part >> 1;
    const bool is_v = sel >= 2, hi = (sel & 1) != 0, to_cur = (sel == 0 || sel == 3);
    const int tile = (sel == 0 ? i + 2 : (sel == 3 ? i : i + 1)) % c.seq_tiles;
    const int stage = to_cur ? BUF : (BUF ^ 1);
    const int jr = 8 * (int)hi + 2 * wave + idx;
    const int r0 = 4 * jr;
    unsigned short* dst = is_v ? (stage ? Vs1 : Vs0) : (stage ? Ks1 : Ks0);
    const char* src = (is_v ? vgb : kgb) + (size_t)(tile * BN + r0) * row_bytes;
    const unsigned off = is_v ? v_off : (k_off ^ (unsigned)(64 * (jr & 3)));
    copy16(src, off, (unsigned)(size_t)&dst[r0 * HD]);
  };
  auto tile_sync = [&]() __attribute__((always_inline)) {
    if constexpr (BAR) { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); __syncthreads(); }
  };
  auto k_frag = [&](int stage, int kvb, int kk) __attribute__((always_inline)) {
    const char* kb = (const char*)(stage ? Ks1 : Ks0);
    if constexpr (!LDSR) return kfr[(kk + kvb) & 7];
    else return *(const bf16x8*)(kb + kvb * 32 * HD * 2 + (ks_rd ^ (unsigned)(kk * 32)));
  };
  auto v_frag = [&](int stage, int db, int s2) __attribute__((always_inline)) {
    const char* vb = (const char*)(stage ? Vs1 : Vs0);
    if constexpr (!LDSR) return kfr[(db + s2) & 7];
    else {
      const char* a = vb + (vt_rd ^ (unsigned)(db * 64)) + s2 * 16 * HD * 2;
      const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)a);
      const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(a + 8 * HD * 2));
      const i16x8 both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      return __builtin_bit_cast(bf16x8, both);
    }
  };

  // first tile resident before the clock starts
  if (KIND != 0) {
    for (int part = 0; part < 8; ++part) { copy_part(0, 0, part); copy_part(1, 1, part); }  // (the skewed loop starts with both stages filled)
    if (!COPY) {
      for (int i = tid; i < BN * HD; i += 256) { Ks0[i] = ((const unsigned short*)c.k)[i]; Ks1[i] = ((const unsigned short*)c.k)[i + BN * HD];
                                                 Vs0[i] = ((const unsigned short*)c.v)[i]; Vs1[i] = ((const unsigned short*)c.v)[i + BN * HD]; }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }

  f32x16 sblk[2] = {zero, zero};
  unsigned pw[2][8];
#pragma unroll
  for (int i = 0; i < 8; ++i) pw[0][i] = pw[1][i] = 0u;
  float sk_t[8], sk_r[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) sk_t[i] = sk_r[i] = 0.f;

  // plain arrangement: the forward kernel's slot schedule of an unmasked tile
  auto tile_plain = [&](auto buf_tag, int it) __attribute__((always_inline)) {
    constexpr int BUF = decltype(buf_tag)::value;
    constexpr int PDK = 6, PDV = 10;
    bf16x8 F[32];
    auto frag_req = [](int s) constexpr { return s < PDK ? -1 : (s < 16 ? s - PDK : (s - PDV > 0 ? s - PDV : 0)); };
    auto slot_frag = [&](int s) __attribute__((always_inline)) { return s < 16 ? k_frag(BUF, s >> 3, s & 7) : v_frag(BUF, (s - 16) & 3, (s - 16) >> 2); };
#pragma unroll
    for (int s = 0; s < 32; ++s)
      if (frag_req(s) < 0) F[s] = slot_frag(s);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < 32; ++s) {
#pragma unroll
      for (int u = s + 1; u < 32; ++u)
        if (frag_req(u) == s) F[u] = slot_frag(u);
      __builtin_amdgcn_s_setprio(1);
      if (s < 16) {
        sblk[s >> 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F[s], qf[s & 7], (s & 7) == 0 ? zero : sblk[s >> 3], 0, 0, 0);
      } else {
        const int s2 = (s - 16) >> 2, db = s & 3;
        const u32x4 w = {pw[s2 >> 1][4 * (s2 & 1)], pw[s2 >> 1][4 * (s2 & 1) + 1], pw[s2 >> 1][4 * (s2 & 1) + 2], pw[s2 >> 1][4 * (s2 & 1) + 3]};
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F[s], __builtin_bit_cast(bf16x8, w), acc[db], 0, 0, 0);
      }
      __builtin_amdgcn_s_setprio(0);
      if (s < 8) copy_part(it + 1, BUF ^ 1, s);
      if (s >= 9 && s < 25) {
        const int u = s - 9, blk = u >> 3, e = u & 7;
        if constexpr (SILU) {
          float pe[2];
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const float tv = sblk[blk][2 * e + t] * neg_c;
            pe[t] = tv * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(tv));
          }
          pw[blk][e] = pack_bf16x2(pe[0], pe[1]);
        } else {
          pw[blk][e] = __float_as_uint(sblk[blk][2 * e]) ^ __float_as_uint(sblk[blk][2 * e + 1]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // skewed arrangement: the forward kernel's steady trip
  auto tile_skew = [&](auto buf_tag, int it) __attribute__((always_inline)) {
    constexpr int BUF = decltype(buf_tag)::value;
    constexpr int PD = 3;
    bf16x8 F[32];
    auto slot_frag = [&](int s) __attribute__((always_inline)) {
      if (s < 8) return v_frag(BUF ^ 1, s & 3, 2 + (s >> 2));
      if (s < 16) return k_frag(BUF, 1, s - 8);
      if (s < 24) return k_frag(BUF ^ 1, 0, s - 16);
      return v_frag(BUF, (s - 24) & 3, (s - 24) >> 2);
    };
    auto silu_stage = [&](int s, int stage) __attribute__((always_inline)) {
      const int n = s - (stage - 1);
      const int nn = (n + 32) & 31, e = nn & 7;
      if (stage == 1) sk_t[e] = (nn < 16 ? sblk[0][nn] : sblk[1][nn - 16]) * neg_c;
      else if (stage == 2) sk_r[e] = __builtin_amdgcn_exp2f(sk_t[e]);
      else if (stage == 3) sk_r[e] = 1.0f + sk_r[e];
      else if (stage == 4) sk_r[e] = __builtin_amdgcn_rcpf(sk_r[e]);
      else {
        sk_t[e] = sk_t[e] * sk_r[e];
        if (nn & 1) {
          const unsigned w = pack_bf16x2(sk_t[e - 1], sk_t[e]);
          if (nn < 16) pw[0][nn >> 1] = w; else pw[1][(nn - 16) >> 1] = w;
        }
      }
    };
#pragma unroll
    for (int s = 0; s < PD; ++s) F[s] = slot_frag(s);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < 32; ++s) {
      if (s + PD < 32) F[s + PD] = slot_frag(s + PD);
      if (s < 8) {
        const int w0 = 4 * (s >> 2), db = s & 3;
        const u32x4 w = {pw[1][w0], pw[1][w0 + 1], pw[1][w0 + 2], pw[1][w0 + 3]};
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F[s], __builtin_bit_cast(bf16x8, w), acc[db], 0, 0, 0);
      } else if (s < 16) {
        sblk[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F[s], qf[s - 8], s == 8 ? zero : sblk[1], 0, 0, 0);
      } else if (s < 24) {
        sblk[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F[s], qf[s - 16], s == 16 ? zero : sblk[0], 0, 0, 0);
      } else {
        const int w0 = 4 * ((s - 24) >> 2), db = (s - 24) & 3;
        const u32x4 w = {pw[0][w0], pw[0][w0 + 1], pw[0][w0 + 2], pw[0][w0 + 3]};
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F[s], __builtin_bit_cast(bf16x8, w), acc[db], 0, 0, 0);
      }
      if (s < 8) skew_copy(it, BUF, s);
      if constexpr (SILU) {
#pragma unroll
        for (int stage = 5; stage >= 1; --stage) silu_stage(s, stage);
      } else if (s & 1) {
        pw[s >> 4][(s & 15) >> 1] = __float_as_uint(sblk[s >> 4][s & 15]) ^ __float_as_uint(sblk[s >> 4][(s & 15) - 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  const unsigned long long w0 = wall_clock64();
  const long long c0 = clock64();
  if constexpr (KIND == 0) {
    for (int it = 0; it < c.tiles; ++it) {
#pragma unroll
      for (int s = 0; s < 32; ++s)
        acc[s & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kfr[s & 7], qf[(s >> 2) & 7], acc[s & 3], 0, 0, 0);
    }
  } else {
    for (int it = 0; it < c.tiles; it += 2) {
      if constexpr (KIND == 1) {
        tile_plain(std::integral_constant<int, 0>{}, it); tile_sync();
        tile_plain(std::integral_constant<int, 1>{}, it + 1); tile_sync();
      } else {
        tile_skew(std::integral_constant<int, 0>{}, it); tile_sync();
        tile_skew(std::integral_constant<int, 1>{}, it + 1); tile_sync();
      }
    }
  }
  const long long c1 = clock64();
  const unsigned long long w1 = wall_clock64();
  if (tid == 0) {
    c.stats[4 * blockIdx.x] = (unsigned long long)(c1 - c0); c.stats[4 * blockIdx.x + 1] = w1 - w0;
    c.stats[4 * blockIdx.x + 2] = w0; c.stats[4 * blockIdx.x + 3] = w1;
  }
  float s = 0.f;
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int i = 0; i < 16; ++i) s += acc[g][i];
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int i = 0; i < 16; ++i) s += sblk[g][i];
#pragma unroll
  for (int i = 0; i < 8; ++i) s += __uint_as_float(pw[0][i]) + __uint_as_float(pw[1][i]) + sk_t[i] + sk_r[i];
  c.sink[(size_t)blockIdx.x * 256 + tid] = s;
}

// kind 3: the skewed tile loop with 64 query rows per wave (two 32-row blocks), one workgroup of four
// waves per CU and one wave per SIMD: every K and V^T fragment read from LDS feeds two MFMAs, which
// halves the LDS fragment bytes per MFMA; the 128 output accumulators of a wave live in fixed
// accumulation registers a[0:127] (as variables the register allocator moves them about).  Same
// FLOPs per CU and tile round as two workgroups of kinds 1 and 2.  A design the attention kernel does
// not use; here to price it on the same operands.
#define RECIR_CAL_ACC_CASE(T, LO, HI) \
  case T: asm volatile("v_mfma_f32_32x32x16_bf16 a[" #LO ":" #HI "], %0, %1, a[" #LO ":" #HI "]" ::"v"(a), "v"(b)); break;
__device__ __forceinline__ void cal_acc_mfma(int t, bf16x8 a, bf16x8 b) {
  switch (t) {
    RECIR_CAL_ACC_CASE(0, 0, 15) RECIR_CAL_ACC_CASE(1, 16, 31) RECIR_CAL_ACC_CASE(2, 32, 47) RECIR_CAL_ACC_CASE(3, 48, 63)
    RECIR_CAL_ACC_CASE(4, 64, 79) RECIR_CAL_ACC_CASE(5, 80, 95) RECIR_CAL_ACC_CASE(6, 96, 111) RECIR_CAL_ACC_CASE(7, 112, 127)
  }
}
#undef RECIR_CAL_ACC_CASE
template <int I, int N, class F>
__device__ __forceinline__ void cal_static_for(F&& f) {
  if constexpr (I < N) { f(std::integral_constant<int, I>{}); cal_static_for<I + 1, N>(f); }
}

template <int PIECES>
__global__ __launch_bounds__(256, 1) void hstu_calibration_loop64(CalParams c) {
  constexpr bool SILU = !(PIECES & CAL_NO_SILU), LDSR = !(PIECES & CAL_NO_LDS_READS);
  constexpr bool COPY = !(PIECES & CAL_NO_COPIES), BAR = !(PIECES & CAL_NO_BARRIER);
  constexpr int PD = 4;
  __shared__ __attribute__((aligned(1024))) unsigned short Ks0[BN * HD];
  __shared__ __attribute__((aligned(1024))) unsigned short Ks1[BN * HD];
  __shared__ __attribute__((aligned(1024))) unsigned short Vs0[BN * HD];
  __shared__ __attribute__((aligned(1024))) unsigned short Vs1[BN * HD];
  __shared__ char one_per_cu[36 * 1024];  // with the tiles above: more than half of a CU's LDS
  if (c.tiles < 0) one_per_cu[threadIdx.x] = 1;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, half = lane >> 5;
  constexpr unsigned row_bytes = 4 * HD * 2;
  const int seq = (int)(blockIdx.x % (unsigned)c.sequences), h = (int)((blockIdx.x / (unsigned)c.sequences) & 3);
  const char* kgb = c.k + ((size_t)seq * c.seq_tiles * BN * 4 + h) * (HD * 2);
  const char* vgb = c.v + ((size_t)seq * c.seq_tiles * BN * 4 + h) * (HD * 2);
  const unsigned ks_rd = (unsigned)l32 * (HD * 2) + (unsigned)((half ^ (l32 & 15)) * 16);
  const int tr_s = lane & 15, tr_r = tr_s >> 2, tr_c = tr_s & 3, tr_dgrp = (lane >> 4) & 1;
  const unsigned vt_rd = (unsigned)(4 * half + tr_r) * (HD * 2) + (unsigned)tr_r * 64u + (unsigned)tr_dgrp * 32u + (unsigned)tr_c * 8u;
  const int ld_row = lane >> 4, ld_chunk = lane & 15;
  const unsigned k_off = (unsigned)ld_row * row_bytes + (unsigned)((ld_chunk ^ ld_row) * 16);
  const unsigned v_off = (unsigned)ld_row * row_bytes + (unsigned)((ld_chunk ^ (4 * ld_row)) * 16);

  bf16x8 qf[2][8], kfr[8];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const unsigned short* qrow = (const unsigned short*)c.q + ((size_t)((wave * 64 + b * 32 + l32) & 127) * 4 + h) * HD;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qf[b][kk] = __builtin_bit_cast(bf16x8, *(const u32x4*)(qrow + kk * 16 + half * 8));
  }
  {
    const unsigned short* krow = (const unsigned short*)kgb + (size_t)(wave * 32 + l32) * 4 * HD;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) kfr[kk] = __builtin_bit_cast(bf16x8, *(const u32x4*)(krow + kk * 16 + half * 8));
  }
  asm volatile("" ::: "a0", "a127");  // the accumulation registers are this kernel's by hand
  const float neg_c = c.neg_c;
  f32x16 sb[2][2];  // [key half][query block]
  unsigned pw[2][2][8];
  float sk_t[8], sk_r[8];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int i = 0; i < 16; ++i) sb[a][b][i] = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) pw[a][b][i] = 0u;
    }
#pragma unroll
  for (int i = 0; i < 8; ++i) sk_t[i] = sk_r[i] = 0.f;

  auto k_frag = [&](int stage, int kvb, int kk) __attribute__((always_inline)) {
    const char* kb = (const char*)(stage ? Ks1 : Ks0);
    if constexpr (!LDSR) return kfr[(kk + kvb) & 7];
    else return *(const bf16x8*)(kb + kvb * 32 * HD * 2 + (ks_rd ^ (unsigned)(kk * 32)));
  };
  auto v_frag = [&](int stage, int db, int s2) __attribute__((always_inline)) {
    const char* vb = (const char*)(stage ? Vs1 : Vs0);
    if constexpr (!LDSR) return kfr[(db + s2) & 7];
    else {
      const char* a = vb + (vt_rd ^ (unsigned)(db * 64)) + s2 * 16 * HD * 2;
      const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)a);
      const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(a + 8 * HD * 2));
      const i16x8 both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      return __builtin_bit_cast(bf16x8, both);
    }
  };
  // 16 copy instructions per wave and tile (four waves move the 32 KB of K and V)
  auto copy_part = [&](int it, int stage, int part) __attribute__((always_inline)) {
    if constexpr (!COPY) return;
    const int k0 = (it % c.seq_tiles) * BN;
    const int ps = part >> 1;
    const int r0 = 4 * (4 * wave + (ps & 3));
    unsigned short* Kd = stage ? Ks1 : Ks0;
    unsigned short* Vd = stage ? Vs1 : Vs0;
    if (!(part & 1)) copy16(kgb + (size_t)(k0 + r0) * row_bytes, k_off ^ (unsigned)(64 * (ps & 3)), (unsigned)(size_t)&Kd[r0 * HD]);
    else copy16(vgb + (size_t)(k0 + r0) * row_bytes, v_off, (unsigned)(size_t)&Vd[r0 * HD]);
  };
  for (int part = 0; part < 8; ++part) { copy_part(0, 0, part); copy_part(1, 1, part); }
  if (!COPY) {
    for (int i = tid; i < BN * HD; i += 256) { Ks0[i] = ((const unsigned short*)c.k)[i]; Ks1[i] = ((const unsigned short*)c.k)[i + BN * HD];
                                               Vs0[i] = ((const unsigned short*)c.v)[i]; Vs1[i] = ((const unsigned short*)c.v)[i + BN * HD]; }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // one tile: 32 fragments, each feeding the two query blocks (64 slots); groups of 16 slots in the skewed order
  auto tile = [&](auto buf_tag, int it) __attribute__((always_inline)) {
    constexpr int BUF = decltype(buf_tag)::value;
    bf16x8 F[32];
    auto slot_frag = [&](int f) __attribute__((always_inline)) {
      const int g = f >> 3, j = f & 7;
      if (g == 0) return v_frag(BUF ^ 1, j & 3, 2 + (j >> 2));
      if (g == 1) return k_frag(BUF, 1, j);
      if (g == 2) return v_frag(BUF, j & 3, j >> 2);
      return k_frag(BUF ^ 1, 0, j);
    };
#pragma unroll
    for (int f = 0; f < PD; ++f) F[f] = slot_frag(f);
    __builtin_amdgcn_sched_barrier(0);
    cal_static_for<0, 64>([&](auto S_) __attribute__((always_inline)) {
      constexpr int s = decltype(S_)::value;
      constexpr int f = s >> 1, qb = s & 1, g = f >> 3, j = f & 7;
      if constexpr (qb == 0 && f + PD < 32) F[f + PD] = slot_frag(f + PD);
      if (g == 0 || g == 2) {
        const int ks = (g == 0 ? 2 : 0) + (j >> 2), db = j & 3, blk = g == 0 ? 1 : 0;
        const u32x4 w = {pw[blk][qb][4 * (ks & 1)], pw[blk][qb][4 * (ks & 1) + 1], pw[blk][qb][4 * (ks & 1) + 2], pw[blk][qb][4 * (ks & 1) + 3]};
        cal_acc_mfma(qb * 4 + db, F[f], __builtin_bit_cast(bf16x8, w));
      } else {
        f32x16& d = sb[g == 1 ? 1 : 0][qb];
        const bf16x8 fa = F[f], fb = qf[qb][j];
        if (j == 0) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(fa), "v"(fb));
        else asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(fa), "v"(fb));
      }
      if (s < 32 && !(s & 1)) copy_part(it + 2, ((s >> 2) & 1) ? BUF : (BUF ^ 1), s >> 1);
      if constexpr (SILU) {
        // one score per slot through five stages (scores 0..31 of the lane: key half 0, 32..63: key half 1)
#define RECIR_CAL_SB(sc) sb[(sc) >> 5][((sc) >> 4) & 1][(sc) & 15]
        constexpr int n5 = (s + 60) & 63, n4 = (s + 61) & 63, n3 = (s + 62) & 63, n2 = (s + 63) & 63, n1 = s;
        sk_t[n5 & 7] = sk_t[n5 & 7] * sk_r[n5 & 7];
        if (n5 & 1) pw[n5 >> 5][(n5 >> 4) & 1][(n5 & 15) >> 1] = pack_bf16x2(sk_t[(n5 - 1) & 7], sk_t[n5 & 7]);
        sk_r[n4 & 7] = __builtin_amdgcn_rcpf(sk_r[n4 & 7]);
        sk_r[n3 & 7] = 1.0f + sk_r[n3 & 7];
        sk_r[n2 & 7] = __builtin_amdgcn_exp2f(sk_t[n2 & 7]);
        sk_t[n1 & 7] = RECIR_CAL_SB(n1) * neg_c;
#undef RECIR_CAL_SB
      } else if (s & 1) {
        pw[s >> 5][(s >> 4) & 1][(s & 15) >> 1] = __float_as_uint(sb[s >> 5][(s >> 4) & 1][s & 15]) ^ __float_as_uint(sb[s >> 5][(s >> 4) & 1][(s & 15) - 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  const unsigned long long w0 = wall_clock64();
  const long long c0 = clock64();
  for (int it = 0; it < c.tiles; it += 2) {
    tile(std::integral_constant<int, 0>{}, it);
    if constexpr (BAR) { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); __syncthreads(); }
    tile(std::integral_constant<int, 1>{}, it + 1);
    if constexpr (BAR) { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); __syncthreads(); }
  }
  const long long c1 = clock64();
  const unsigned long long w1 = wall_clock64();
  if (tid == 0) {
    c.stats[4 * blockIdx.x] = (unsigned long long)(c1 - c0); c.stats[4 * blockIdx.x + 1] = w1 - w0;
    c.stats[4 * blockIdx.x + 2] = w0; c.stats[4 * blockIdx.x + 3] = w1;
  }
  float r = 0.f;
  { float t0; asm volatile("s_nop 15\n\tv_accvgpr_read_b32 %0, a5" : "=v"(t0)); r += t0; }
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int i = 0; i < 16; ++i) r += sb[a][b][i];
#pragma unroll
      for (int i = 0; i < 8; ++i) r += __uint_as_float(pw[a][b][i]);
    }
#pragma unroll
  for (int i = 0; i < 8; ++i) r += sk_t[i] + sk_r[i];
  c.sink[(size_t)blockIdx.x * 256 + tid] = r;
}

}  // namespace recir_hstu
