// Tiled MFMA kernels of the HSTU attention backward, head dim 128 (qk and v), bf16 tensors,
// scalar or per-token output scale, optional relative score bias (read only: neither gets a gradient).
//
// Two kernels, as in the reference (recir/ops/pallas/jagged_hstu_attention.py:724-1339 and
// recir/ops/helion/jagged_hstu_attention.py:356-570): every gradient row has one writer.
//
//   hstu_bwd_dq_d128   one workgroup (4 waves x 32 query rows) per (sequence, head, 128-row query
//                      tile); walks the key tiles of 64 rows the forward walks.  Per 32-key block:
//                        S^T  = K Q^T        A = K rows from LDS,   B = Q (registers)
//                        dP^T = V dO^T       A = V rows from LDS,   B = dO (registers)
//                        dS^T = dP^T keep silu'(S^T), rounded to bf16 in registers: the 32 x 32
//                               accumulator layout is the B-operand layout of the next product
//                        dQ^T += K^T dS^T    A = K^T, transposing LDS read of the same K tile
//   hstu_bwd_dkv_d128  one workgroup (4 waves x 32 key rows) per (sequence, head, 128-row key tile);
//                      walks the query tiles of 64 rows that see those keys.  Per 32-query block:
//                        S  = Q K^T          A = Q rows from LDS,   B = K (registers)
//                        dP = dO V^T         A = dO rows from LDS,  B = V (registers)
//                        P  = silu(S) keep, dS = dP keep silu'(S), both rounded to bf16
//                        dV^T += dO^T P      A = dO^T, transposing LDS read of the dO tile
//                        dK^T += Q^T dS      A = Q^T, transposing LDS read of the Q tile
// The products run on the bf16 values as given; alpha (and log2(e), so that sigmoid needs exp2 only)
// multiply the fp32 score, alpha and the output scale are applied once to the fp32 accumulators.
// (Scaling an operand and rounding it back to bf16 perturbs every term of q.k by 2^-9 of itself:
// an error of the score that does not shrink with the score, visible in rows with one kept pair.)
//
// LDS tile layout, shared by all four staged matrices: [64 rows][256 bytes], 16-byte chunk c of row
// r stored at chunk c ^ f(r & 7) with f(r) = ((r & 3) << 1) | (r >> 2).  Eight consecutive rows then
// put one logical chunk on all banks (ds_read_b128 fragments), and four consecutive rows put one
// logical 32-byte slot on all banks (ds_read_b64_tr_b16 fragments), so both read patterns of a
// tile are free of bank conflicts on 32 banks.  (gfx950's LDS has 64: both patterns then run at half
// of its 256 bytes per clock.  The 16-row variant c ^ (((r & 3) << 2) | ((r >> 2) & 3)) removes that,
// but measured no faster and costs address registers, so the 8-row form stays.)
// Tiles travel HBM -> LDS with global_load_lds_dwordx4 (64 lanes
// x 16 bytes land on consecutive LDS addresses; the swizzle is applied to the address each lane
// fetches), two stages, one barrier per tile.
#pragma once
#include <type_traits>

#include "hstu_common.h"
#include "hstu_bwd_acc_regs.h"
#include "hstu_tiled_d128_dl.h"  // i16x4, i16x8, lds_void, lds_i16x4

#ifndef HSTU_BWD_DQ_PD
#define HSTU_BWD_DQ_PD 2  // (0: a measurement build of the dQ kernel with every fragment read right before its product)
#endif

namespace recir_hstu {

// Waves per SIMD the dQ kernel is compiled for.  Two fit once the phases of its tile body are fenced
// (the compiler otherwise hoists every fragment read to the top and spills).
#ifndef BWD_DQ_OCC
#define BWD_DQ_OCC 2
#endif
constexpr int BWD_BM = 128;  // rows a workgroup owns (query rows for dQ, key rows for dK/dV)
constexpr int BWD_BN = 64;   // rows of a staged tile
constexpr float kLn2 = 0.6931471805599453f;

// per-lane constants of the LDS access patterns
struct BwdLanes {
  unsigned rd;        // ds_read_b128 fragment: row l32 of a 32-row block, chunk (2 kk + half)
  unsigned tr_e;      // transposing fragment, even 32-column block
  unsigned tr_o;      // ... odd block
  int ld_row;         // row (0..3) and physical chunk a lane fills in one copy instruction
  int ld_chunk;
  unsigned ld_swz_e;  // logical chunk fetched for copy instructions with even / odd index
  unsigned ld_swz_o;
};

__device__ __forceinline__ BwdLanes bwd_lanes(int lane) {
  const int l32 = lane & 31, half = lane >> 5;
  BwdLanes c;
  const unsigned f = (unsigned)(((l32 & 3) << 1) | ((l32 >> 2) & 1));
  c.rd = (unsigned)l32 * 256u + (((unsigned)half ^ f) * 16u);
  // transposing read: source lane s = lane & 15 of a 16-lane group supplies the 8 bytes at row
  // 4 half + (s >> 2) (+ 16 per k-step + 8 for the second read) and columns
  // 32 db + 16 dgrp + 4 (s & 3) .. + 3; the row's swizzle value is ((s >> 2) << 1) | half
  const int s = lane & 15, tr_r = s >> 2, tr_c = s & 3, dgrp = (lane >> 4) & 1;
  const unsigned x = (unsigned)(2 * dgrp + (tr_c >> 1)) ^ (unsigned)((tr_r << 1) | half);
  const unsigned row = (unsigned)(4 * half + tr_r) * 256u + (unsigned)(tr_c & 1) * 8u;
  c.tr_e = row + x * 16u;
  c.tr_o = row + (x ^ 4u) * 16u - 64u;
  c.ld_row = lane >> 4;
  c.ld_chunk = lane & 15;
  c.ld_swz_e = (unsigned)(c.ld_chunk ^ (c.ld_row << 1));
  c.ld_swz_o = (unsigned)(c.ld_chunk ^ ((c.ld_row << 1) | 1));
  return c;
}

// A-operand fragment of rows [32 blk, 32 blk + 32) x columns [16 kk, 16 kk + 16) of a staged tile
__device__ __forceinline__ bf16x8 bwd_row_frag(const char* tile, const BwdLanes& c, int blk, int kk) {
  return *(const bf16x8*)(tile + blk * 32 * 256 + (c.rd ^ (unsigned)((kk & 3) * 32)) + (kk >> 2) * 128);
}

// A-operand fragment of the transposed tile: columns [32 db, 32 db + 32) x rows [16 s2, 16 s2 + 16)
__device__ __forceinline__ bf16x8 bwd_tr_frag(const char* tile, const BwdLanes& c, int db, int s2) {
  const char* a = tile + ((db & 1) ? c.tr_o : c.tr_e) + db * 64 + s2 * 16 * 256;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)a);
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(a + 8 * 256));
  const i16x8 both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, both);
}

// This wave's share (4 of 16 instructions) of the copy of rows [r_first, r_first + 64) of a
// [rows, H, 128] bf16 matrix into a staged tile.  Rows past `last` (relative to r_first) re-read
// row `last`; what they contribute is masked by the caller.
template <bool PIN_BASE>
__device__ __forceinline__ void bwd_issue_rows(const char* gbase, unsigned row_bytes, int last, unsigned short* tile,
                                               const BwdLanes& c, int wave) {
  // the base is the same for every lane; PIN_BASE says so where the compiler cannot prove it (the
  // copy takes it in scalar registers)
  const size_t gb = (size_t)gbase;
  if (PIN_BASE) gbase = (const char*)(((size_t)(unsigned)__builtin_amdgcn_readfirstlane((int)(gb >> 32)) << 32) |
                        (size_t)(unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)gb));
#pragma unroll
  for (int ps = 0; ps < 4; ++ps) {
    const int j = 4 * wave + ps;
    const int row = min(4 * j + c.ld_row, last);
    const unsigned chunk = (ps & 1) ? c.ld_swz_o : c.ld_swz_e;
    copy16(gbase, (unsigned)row * row_bytes + chunk * 16u, (unsigned)(size_t)&tile[j * 512]);
  }
}

// B-operand fragments of one [*, H, 128] bf16 row: columns 16 kk + 8 half .. + 7, optionally
// multiplied by `mul` and rounded back to bf16
__device__ __forceinline__ void bwd_load_row_frags(const void* base, size_t row, int H, int h, int half, bool valid,
                                                   bool scaled, float mul, bf16x8 (&f)[8]) {
  const unsigned short* src = (const unsigned short*)base + ((size_t)(valid ? row : 0) * H + h) * HD;
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  u32x4 t[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) t[kk] = valid ? *(const u32x4*)(src + kk * 16 + half * 8) : zero4;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    u32x4 sc = t[kk];
    if (scaled) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sc[i] = pack_bf16x2(__uint_as_float(t[kk][i] << 16) * mul, __uint_as_float(t[kk][i] & 0xffff0000u) * mul);
    }
    f[kk] = __builtin_bit_cast(bf16x8, sc);
  }
}

// largest bf16 magnitude (15 bits) among the 64 values a lane holds of a row
__device__ __forceinline__ unsigned bwd_frag_absmax(const bf16x8 (&f)[8]) {
  unsigned mx = 0;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    const u32x4 w = __builtin_bit_cast(u32x4, f[kk]);
#pragma unroll
    for (int i = 0; i < 4; ++i) mx = max(mx, max(w[i] & 0x7fffu, (w[i] >> 16) & 0x7fffu));
  }
  return mx;
}

__device__ __forceinline__ float bwd_output_scale(const Params& p) {
  return p.attn_scale ? p.attn_scale[0] : 1.0f / (float)p.N;
}

// Score bias in the tiled kernels.  The copies of a tile are assembly the compiler cannot count, so
// every wait it inserts for a load of its own waits for the copies in flight as well: bias values
// fetched from global memory inside a tile body would expose a copy round trip per tile.  Instead
// the 191 entries rab[h, m - j + N - 1] one (128-row, 64-row) tile pair can touch are staged in LDS,
// two stages like the tiles: the load goes out before the tile's copies, the store (scaled by
// log2(e), index clamped to the row) follows at the end of the tile, where everything is waited for
// anyway; the bias joins the fp32 score in the fused multiply-add that applies alpha * log2(e).
constexpr int BWD_BAND = BWD_BM + BWD_BN;  // 191 used
constexpr int BWD_DKV_WG_PER_XCD = 32;     // the key-tile kernel runs one workgroup per CU
__device__ __forceinline__ float bwd_band_load(const float* __restrict__ rab_row, int rab_w, int first_idx, int tid) {
  return rab_row[min(max(first_idx + tid, 0), rab_w - 1)];
}
// REVERSED: entry 190 - i holds index first + i, for the kernel whose elements run over keys (the
// index falls with the key): a lane's elements then sit at ascending addresses.
template <bool REVERSED>
__device__ __forceinline__ void bwd_band_store(float* band, float val, int tid, float mul) {
  asm volatile("" : "+v"(val));  // first use of the loaded value: the wait for it stays here
  if (tid < BWD_BAND - 1) band[REVERSED ? (BWD_BAND - 2) - tid : tid] = val * mul;
}

// ---------------------------------------------------------------------------------------------
// dQ
// ---------------------------------------------------------------------------------------------
// SEMI: semi-local mask (max_attn_len > 0), as in the forward kernel.
// HAS_RAB: scores carry the relative bias rab[h, query - key + N - 1] (no gradient flows to it).
// PER_TOKEN: the output scale is a [T] vector; P and dS of query row m carry attn_scale[m].
// RAB_GRAD (with HAS_RAB): also the gradient of the bias table, drab[h, m - j + N - 1] += dS(m, j).
//   The dS of a tile are added, as fixed-point integers, into an LDS band with the bias band's own
//   indexing (ds_add_u32; the elements one instruction adds lie on different diagonals up to a
//   two-way overlap of the lane halves), and the band of a finished tile is flushed to global
//   memory with one float atomic per diagonal while the next tile computes into the other stage.
//   The flush sums floats in arrival order: not bitwise reproducible, unlike dq, dk and dv.
template <bool SEMI, bool HAS_RAB, bool PER_TOKEN, bool RAB_GRAD = false>
__global__ __launch_bounds__(256, BWD_DQ_OCC) void hstu_bwd_dq_d128(BwdParams bp) {
  const Params& p = bp.f;
  __shared__ __attribute__((aligned(1024))) unsigned short Ks0[BWD_BN * HD];
  __shared__ __attribute__((aligned(1024))) unsigned short Ks1[BWD_BN * HD];
  __shared__ __attribute__((aligned(1024))) unsigned short Vs0[BWD_BN * HD];
  __shared__ __attribute__((aligned(1024))) unsigned short Vs1[BWD_BN * HD];
  __shared__ float band0[HAS_RAB ? BWD_BAND : 1];
  __shared__ float band1[HAS_RAB ? BWD_BAND : 1];
  __shared__ float gband0[RAB_GRAD ? BWD_BAND : 1];
  __shared__ float gband1[RAB_GRAD ? BWD_BAND : 1];
  static_assert(!RAB_GRAD || HAS_RAB, "the bias gradient needs the bias");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int half = lane >> 5;
  const BwdLanes lc = bwd_lanes(lane);

  zero_tail_rows_of<256>(p, bp.dq, (size_t)p.H * HD * 2);
  if (RAB_GRAD && tid < BWD_BAND) { gband0[tid] = 0.f; gband1[tid] = 0.f; }  // published by the first tile's barrier
  // Gradient of the bias table: the sums along the diagonals are kept in LDS as fixed-point integers.  An LDS float atomic takes three cycles per lane, one lane at a time
  // (192 cycles for a wave's instruction), an integer one 4-16 cycles for the whole instruction.  The
  // scale is a power of two per head, the same for every item of the call (drab_fx_bound): the tile
  // sums are flushed as 64-bit integer additions to a table of the same scale, so the result does not
  // depend on the order in which tiles and workgroups arrive, and a last kernel turns the table into
  // floats.  What the conversion drops is below 2^-30 of the bound per pair, rounded to nearest.
  // Non-finite inputs make the scale zero and every value of the head NaN.
  constexpr bool FIXED = RAB_GRAD;
  float fx_scale = 0.f, fx_inv = 0.f;

  const int xcd = blockIdx.x % NUM_XCD;
  const int list_len = p.ws_counts[xcd];
  const WorkItem* __restrict__ list = p.ws_items + (size_t)xcd * p.items_cap;
  for (int slot = blockIdx.x / NUM_XCD; slot < list_len; slot += p.grid_slots) {
    const WorkItem wi = list[slot];
    SeqInfo si;
    si.s = wi.s; si.n = wi.n; si.cap = wi.cap; si.ctx_eff = wi.ctx_eff;
    si.win = WIN_ALL; si.tail0 = 0x7fffffff;
    if (SEMI) mask_window(p, si.cap, si.win, si.tail0);
    const int q0 = wi.q0;
    const int q_end = wi.q_end;  // rows [q0, q_end) belong to this item
    const int h = wi.h;
    const unsigned row_bytes = (unsigned)p.H * HD * 2u;
    const char* __restrict__ kgb = (const char*)p.k + ((size_t)si.s * p.H + h) * (HD * 2);
    const char* __restrict__ vgb = (const char*)p.v + ((size_t)si.s * p.H + h) * (HD * 2);
    const int rab_w = 2 * p.N - 1;
    const float* __restrict__ rab_row = HAS_RAB ? p.rab + (size_t)h * rab_w : nullptr;

    const int qw0 = q0 + wave * 32;
    const int m = qw0 + l32;
    const int m_lo = qw0;
    const int m_hi = min(qw0 + 31, q_end - 1);
    const bool wave_has_rows = m_lo < q_end;
    const int idm = min(m, si.cap);
    const bool tail_row = idm >= si.tail0;
    const int idlo_w = min(m_lo, si.cap), idhi_w = min(m_hi, si.cap);
    const bool wave_has_tail = idhi_w >= si.tail0;
    // causal mask of this lane's row as bounds on the key index (key k0 + 4 half + c, c a
    // compile-time constant per element): kept iff j < max(min(idm, n), min(ctx_eff, n)) or j == m
    const int mk_eq = (m < si.n ? m : -0x40000000) - 4 * half;
    const int mk_top = max(min(idm, si.n), min(si.ctx_eff, si.n)) - 4 * half;

    // key tiles [0, nkv) minus the run [skip_a, skip_b) that holds only target keys off this query
    // tile's diagonal (and no contextual key): the tiles the forward walks
    const int kv_end = min(si.n, max(q_end, si.ctx_eff));
    const int nkv = (kv_end + BWD_BN - 1) / BWD_BN;
    const int cap0 = si.cap > 0 ? si.cap : 0;
    const int skip_a = (max(cap0, si.ctx_eff) + BWD_BN - 1) / BWD_BN;
    const int skip_b = q0 / BWD_BN;
    const bool has_skip = skip_a < skip_b;
    auto next_tile = [&](int it) { return (has_skip && it + 1 == skip_a) ? skip_b : it + 1; };

    auto issue_tile = [&](int it, auto buf_tag) __attribute__((always_inline)) {
      constexpr int BUF = decltype(buf_tag)::value;
      const int k0 = it * BWD_BN;
      const int last = si.n - 1 - k0;
      bwd_issue_rows<HAS_RAB>(kgb + (size_t)k0 * row_bytes, row_bytes, last, BUF ? Ks1 : Ks0, lc, wave);
      bwd_issue_rows<HAS_RAB>(vgb + (size_t)k0 * row_bytes, row_bytes, last, BUF ? Vs1 : Vs0, lc, wave);
    };

    // The band is staged reversed: the entry for this lane's row and the key at offset 4 half + c of
    // a tile is at byte 4 (127 - (m - q0) + 4 half + c) of the stage, ascending with c.  The lane
    // part is made opaque to the compiler, which otherwise forms an address register per pair of
    // elements and spills them.
    unsigned band_lane = 4u * (unsigned)(127 - (m - q0) + 4 * half);
    asm volatile("" : "+v"(band_lane));
    // bias band of key tile t: entry i is rab index q0 - 64 t - 63 + N - 1 + i
    auto band_of = [&](int t) __attribute__((always_inline)) {
      return bwd_band_load(rab_row, rab_w, q0 - t * BWD_BN - (BWD_BN - 1) + p.N - 1, tid);
    };
    int it0 = 0;  // semi-local: key tiles below the first row's window are not walked
    if (SEMI && si.ctx_eff <= 0 && min(q_end - 1, si.cap) < si.tail0) it0 = max(min(q0, si.cap) - si.win, 0) / BWD_BN;
    int it = (has_skip && it0 >= skip_a) ? max(it0, skip_b) : it0;
    float band_first = 0.f;
    if (HAS_RAB && it < nkv) band_first = band_of(it);
    if (it < nkv) issue_tile(it, std::integral_constant<int, 0>{});

    bf16x8 qf[8], gf[8];
    bwd_load_row_frags(p.q, (size_t)si.s + m, p.H, h, half, m < q_end, false, 1.0f, qf);
    // a per-token output scale multiplies row m of P, hence row m of dS (this lane's row)
    constexpr bool per_token = PER_TOKEN;
    const float row_scale = per_token ? p.attn_scale[si.s + min(m, si.n - 1)] : 1.0f;
    bwd_load_row_frags(bp.dout, (size_t)si.s + m, p.H, h, half, m < q_end, false, 1.0f, gf);
    const float score_c = p.alpha * kLog2e, neg_c = -score_c;
    // the bias is staged multiplied by log2(e) and joins the score in the multiply-add that applies alpha log2(e)
    const float bias_mul = kLog2e;
    // what the staged band is multiplied with: 0 for a diagonal outside the table (possible only in a
    // sequence longer than max_seq_len; the load clamps its index), which then has no bias
    auto band_mul_of = [&](int t) __attribute__((always_inline)) {
      return (unsigned)(q0 - t * BWD_BN - (BWD_BN - 1) + p.N - 1 + tid) < (unsigned)rab_w ? bias_mul : 0.f;
    };

    f32x16 acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
#if BWD_DQ_OCC == 1
      // the accumulators are MFMA operands only until the epilogue: start them out in the
      // accumulation registers
      asm volatile("" : "+a"(acc[i]));
#endif
    }

    // Semi-local mask of a history row (m < cap) against keys that are not contextual: key j is kept
    // iff m - win <= j <= m (0 <= j <= m for a row of the full-attention tail): one unsigned
    // comparison of j - lo with m - lo, as in the forward kernel
    const int rng_lo = tail_row ? 0 : m - si.win;
    const unsigned rng_w = (unsigned)(m - rng_lo);
    const int rng_lane = 4 * half - rng_lo;
    auto tile_body = [&](auto masked_tag, auto buf_tag, int k0) __attribute__((always_inline)) {
      constexpr int MASKED = decltype(masked_tag)::value;  // 0 none, 1 general predicate, 2 range of a history row
      const int rng_base = k0 + rng_lane;
      constexpr int BUF = decltype(buf_tag)::value;
      const char* kb = (const char*)(BUF ? Ks1 : Ks0);
      const char* vb = (const char*)(BUF ? Vs1 : Vs0);
      const unsigned band_addr = (unsigned)(size_t)(BUF ? band1 : band0) + band_lane;  // LDS byte address
      const f32x16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kvb = 0; kvb < 2; ++kvb) {
        f32x16 st = zero, dpt = zero;
        // phases are fenced so that the fragment reads of one are not hoisted over the previous one
        // (keeps the live registers within the two-waves-per-SIMD budget)
        __builtin_amdgcn_sched_barrier(0);
        constexpr int PD = HSTU_BWD_DQ_PD;  // fragments requested this many products ahead
        if constexpr (PD > 0) {
          auto frag = [&](int i) __attribute__((always_inline)) { return bwd_row_frag((i & 1) ? vb : kb, lc, kvb, i >> 1); };
          bf16x8 F[16];
#pragma unroll
          for (int i = 0; i < PD; ++i) F[i] = frag(i);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            if (i + PD < 16) F[i + PD] = frag(i + PD);
            if (i & 1) dpt = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F[i], gf[i >> 1], dpt, 0, 0, 0);
            else st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F[i], qf[i >> 1], st, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
          }
        } else {
#pragma unroll
          for (int kk = 0; kk < 8; ++kk) {
            st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bwd_row_frag(kb, lc, kvb, kk), qf[kk], st, 0, 0, 0);
            dpt = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bwd_row_frag(vb, lc, kvb, kk), gf[kk], dpt, 0, 0, 0);
            if (kk == 3) __builtin_amdgcn_sched_barrier(0);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        // dS^T = dP^T silu'(S^T) on the kept pairs; element r of the block is key
        // 32 kvb + 8 (r / 4) + 4 half + r % 4 for this lane's query row
        u32x4 w0, w1;
        float ds[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          // (the bias is added here, not taken as the accumulator's start as the dK/dV kernel does: by
          // now the fragment registers of the products are free, before them this kernel is at its
          // register limit; measured: 3 % slower at configuration 3, 9 % with the bias-table gradient)
          // silu'(x) = sig (1 + x (1 - sig)), x = alpha s (+ bias): without a bias alpha goes into
          // (1 - sig), so no instruction is spent on x itself
          float sig, inner;
          if (HAS_RAB) {
            const float u = __builtin_fmaf(st[r], score_c, *(lds_cfloat*)(band_addr + 4u * (unsigned)(kvb * 32 + 8 * (r >> 2) + (r & 3))));
            sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-u));
            inner = __builtin_fmaf(u, __builtin_fmaf(sig, -kLn2, kLn2), 1.0f);  // x (1 - sig) with x = u ln 2
          } else {
            sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(st[r] * neg_c));
            inner = __builtin_fmaf(st[r], __builtin_fmaf(sig, -p.alpha, p.alpha), 1.0f);
          }
          float g = dpt[r] * (sig * inner);
          if (per_token) g *= row_scale;
          if (MASKED == 1) {
            const int c = kvb * 32 + 8 * (r >> 2) + (r & 3);
            const int j = k0 + 4 * half + c;
            const bool kp = SEMI ? ((m == j) | ((j < idm) & ((idm - j <= si.win) | tail_row)) | (j < si.ctx_eff)) & (j < si.n)
                                 : ((c < mk_top - k0) | (c == mk_eq - k0));
            g = kp ? g : 0.f;
          }
          if (MASKED == 2) g = (unsigned)(rng_base + (kvb * 32 + 8 * (r >> 2) + (r & 3))) <= rng_w ? g : 0.f;
          ds[r] = g;
        }
        if constexpr (FIXED) {
          int* gi = (int*)(BUF ? gband1 : gband0) + (band_lane >> 2);
#pragma unroll
          for (int r = 0; r < 16; ++r)
            __hip_atomic_fetch_add(gi + (kvb * 32 + 8 * (r >> 2) + (r & 3)), __float2int_rn(ds[r] * fx_scale), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          w0[i] = pack_bf16x2(ds[2 * i], ds[2 * i + 1]);
          w1[i] = pack_bf16x2(ds[8 + 2 * i], ds[8 + 2 * i + 1]);
        }
        const bf16x8 b0 = __builtin_bit_cast(bf16x8, w0), b1 = __builtin_bit_cast(bf16x8, w1);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (PD > 0) {
          auto frag = [&](int i) __attribute__((always_inline)) { return bwd_tr_frag(kb, lc, i >> 1, 2 * kvb + (i & 1)); };
          bf16x8 F[8];
#pragma unroll
          for (int i = 0; i < PD; ++i) F[i] = frag(i);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            if (i + PD < 8) F[i + PD] = frag(i + PD);
            acc[i >> 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F[i], (i & 1) ? b1 : b0, acc[i >> 1], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
          }
        } else {
#pragma unroll
          for (int db = 0; db < 4; ++db) {
            acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bwd_tr_frag(kb, lc, db, 2 * kvb), b0, acc[db], 0, 0, 0);
            acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bwd_tr_frag(kb, lc, db, 2 * kvb + 1), b1, acc[db], 0, 0, 0);
            if (db == 1) __builtin_amdgcn_sched_barrier(0);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };

    auto compute_tile = [&](int itc, auto buf_tag) __attribute__((always_inline)) {
      const int k0 = itc * BWD_BN;
      const int k1 = k0 + BWD_BN;
      bool any_kept = wave_has_rows && ((k0 <= m_hi && k1 > m_lo) || (k0 < si.cap && k0 <= m_hi) ||
                                        (k0 < si.ctx_eff));
      if (SEMI)
        any_kept = wave_has_rows && ((k0 <= m_hi && k1 > m_lo) || (k0 < si.ctx_eff) ||
                                     (k0 < idhi_w && (wave_has_tail || k1 > idlo_w - si.win)));
      if (!any_kept) return;
      bool full = (k1 - 1 <= m_lo) && (k1 <= si.cap);  // implies k1 <= n
      if (SEMI) full = full && (idlo_w >= si.tail0 || k0 >= idhi_w - si.win);
      if (full) tile_body(std::integral_constant<int, 0>{}, buf_tag, k0);
      else if (SEMI && m_hi < si.cap && k0 >= si.ctx_eff) tile_body(std::integral_constant<int, 2>{}, buf_tag, k0);
      else tile_body(std::integral_constant<int, 1>{}, buf_tag, k0);
    };

    // Gradient band of a finished key tile t -> the head's fixed-point table (entry 190 - i of the
    // stage is rab index first + i, as in the bias band), and the stage is cleared for the tile after
    // the next.  Integer additions: the table does not depend on who arrives first.
    auto flush_gband = [&](int t, float* g) __attribute__((always_inline)) {
      if (tid < BWD_BAND - 1) {
        const int iv = __float_as_int(g[(BWD_BAND - 2) - tid]);
        g[(BWD_BAND - 2) - tid] = 0.f;
        const int idx = q0 - t * BWD_BN - (BWD_BN - 1) + p.N - 1 + tid;
        if (iv != 0 && idx >= 0 && idx < rab_w)
          atomicAdd((unsigned long long*)&bp.drab_fx[(size_t)h * rab_w + idx], (unsigned long long)(long long)iv);
      }
    };
    int prev_tile = -1;
    // two tiles per trip so that the stage index is a compile-time constant
    if (HAS_RAB && it < nkv) bwd_band_store<true>(band0, band_first, tid, band_mul_of(it));
    while (it < nkv) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's copies of tile `it` have landed
      __syncthreads();                                   // everybody's; the other stage is free again
      if constexpr (FIXED) {
        if (prev_tile < 0) drab_fx_scales(drab_fx_bound(bp, h, per_token), fx_scale, fx_inv);  // (the head's scale)
      }
      if (RAB_GRAD && prev_tile >= 0) flush_gband(prev_tile, gband1);
      int nxt = next_tile(it);
      float band_nxt = 0.f;
      if (HAS_RAB && nxt < nkv) band_nxt = band_of(nxt);
      if (nxt < nkv) issue_tile(nxt, std::integral_constant<int, 1>{});
      compute_tile(it, std::integral_constant<int, 0>{});
      if (HAS_RAB && nxt < nkv) bwd_band_store<true>(band1, band_nxt, tid, band_mul_of(nxt));
      prev_tile = it;
      it = nxt;
      if (it >= nkv) {
        if (RAB_GRAD) { __syncthreads(); flush_gband(prev_tile, gband0); }
        break;
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (RAB_GRAD) flush_gband(prev_tile, gband0);
      nxt = next_tile(it);
      if (HAS_RAB && nxt < nkv) band_nxt = band_of(nxt);
      if (nxt < nkv) issue_tile(nxt, std::integral_constant<int, 0>{});
      compute_tile(it, std::integral_constant<int, 1>{});
      if (HAS_RAB && nxt < nkv) bwd_band_store<true>(band0, band_nxt, tid, band_mul_of(nxt));
      prev_tile = it;
      it = nxt;
      if (RAB_GRAD && it >= nkv) { __syncthreads(); flush_gband(prev_tile, gband1); }
    }

    // dQ^T accumulators -> dq[s + m, h, :]; element 4 rq + i of block db is column 32 db + 8 rq + 4 half + i
    if (m < q_end) {
      const float oscale = per_token ? p.alpha : p.alpha * bwd_output_scale(p);
      unsigned short* orow = (unsigned short*)bp.dq + ((size_t)(si.s + m) * p.H + h) * HD;
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
    __syncthreads();  // LDS stages are reused by the next item
  }
}

// ---------------------------------------------------------------------------------------------
// dK, dV
// ---------------------------------------------------------------------------------------------
template <bool SEMI, bool HAS_RAB, bool PER_TOKEN>
__global__ __launch_bounds__(256, 1) void hstu_bwd_dkv_d128(BwdParams bp) {
  const Params& p = bp.f;
  __shared__ __attribute__((aligned(1024))) unsigned short Qs0[BWD_BN * HD];
  __shared__ __attribute__((aligned(1024))) unsigned short Qs1[BWD_BN * HD];
  __shared__ __attribute__((aligned(1024))) unsigned short Gs0[BWD_BN * HD];
  __shared__ __attribute__((aligned(1024))) unsigned short Gs1[BWD_BN * HD];
  __shared__ float band0[HAS_RAB ? BWD_BAND : 1];
  __shared__ float band1[HAS_RAB ? BWD_BAND : 1];
  __shared__ int next_rec[16];  // the next item of this workgroup: its record (8 words), then its list position

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int half = lane >> 5;
  const BwdLanes lc = bwd_lanes(lane);

  zero_tail_rows_of<256>(p, bp.dk, (size_t)p.H * HD * 2);
  zero_tail_rows_of<256>(p, bp.dv, (size_t)p.H * HD * 2);

  // One workgroup per CU, so nothing hides what a workgroup waits for between two items.  The
  // workgroups stay: the first item of each is the list position of its index, after that it draws
  // positions from the list's counter (heaviest first, whoever is free first), one draw per item it
  // runs, issued two query tiles before the item ends; the drawn item's record is fetched into LDS
  // during the last tile.  The workgroup whose draw returns the last value any draw of this launch
  // can return puts the counter back for the next launch (work lists reused or not).
  const int xcd = blockIdx.x % NUM_XCD;
  const int list_len = p.ws_counts[xcd];
  int* const draw_ctr = p.ws_counts + NUM_XCD + xcd;
  const WorkItem* __restrict__ list = p.ws_items + (size_t)xcd * p.items_cap;
  int slot = blockIdx.x / NUM_XCD;
  WorkItem wi;
  if (slot < list_len) wi = list[slot];
  while (slot < list_len) {
    int drawn_v = 0;    // (wave 0) value of this item's draw, in flight until the tile ends
    int drawn = 0;      // 0: not drawn yet, 1: draw issued, 2: value read and record requested
    int next_slot = 0;
    auto draw_value_arrived = [&]() __attribute__((always_inline)) {
      next_slot = __builtin_amdgcn_readfirstlane(drawn_v);
      if (next_slot == p.grid_slots + list_len - 1 && lane == 0) *draw_ctr = p.grid_slots;  // nobody draws after this one
      // eight lanes fetch the eight words of the record straight into LDS; word 8 is the list position
      if (next_slot < list_len && lane < 8)
        copy4((const char*)(list + next_slot), (unsigned)lane * 4u, (unsigned)(size_t)&next_rec[0]);
      if (lane == 0) next_rec[8] = next_slot;
      drawn = 2;
    };
    auto draw_step = [&](int left) __attribute__((always_inline)) {
      if (wave != 0) return;
      if (drawn == 0 && left <= 2) {
        if (lane == 0) drawn_v = atomicAdd(draw_ctr, 1);
        drawn = 1;
      } else if (drawn == 1) {  // the tile in between ended with a wait for everything in flight
        draw_value_arrived();
      }
    };
    auto draw_finish = [&]() __attribute__((always_inline)) {
      if (wave != 0) return;
      if (drawn == 0) {
        if (lane == 0) drawn_v = atomicAdd(draw_ctr, 1);
        drawn = 1;
      }
      if (drawn == 1) draw_value_arrived();
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    };
    SeqInfo si;
    si.s = wi.s; si.n = wi.n; si.cap = wi.cap; si.ctx_eff = wi.ctx_eff;
    si.win = WIN_ALL; si.tail0 = 0x7fffffff;
    if (SEMI) mask_window(p, si.cap, si.win, si.tail0);
    const int j0 = wi.q0;  // first key row of this workgroup's tile
    const int h = wi.h;
    const unsigned row_bytes = (unsigned)p.H * HD * 2u;
    const char* __restrict__ qgb = (const char*)p.q + ((size_t)si.s * p.H + h) * (HD * 2);
    const char* __restrict__ ggb = (const char*)bp.dout + ((size_t)si.s * p.H + h) * (HD * 2);
    const int rab_w = 2 * p.N - 1;
    const float* __restrict__ rab_row = HAS_RAB ? p.rab + (size_t)h * rab_w : nullptr;

    const int jw0 = j0 + wave * 32;
    const int j = jw0 + l32;  // this lane's key row
    const int j_lo = jw0;
    const int j_hi = min(jw0 + 31, si.n - 1);
    const bool wave_has_rows = j_lo < si.n;
    // causal mask of this lane's key as bounds on the query index (row m0 + 4 half + c): a contextual
    // key is seen by every row, a history key by the rows from its own on, a target key by its own
    // row only; rows end at n
    const int mk_from = (j < si.ctx_eff ? 0 : (j < si.cap ? j : 0x40000000)) - 4 * half;
    const int mk_own = j - 4 * half;
    const int mk_end = si.n - 4 * half;

    // Query tiles that see a key of [j0, j0 + 128): from the diagonal (from 0 when the tile holds a
    // contextual key) to the end of the sequence when the tile holds a history key, else through
    // the diagonal only.
    const int j_end = min(j0 + BWD_BM, si.n);
    const bool has_ctx = j0 < si.ctx_eff;
    const bool has_hist = j0 < si.cap;
    const int t_first = has_ctx ? 0 : j0 / BWD_BN;
    const int t_last = (has_hist || has_ctx) ? (si.n - 1) / BWD_BN : (j_end - 1) / BWD_BN;  // inclusive
    const int nq = t_last + 1;
    // Semi-local mask: the last of this tile's keys is inside the window of the rows up to
    // j_end - 1 + win; after them no row sees any of the keys until the rows of the full-attention
    // tail begin (rows from tail0 on, which include the target rows; without a tail: no row at all).
    // The query tiles in between, [gap_a, gap_b), are not walked.  (Unless the window reaches the
    // target rows, whose position is cap, or the tile holds a contextual key.)
    int gap_a = nq, gap_b = nq;
    if (SEMI && has_hist && !has_ctx) {
      const long long reach = (long long)(j_end - 1) + si.win;
      if (reach < (long long)si.cap) {
        const int resume_row = si.tail0 == 0x7fffffff ? si.n : max(si.tail0, 0);
        const int a = (int)(reach / BWD_BN) + 1, b = min(resume_row / BWD_BN, nq);
        if (a < b) { gap_a = a; gap_b = b; }
      }
    }
    auto next_tile = [&](int t) { return t + 1 == gap_a ? gap_b : t + 1; };
    auto tiles_left = [&](int t) { return t < gap_a ? (gap_a - t) + (nq - gap_b) : nq - t; };  // from t on, t included

    auto issue_tile = [&](int it, auto buf_tag) __attribute__((always_inline)) {
      constexpr int BUF = decltype(buf_tag)::value;
      const int m0 = it * BWD_BN;
      const int last = si.n - 1 - m0;
      bwd_issue_rows<HAS_RAB>(qgb + (size_t)m0 * row_bytes, row_bytes, last, BUF ? Qs1 : Qs0, lc, wave);
      bwd_issue_rows<HAS_RAB>(ggb + (size_t)m0 * row_bytes, row_bytes, last, BUF ? Gs1 : Gs0, lc, wave);
    };

    // bias band of query tile t: entry i is rab index 64 t - j0 - 127 + N - 1 + i
    auto band_of = [&](int t) __attribute__((always_inline)) {
      return bwd_band_load(rab_row, rab_w, t * BWD_BN - j0 - (BWD_BM - 1) + p.N - 1, tid);
    };
    int it = t_first;
    float band_first = 0.f;
    if (HAS_RAB && it < nq) band_first = band_of(it);
    if (it < nq) issue_tile(it, std::integral_constant<int, 0>{});

    bf16x8 kf[8], vf[8];
    bwd_load_row_frags(p.k, (size_t)si.s + j, p.H, h, half, j < si.n, false, 1.0f, kf);
    const float score_c = p.alpha * kLog2e, neg_c = -score_c;
    // The bias is staged divided by alpha and starts the score accumulators: alpha (s + bias / alpha)
    // is the biased score, and the arithmetic below is that of the kernel without a bias.  (The host
    // sends a bias with alpha = 0 to the generic kernels.)
    const float bias_mul = HAS_RAB ? 1.0f / p.alpha : 0.f;
    auto band_mul_of = [&](int t) __attribute__((always_inline)) {  // 0 for a diagonal outside the table, as in the dQ kernel
      return (unsigned)(t * BWD_BN - j0 - (BWD_BM - 1) + p.N - 1 + tid) < (unsigned)rab_w ? bias_mul : 0.f;
    };
    bwd_load_row_frags(p.v, (size_t)si.s + j, p.H, h, half, j < si.n, false, 1.0f, vf);

    bwd_acc_zero();  // dK^T and dV^T accumulators (fixed AGPRs)

    auto tile_body = [&](auto masked_tag, auto buf_tag, int m0) __attribute__((always_inline)) {
      // 0 no mask; 1 the general predicate; 2 (semi-local) keys of the wave all history keys outside the
      // contextual prefix and the query tile whole and either all window rows (history rows below the
      // full-attention tail: kept iff 0 <= m - j <= win) or all tail rows (kept iff m >= j): one
      // unsigned comparison of m - j with a bound that is the same for the whole wave
      constexpr int MASKED = decltype(masked_tag)::value;
      const int rng_base = m0 + 4 * half - j;
      const unsigned rng_w = min(m0, si.cap) >= si.tail0 ? 0x7fffffffu : (unsigned)si.win;
      constexpr int BUF = decltype(buf_tag)::value;
      const char* qb = (const char*)(BUF ? Qs1 : Qs0);
      const char* gb = (const char*)(BUF ? Gs1 : Gs0);
      const float* bandt = BUF ? band1 : band0;
      // The products are written out as instructions with their register classes named: scores in
      // VGPRs (the arithmetic reads them), the dK and dV accumulators in fixed AGPRs
      // (hstu_bwd_acc_regs.h).  Left to choose, the compiler puts every MFMA result of this
      // 512-register kernel into AGPRs and moves them: 250 of a tile's 570 VALU instructions were
      // such moves.
      // The two 32-row query blocks of the tile are software-pipelined, one wave per SIMD having
      // nothing else to hide its arithmetic behind:
      //   1: S, dP of block 0                           (16 MFMAs)
      //   2: S, dP of block 1   | P, dS of block 0      (one element per MFMA)
      //   3: dV, dK += block 0  | P, dS of block 1
      //   4: dV, dK += block 1
      auto score_mfma = [&](int qb32, int i, f32x16& s, f32x16& dp, bf16x8 f) __attribute__((always_inline)) {
        // i = 2 kk: S += Q[kk] K[kk];  i = 2 kk + 1: dP += dO[kk] V[kk]
        const int kk = i >> 1;
        const bf16x8 kfr = kf[kk], vfr = vf[kk];
        if (!(i & 1)) {
          if (kk == 0 && !HAS_RAB) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(s) : "v"(f), "v"(kfr));
          else asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(s) : "v"(f), "v"(kfr));  // (with a bias: s starts from it)
        } else {
          if (kk == 0) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(dp) : "v"(f), "v"(vfr));
          else asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(dp) : "v"(f), "v"(vfr));
        }
      };
      auto score_frag = [&](int qb32, int i) __attribute__((always_inline)) {
        return (i & 1) ? bwd_row_frag(gb, lc, qb32, i >> 1) : bwd_row_frag(qb, lc, qb32, i >> 1);
      };
      // product i of a block's sixteen into the accumulators: key step i / 8, block (i / 2) % 4, dV (even) or dK (odd)
      auto acc_frag = [&](int qb32, int i) __attribute__((always_inline)) {
        return bwd_tr_frag((i & 1) ? qb : gb, lc, (i >> 1) & 3, 2 * qb32 + (i >> 3));
      };
      // P and dS of element r of block qb32 (query row m0 + 32 qb32 + 8 (r / 4) + 4 half + r % 4, this lane's key)
      auto element = [&](int qb32, int r, float sv_raw, float dpv, float tsv, float& pe, float& g) __attribute__((always_inline)) {
        // P = x sig and silu'(x) = sig (1 + x (1 - sig)), x = alpha s (s with the bias / alpha it started
        // from).  No instruction is spent on x: alpha goes into (1 - sig), and P is kept as s sig, its
        // alpha applied to the dV accumulators at the end
        const float sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(sv_raw * neg_c));
        const float inner = __builtin_fmaf(sv_raw, __builtin_fmaf(sig, -p.alpha, p.alpha), 1.0f);
        pe = sv_raw * sig;
        g = dpv * (sig * inner);
        if (PER_TOKEN) { pe *= tsv; g *= tsv; }
        if (MASKED == 2) {
          const bool kp = (unsigned)(rng_base + (qb32 * 32 + 8 * (r >> 2) + (r & 3))) <= rng_w;
          pe = kp ? pe : 0.f;
          g = kp ? g : 0.f;
        }
        if (MASKED == 1) {
          const int c = qb32 * 32 + 8 * (r >> 2) + (r & 3);
          const int m = m0 + 4 * half + c;
          const int idm = min(m, si.cap);
          const bool kp = SEMI ? ((m == j) | ((j < idm) & ((idm - j <= si.win) | (idm >= si.tail0))) | (j < si.ctx_eff)) & (m < si.n)
                               : ((c >= mk_from - m0) | (c == mk_own - m0)) & (c < mk_end - m0);
          pe = kp ? pe : 0.f;
          g = kp ? g : 0.f;
        }
      };
      // the staged bias (already divided by alpha) as the start of a block's score accumulators
      auto load_bias = [&](int qb32, f32x16& sacc) __attribute__((always_inline)) {
        if (!HAS_RAB) return;
#pragma unroll
        for (int r = 0; r < 16; ++r)
          sacc[r] = bandt[(qb32 * 32 + 8 * (r >> 2) + 4 * half + (r & 3)) - (j - j0) + (BWD_BM - 1)];
      };
      auto load_ts = [&](int qb32, float (&ts)[16]) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          ts[r] = PER_TOKEN ? p.attn_scale[si.s + min(m0 + qb32 * 32 + 8 * (r >> 2) + 4 * half + (r & 3), si.n - 1)] : 1.0f;
      };
      constexpr int PD = 3;  // fragments requested this many products ahead (5 and 8 measured the same)
      f32x16 sA, dpA, sB, dpB;
      float ts[16];
      unsigned pwA[8], dwA[8], pwB[8], dwB[8];  // packed P and dS of the two blocks
      // phase 1 (its fragments requested ahead like those of the other phases: read one by one, each right
      // before its product, they left this wave, alone on its SIMD, waiting for the LDS sixteen times a tile)
      load_bias(0, sA);
      {
        bf16x8 F[16];
#pragma unroll
        for (int i = 0; i < PD; ++i) F[i] = score_frag(0, i);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          if (i + PD < 16) F[i + PD] = score_frag(0, i + PD);
          score_mfma(0, i, sA, dpA, F[i]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      load_ts(0, ts);
      // an MFMA result may be read by other instructions 11 cycles after the MFMA at the earliest; the
      // compiler does not count for instructions it did not place
      asm volatile("s_nop 15" : "+v"(sA), "+v"(dpA));
      // phase 2
      {
        bf16x8 F[16];
#pragma unroll
        for (int i = 0; i < PD; ++i) F[i] = score_frag(1, i);
        float pe_prev = 0.f, g_prev = 0.f;
        load_bias(1, sB);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          if (i + PD < 16) F[i + PD] = score_frag(1, i + PD);
          score_mfma(1, i, sB, dpB, F[i]);
          float pe, g;
          element(0, i, sA[i], dpA[i], ts[i], pe, g);
          if (i & 1) { pwA[i >> 1] = pack_bf16x2(pe_prev, pe); dwA[i >> 1] = pack_bf16x2(g_prev, g); }
          pe_prev = pe; g_prev = g;
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      load_ts(1, ts);
      asm volatile("s_nop 15" : "+v"(sB), "+v"(dpB));
      // phase 3
      {
        const u32x4 pa0 = {pwA[0], pwA[1], pwA[2], pwA[3]}, pa1 = {pwA[4], pwA[5], pwA[6], pwA[7]};
        const u32x4 da0 = {dwA[0], dwA[1], dwA[2], dwA[3]}, da1 = {dwA[4], dwA[5], dwA[6], dwA[7]};
        const bf16x8 opA[4] = {__builtin_bit_cast(bf16x8, pa0), __builtin_bit_cast(bf16x8, da0),
                               __builtin_bit_cast(bf16x8, pa1), __builtin_bit_cast(bf16x8, da1)};
        bf16x8 F[16];
#pragma unroll
        for (int i = 0; i < PD; ++i) F[i] = acc_frag(0, i);
        float pe_prev = 0.f, g_prev = 0.f;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          if (i + PD < 16) F[i + PD] = acc_frag(0, i + PD);
          bwd_acc_mfma1(((i & 1) ? 4 : 0) + ((i >> 1) & 3), F[i], opA[2 * (i >> 3) + (i & 1)]);
          float pe, g;
          element(1, i, sB[i], dpB[i], ts[i], pe, g);
          if (i & 1) { pwB[i >> 1] = pack_bf16x2(pe_prev, pe); dwB[i >> 1] = pack_bf16x2(g_prev, g); }
          pe_prev = pe; g_prev = g;
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      // phase 4
      {
        const u32x4 pb0 = {pwB[0], pwB[1], pwB[2], pwB[3]}, pb1 = {pwB[4], pwB[5], pwB[6], pwB[7]};
        const u32x4 db0 = {dwB[0], dwB[1], dwB[2], dwB[3]}, db1 = {dwB[4], dwB[5], dwB[6], dwB[7]};
        const bf16x8 opB[4] = {__builtin_bit_cast(bf16x8, pb0), __builtin_bit_cast(bf16x8, db0),
                               __builtin_bit_cast(bf16x8, pb1), __builtin_bit_cast(bf16x8, db1)};
        bf16x8 F[16];
#pragma unroll
        for (int i = 0; i < PD; ++i) F[i] = acc_frag(1, i);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          if (i + PD < 16) F[i + PD] = acc_frag(1, i + PD);
          bwd_acc_mfma1(((i & 1) ? 4 : 0) + ((i >> 1) & 3), F[i], opB[2 * (i >> 3) + (i & 1)]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };

    auto compute_tile = [&](int itc, auto buf_tag) __attribute__((always_inline)) {
      const int m0 = itc * BWD_BN;
      const int m1 = min(m0 + BWD_BN, si.n);  // exclusive
      // any pair of (query tile, this wave's keys) kept?
      bool any_kept = wave_has_rows && ((m0 <= j_hi && m1 > j_lo) ||           // diagonal
                                        (j_lo < si.cap && m1 - 1 >= j_lo) ||  // history key, later query
                                        (j_lo < si.ctx_eff));                  // contextual key
      if (SEMI) {
        // a history key counts only for rows whose window reaches it or rows of the full-attention tail
        const int id0 = min(m0, si.cap), id1 = min(m1 - 1, si.cap);
        any_kept = wave_has_rows && ((m0 <= j_hi && m1 > j_lo) || (j_lo < si.ctx_eff) ||
                                     (j_lo < si.cap && m1 - 1 >= j_lo && (id0 - j_hi <= si.win || id1 >= si.tail0)));
      }
      if (!any_kept) return;
      // every pair kept: all keys are history keys (or contextual) below every query row, tile whole
      bool full = (m0 + BWD_BN <= si.n) && (jw0 + 31 < si.n) &&
                  ((jw0 + 31 <= m0 && jw0 + 31 < si.cap) || (jw0 + 31 < si.ctx_eff));
      if (SEMI)
        full = full && ((jw0 + 31 < si.ctx_eff) || min(m0, si.cap) >= si.tail0 ||
                        min(m0 + BWD_BN - 1, si.cap) - jw0 <= si.win);
      const bool range_mask = SEMI && jw0 + 31 < si.cap && jw0 >= si.ctx_eff && m0 + BWD_BN <= si.n &&
                              (min(m0, si.cap) >= si.tail0 || m0 + BWD_BN - 1 < min(si.cap, si.tail0));
      if (full) tile_body(std::integral_constant<int, 0>{}, buf_tag, m0);
      else if (SEMI && range_mask) tile_body(std::integral_constant<int, 2>{}, buf_tag, m0);
      else tile_body(std::integral_constant<int, 1>{}, buf_tag, m0);
    };

    if (HAS_RAB && it < nq) bwd_band_store<false>(band0, band_first, tid, band_mul_of(it));
    while (it < nq) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      int nxt = next_tile(it);
      float band_nxt = 0.f;
      if (HAS_RAB && nxt < nq) band_nxt = band_of(nxt);
      if (nxt < nq) issue_tile(nxt, std::integral_constant<int, 1>{});
      draw_step(tiles_left(it));
      compute_tile(it, std::integral_constant<int, 0>{});
      if (HAS_RAB && nxt < nq) bwd_band_store<false>(band1, band_nxt, tid, band_mul_of(nxt));
      it = nxt;
      if (it >= nq) break;
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      nxt = next_tile(it);
      if (HAS_RAB && nxt < nq) band_nxt = band_of(nxt);
      if (nxt < nq) issue_tile(nxt, std::integral_constant<int, 0>{});
      draw_step(tiles_left(it));
      compute_tile(it, std::integral_constant<int, 1>{});
      if (HAS_RAB && nxt < nq) bwd_band_store<false>(band0, band_nxt, tid, band_mul_of(nxt));
      it = nxt;
    }
    draw_finish();
    // (here, where everything in flight has been waited for: at the item's start the wait for the word's
    // value would also wait for the first tile's copies)
    if (bp.absmax) {  // the query-tile kernel's fixed-point sums need the largest |v| of the call
      unsigned mx = bwd_frag_absmax(vf);
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) mx = max(mx, (unsigned)__shfl_xor((int)mx, d, 64));
      mx <<= 16;
      if (lane == 0 && mx > __hip_atomic_load(bp.absmax + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) atomicMax(bp.absmax + 1, mx);
    }

    if (j < si.n) {
      const float oscale = PER_TOKEN ? 1.0f : bwd_output_scale(p);
      const float kscale = p.alpha * oscale;
      const float vscale = kscale;  // P was kept without its alpha
      unsigned short* krow = (unsigned short*)bp.dk + ((size_t)(si.s + j) * p.H + h) * HD;
      unsigned short* vrow = (unsigned short*)bp.dv + ((size_t)(si.s + j) * p.H + h) * HD;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        float av[16], ak[16];
        bwd_acc_read(db, av);
        bwd_acc_read(4 + db, ak);
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          u32x2 o;
          o.x = pack_bf16x2(ak[4 * rq + 0] * kscale, ak[4 * rq + 1] * kscale);
          o.y = pack_bf16x2(ak[4 * rq + 2] * kscale, ak[4 * rq + 3] * kscale);
          *(u32x2*)(krow + db * 32 + 8 * rq + 4 * half) = o;
          o.x = pack_bf16x2(av[4 * rq + 0] * vscale, av[4 * rq + 1] * vscale);
          o.y = pack_bf16x2(av[4 * rq + 2] * vscale, av[4 * rq + 3] * vscale);
          *(u32x2*)(vrow + db * 32 + 8 * rq + 4 * half) = o;
        }
      }
    }
    __syncthreads();  // LDS is reused by the next item; its record is in
    // (the same for every lane: said so, because the tile copies take their base address in scalar registers)
    auto uni = [](int x) { return __builtin_amdgcn_readfirstlane(x); };
    slot = uni(next_rec[8]);
    if (slot < list_len) {
      wi.s = uni(next_rec[0]); wi.n = uni(next_rec[1]); wi.cap = uni(next_rec[2]); wi.ctx_eff = uni(next_rec[3]);
      wi.q0 = uni(next_rec[4]); wi.h = uni(next_rec[5]); wi.b = uni(next_rec[6]); wi.q_end = uni(next_rec[7]);
    }
    __syncthreads();  // next_rec is written again during the item
  }
}

// Everything the bias-table gradient accumulates into, cleared by one launch: the three maxima words,
// the per-head maxima of dout and the fixed-point table.
__global__ __launch_bounds__(256) void hstu_drab_prepare(unsigned* am, unsigned* dout_max, int H, long long* tab, size_t tab_words) {
  const size_t first = (size_t)blockIdx.x * blockDim.x + threadIdx.x, stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = first; i < tab_words; i += stride) tab[i] = 0;
  if (blockIdx.x == 0) {
    if (threadIdx.x < 4) am[threadIdx.x] = 0u;
    for (int h = threadIdx.x; h < H; h += blockDim.x) dout_max[h] = 0u;
  }
}

// Largest |attn_scale[r]| over the rows of the sequences (per-token scale), as the bits of a float,
// merged into *out with an integer maximum (the bits of non-negative floats order like integers;
// a NaN's bits are above every finite value's, so it ends up in the bound and makes it unusable).
__global__ __launch_bounds__(256) void hstu_scale_absmax(const float* scale, const void* seq_end, int i32, int T, unsigned* out) {
  const long long e = i32 ? (long long)*(const int*)seq_end : *(const long long*)seq_end;
  const int rows = (int)(e < 0 ? 0 : (e > T ? T : e));
  unsigned mx = 0;
  for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += gridDim.x * blockDim.x)
    mx = max(mx, __float_as_uint(scale[r]) & 0x7fffffffu);
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) mx = max(mx, (unsigned)__shfl_xor((int)mx, d, 64));
  if ((threadIdx.x & 63) == 0 && mx) atomicMax(out, mx);
}

// Fixed-point table of the bias-table gradient -> drab[h, i] in floats: the head's scale taken out,
// then the global output scale of P (a per-token scale is already inside the sums).
__global__ __launch_bounds__(256) void hstu_drab_finalize(BwdParams bp, int per_token) {
  const Params& p = bp.f;
  const int rab_w = 2 * p.N - 1;
  const size_t n = (size_t)p.H * rab_w;
  const float out_scale = per_token ? 1.0f : bwd_output_scale(p);
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const int h = (int)(i / rab_w);
    float fx_scale, fx_inv;
    drab_fx_scales(drab_fx_bound(bp, h, per_token != 0), fx_scale, fx_inv);
    bp.drab[i] = (float)((double)bp.drab_fx[i]) * fx_inv * out_scale;
  }
}

}  // namespace recir_hstu
