// Tiled MFMA kernel of the HSTU attention forward, head dim 128 (qk and v), bf16 values, with K and
// V tiles copied global -> LDS directly (no register staging) and V^T fragments produced by the
// LDS transposing read.
//
// One workgroup (4 waves) per (sequence, query tile of BM = 128 rows, head); wave w owns query rows
// [32w, 32w+32) of the tile.  For every key tile of BN = 64 rows:
//   S^T[kv, q]  = K[kv, d] . Q^T[d, q]        v_mfma_f32_32x32x16_bf16, A = K from LDS, B = Q in VGPRs
//   P^T         = silu(S^T (+rab)) masked, rounded to bf16, kept in registers: the 32x32 accumulator
//                 layout (lane = query column, 8 key rows per lane half) is exactly the B-operand
//                 layout of the next contraction
//   O^T[d, q]  += V^T[d, kv] . P^T[kv, q]     A = V^T, read from the row-major V tile with
//                 ds_read_b64_tr_b16 (each 16-lane group transposes a 4 x 16 block)
// The score accumulators hold the raw products S' = q . k (+ bias / alpha): q is not rescaled, so no
// rounding beyond the operands' own enters a score.  With c = alpha * log2(e), sigmoid(alpha S') =
// 1 / (1 + exp2(-c S')) and P' = S' sigmoid(alpha S') is what is rounded to bf16; the remaining factor
// (alpha and the 1/N scale) is applied once to the fp32 output accumulator.
//
// Pipeline: two LDS stages.  The global_load_lds of tile i+1 are issued while the first MFMAs of
// tile i run and must have landed (vmcnt) before the barrier that ends tile i.
//
// LDS layouts (both tiles are [BN rows][256 bytes], swizzled in place of padding):
//   K  16-byte chunk c of row r sits at chunk c ^ (r & 15)
//   V  32-byte slot  s of row r sits at slot  s ^ 2 (r & 3)
// These are free of bank conflicts on gfx950's 64 banks (256 bytes per clock) for the K fragment
// reads (ds_read_b128) and the transposing V reads.  (The forms for 32 banks, c ^ (r & 7) and
// s ^ (r & 3), run those reads at half rate; they need six address registers fewer and measured
// 1-2 % slower once nothing spilled.)
// A global_load_lds instruction writes 64 lanes x 16 bytes to consecutive LDS addresses, so the
// swizzle is applied to the global address each lane fetches.
#pragma once
#include <type_traits>

#include "hstu_common.h"

namespace recir_hstu {

typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef __attribute__((ext_vector_type(8))) short i16x8;
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) const float lds_cfloat;
typedef __attribute__((address_space(3))) float lds_float;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

typedef __attribute__((ext_vector_type(8))) int i32x8;

// FP8: q and k are OCP e4m3 bytes ([T, H, 128] of one byte each) with per-head dequantisation factors;
// the scores come from v_mfma_scale_f32_32x32x64_f8f6f4 (two per 32 x 32 block, unit block scales) and
// are multiplied by alpha * q_scale[h] * k_scale[h] * log2(e) in fp32; v, P and the second
// contraction stay bf16.  The K tile is then [BN rows][128 bytes], chunk c of row r at c ^ (r & 7).
// SEMI: the semi-local mask (max_attn_len > 0) -- window test in the partial tiles, key tiles below
// every row's window not walked; the causal instantiation carries none of it.
// One global -> LDS copy instruction: 64 lanes x 16 bytes from base + per-lane offset to 1 KB of
// consecutive LDS.  Written as assembly so that the compiler does not treat it as an access that
// may touch both memories: with the builtin every later wait for an LDS read becomes a wait for
// all of them (and for nothing less), which exposes a full LDS round trip several times per tile.
// Ordering against LDS reads is the caller's (vmcnt wait + barrier).
__device__ __forceinline__ void copy16(const void* base, unsigned lane_off, unsigned lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_addr), "v"(lane_off), "s"(base) : "memory");
}
// The same with four bytes per lane (lane i lands at lds_addr + 4 i).
__device__ __forceinline__ void copy4(const void* base, unsigned lane_off, unsigned lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds_addr), "v"(lane_off), "s"(base) : "memory");
}
constexpr int KSWZ = 15;  // K chunk ^ (row & 15)
constexpr int VSWZ = 4;   // V 16-byte chunk ^ 4 (row & 3), i.e. 32-byte slot ^ 2 (row & 3)

// Schedule constants of the tile bodies, each the best of a measured range (configurations 2 and 4).
constexpr int DL_PDK = 6;       // K fragments (slots 0..15) are requested this many slots ahead
constexpr int DL_PDV = 10;      // V fragments (slots 16..31) likewise
constexpr int DL_PDK_RAB = 6;   // K fragments in flight when a tile opens, bias instantiations
constexpr int DL_PD_SLOW = 3;   // fragment prefetch distance of the bodies that carry mask or clamping state
constexpr int DL_B1 = 5;        // slot in which the bias of the second score block is read (first used in slot 8)
constexpr int DL_U0 = 9;        // slot of the first SiLU unit
constexpr int DL_SKEW_MIN = 2;  // fewest leading tiles worth the skewed loop's entry and exit
constexpr int DL_SKEW_PD = 3;   // the skewed loop's fragment prefetch distance in slots
// Measurement switch (python -m recir_amd.build --trace -DHSTU_DL_SKEW=0): 0 walks the leading
// unmasked tiles with the plain loop, for timing the two loops against each other.
#ifndef HSTU_DL_SKEW
#define HSTU_DL_SKEW 1
#endif
#define HSTU_DL_TILE_SYNC() do { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); __syncthreads(); } while (0)
template <bool HAS_RAB, bool FP8, bool SEMI>
__global__ __launch_bounds__(256, 2) void hstu_fwd_tiled_d128_dl(Params p) {
  // The two pipeline stages are separate objects and every access names its stage at compile time:
  // the compiler then knows that an LDS read of one stage cannot alias the global -> LDS copies in
  // flight into the other, and does not wait for them.
  __shared__ __attribute__((aligned(1024))) unsigned short Ks0[BN * HD];
  __shared__ __attribute__((aligned(1024))) unsigned short Ks1[BN * HD];
  __shared__ __attribute__((aligned(1024))) unsigned short Vs0[BN * HD];
  __shared__ __attribute__((aligned(1024))) unsigned short Vs1[BN * HD];
  __shared__ float rabs0[HAS_RAB ? (BM + BN) : 1];
  __shared__ float rabs1[HAS_RAB ? (BM + BN) : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int half = lane >> 5;

  // ---- per-lane constants of the LDS access patterns ----
  // K fragment (ds_read_b128): row 32 kvb + l32, chunk (2 kk + half) ^ (l32 & 15); kk enters as an
  // XOR of address bits 5..7
  const unsigned ks_rd = (unsigned)l32 * (HD * 2) + (unsigned)((half ^ (l32 & KSWZ)) * 16);
  // V^T fragment (two ds_read_b64_tr_b16): source lane s = lane & 15 of a 16-lane group supplies the
  // 8 bytes at row 4 half + (s >> 2) (+ 16 s2 + 8 rd), d = 32 db + 16 dgrp + 4 (s & 3) .. +3
  const int tr_s = lane & 15, tr_r = tr_s >> 2, tr_c = tr_s & 3, tr_dgrp = (lane >> 4) & 1;
  const unsigned vt_rd = (unsigned)(4 * half + tr_r) * (HD * 2) + (unsigned)tr_r * 64u + (unsigned)tr_dgrp * 32u + (unsigned)tr_c * 8u;
  // global -> LDS copies: instruction j of a tile (16 per matrix, wave w issues j = 4 w + ps) fills rows
  // 4 j .. 4 j + 3; lane i lands at row 4 j + (i >> 4), physical chunk i & 15
  const int ld_row = lane >> 4, ld_chunk = lane & 15;
  // fp8 K: fragment = 32 bytes at row 32 kvb + l32, chunks (4 st + 2 half + {0, 1}) ^ ((l32 >> 1) & 7)
  // (rows of 128 bytes: two rows per pass over the banks); a copy
  // instruction fills 8 rows of 128 bytes, lane i lands at row 8 j + (i >> 3), physical chunk i & 7
  const unsigned k8_rd = (unsigned)l32 * 128u + (unsigned)(((2 * half) ^ ((l32 >> 1) & 7)) * 16);
  const int ld8_row = lane >> 3, ld8_chunk = lane & 7;

  // Work list of the XCD this workgroup runs on.  The list length and the workgroup's item are written by an earlier launch and only read here:
  // both go through the constant address space (scalar loads, issued side by side before anything
  // is waited for; the item is fetched whether or not its slot is inside the list, the slot always
  // being inside the list's storage).
  typedef const __attribute__((address_space(4))) int* const_ints;
  const int xcd = blockIdx.x % NUM_XCD;
  const int slot0 = blockIdx.x / NUM_XCD;  // < grid_slots <= items_cap
  const WorkItem* list = p.ws_items + (size_t)xcd * p.items_cap;
  auto load_item = [&](int slot) __attribute__((always_inline)) {
    const_ints w = (const_ints)(size_t)(list + slot);
    WorkItem it;
    it.s = w[0]; it.n = w[1]; it.cap = w[2]; it.ctx_eff = w[3]; it.q0 = w[4]; it.h = w[5]; it.b = w[6]; it.q_end = w[7];
    return it;
  };
  WorkItem wi = load_item(slot0);
  const int list_len = ((const_ints)(size_t)p.ws_counts)[xcd];
  // Normally one item per workgroup; the stride loop only matters when a list is longer than the
  // launch assumed (sequences above max_seq_len).
  for (int slot = slot0; slot < list_len; slot += p.grid_slots) {
    HSTU_TR(const unsigned long long tr_start = wall_clock64(); unsigned long long tr_ready = tr_start, tr_ticks[5] = {0, 0, 0, 0, 0};
            unsigned tr_count[5] = {0, 0, 0, 0, 0}; long long tr_c0_item = clock64();)
    if (slot != slot0) wi = load_item(slot);
    SeqInfo si;
    si.s = wi.s; si.n = wi.n; si.cap = wi.cap; si.ctx_eff = wi.ctx_eff;
    si.win = WIN_ALL; si.tail0 = 0x7fffffff;
    if (SEMI) mask_window(p, si.cap, si.win, si.tail0);
    const int q0 = wi.q0;
    const int q_end = wi.q_end;  // rows [q0, q_end) belong to this item
    const int h = wi.h;

    const unsigned row_bytes = (unsigned)p.H * HD * 2u;                   // bf16 rows (v, and k unless FP8)
    const unsigned krow_bytes = FP8 ? (unsigned)p.H * HD : row_bytes;
    const char* __restrict__ kgb = (const char*)p.k + ((size_t)si.s * p.H + h) * (FP8 ? HD : HD * 2);
    const char* __restrict__ vgb = (const char*)p.v + ((size_t)si.s * p.H + h) * (HD * 2);
    const int rab_w = 2 * p.N - 1;
    const float* __restrict__ rabg = HAS_RAB ? p.rab + (size_t)h * rab_w : nullptr;
    // score_c: the factor between an accumulator value S' and x log2(e), x the argument of SiLU:
    //   alpha log2(e) (fp8: alpha q_scale[h] k_scale[h] log2(e)); bias_mul: what the bias is staged with
    //   (log2(e) / score_c).  With t = -score_c S' = -x log2(e): sigmoid(x) = 1 / (1 + exp2(t)), and P is
    //   kept as t sigmoid(x) = -log2(e) silu(x), so the score itself is read once; the output carries
    //   -1 / log2(e) on top of the scale
    float score_c = p.alpha * kLog2e;
    if (FP8) score_c *= p.q_scale[h] * p.k_scale[h];
    const float neg_c = -score_c;
    const float bias_mul = HAS_RAB ? kLog2e / score_c : 0.f;

    // logical 16-byte chunk each lane fetches so that the swizzled layout comes out
    const unsigned k_off = (unsigned)ld_row * row_bytes + (unsigned)((ld_chunk ^ ld_row) * 16);  // rows 16 a + 0..3; ^ 64 ps for rows 16 a + 4 ps + 0..3
    const unsigned v_off = (unsigned)ld_row * row_bytes + (unsigned)((ld_chunk ^ (VSWZ * ld_row)) * 16);
    const unsigned k8_off = (unsigned)ld8_row * krow_bytes + (unsigned)((ld8_chunk ^ (ld8_row >> 1)) * 16);  // rows 16 a + 0..7; ^ 64 for rows 16 a + 8..15

    const int qw0 = q0 + wave * 32;
    const int m = qw0 + l32;
    const int m_lo = qw0;
    const int m_hi = min(qw0 + 31, q_end - 1);
    const bool wave_has_rows = m_lo < q_end;
    // semi-local: target-clamped position of this lane's row and of the wave's first and last row
    const int idm = min(m, si.cap);
    const bool tail_row = idm >= si.tail0;
    const int idlo_w = min(m_lo, si.cap), idhi_w = min(m_hi, si.cap);
    const bool wave_has_tail = idhi_w >= si.tail0;
    // The staged bias band is stored reversed (entry 190 - i holds rab index first + i), so that the
    // elements a lane holds, keys k0 + 4 half + c with ascending c, sit at ascending addresses:
    // byte 4 (127 - (m - q0) + 4 half + c) of the stage.  The lane part is made opaque to the compiler,
    // which otherwise forms an address register per pair of elements.
    unsigned rab_lane = 4u * (unsigned)(127 - (m - q0) + 4 * half);
    if (HAS_RAB) asm volatile("" : "+v"(rab_lane));
    // Causal mask of this lane's row as bounds on the key index: key j is kept iff
    //   j < max(min(idm, n), min(ctx_eff, n))  or  j == m (and m < n).
    // Element r of a score block is key k0 + 4 half + c with a compile-time c, so the bounds are
    // kept relative to 4 half and, per tile, to k0: two comparisons against constants per element
    // instead of the predicate's five.  (The semi-local predicate in the same form needs four and
    // measured slower than the direct one.)
    const int mk_eq = (m < si.n ? m : -0x40000000) - 4 * half;
    const int mk_top = max(min(idm, si.n), min(si.ctx_eff, si.n)) - 4 * half;
    auto kept = [&](int k0, int c) __attribute__((always_inline)) {
      if (SEMI) {
        const int j = k0 + 4 * half + c;
        return (bool)(((m == j) | ((j < idm) & ((idm - j <= si.win) | tail_row)) | (j < si.ctx_eff)) & (j < si.n));
      }
      return (bool)((c < mk_top - k0) | (c == mk_eq - k0));
    };
    // Semi-local mask of a history row (m < cap) against keys that are not contextual: key j is kept
    // iff m - win <= j <= m (0 <= j <= m for a row of the full-attention tail), one unsigned
    // comparison of j - lo with m - lo.  Per tile the lane keeps k0 + 4 half - lo, per element the
    // compile-time c is added: three instructions per score instead of the predicate's dozen.
    // (Derived again in every tile from a copy of m the compiler cannot see through: kept across the
    // tile loop the three values cost the kernel's last registers and the loop reloaded spills.)
    auto rng_of = [&](int k0, int& base, unsigned& w) __attribute__((always_inline)) {
      int mm = m;
      asm volatile("" : "+v"(mm));
      const int lo = min(mm, si.cap) >= si.tail0 ? 0 : mm - si.win;
      w = (unsigned)(mm - lo);
      base = k0 + 4 * half - lo;
    };

    // key tiles [0, nkv) minus the run [skip_a, skip_b) that holds only target keys off this query
    // tile's diagonal (and no contextual key)
    const int kv_end = min(si.n, max(q_end, si.ctx_eff));
    const int nkv = (kv_end + BN - 1) / BN;
    const int cap0 = si.cap > 0 ? si.cap : 0;
    const int skip_a = (max(cap0, si.ctx_eff) + BN - 1) / BN;
    const int skip_b = q0 / BN;
    const bool has_skip = skip_a < skip_b;
    auto next_tile = [&](int it) { return (has_skip && it + 1 == skip_a) ? skip_b : it + 1; };

    // Copies of one tile: 4 + 4 instructions per wave.  Rows at or past the end of the sequence
    // (last, partial tile only) re-read the sequence's last row; the mask zeroes their contribution.
    // part 2 ps (+ 1) = the K (V) instruction of rows 16 wave + 4 ps .. + 3; part 8 = fp8 K
    auto issue_part = [&](int it, auto buf_tag, auto whole_tag, int part) __attribute__((always_inline)) {
      constexpr int BUF = decltype(buf_tag)::value;
      constexpr bool KNOWN_WHOLE = decltype(whole_tag)::value;  // caller guarantees k0 + BN <= n
      unsigned short* Kd = BUF ? Ks1 : Ks0;
      unsigned short* Vd = BUF ? Vs1 : Vs0;
      const int k0 = it * BN;
      const char* kt = kgb + (size_t)k0 * krow_bytes;
      const char* vt = vgb + (size_t)k0 * row_bytes;
      const bool whole = KNOWN_WHOLE || k0 + BN <= si.n;
      const int last = si.n - 1 - k0;
      if (part < 8) {
        const int ps = part >> 1;
        const bool is_v = part & 1;
        const int r0 = 4 * (4 * wave + ps);  // first row this instruction fills
        unsigned ko = k_off ^ (unsigned)(64 * (ps & (KSWZ >> 2)));
        unsigned vo = v_off;
        const char* kr = kt + (size_t)r0 * krow_bytes;
        const char* vr = vt + (size_t)r0 * row_bytes;
        if (!whole) {
          asm volatile("" ::: "memory");  // keep the clamping arithmetic off the steady-state path
          const int row = min(r0 + ld_row, last);
          ko = (unsigned)row * krow_bytes + (unsigned)((ld_chunk ^ ((r0 + ld_row) & KSWZ)) * 16);
          vo = (unsigned)row * row_bytes + (unsigned)((ld_chunk ^ (VSWZ * ld_row)) * 16);
          kr = kt;
          vr = vt;
        }
        if (!is_v) { if (!FP8) copy16(kr, ko, (unsigned)(size_t)&Kd[r0 * HD]); }
        else copy16(vr, vo, (unsigned)(size_t)&Vd[r0 * HD]);
        return;
      }
      if (FP8) {
#pragma unroll
        for (int ps = 0; ps < 2; ++ps) {
          const int r0 = 8 * (2 * wave + ps);
          unsigned ko = k8_off ^ (unsigned)(64 * (ps & 1));
          const char* kr = kt + (size_t)r0 * krow_bytes;
          if (!whole) {
            asm volatile("" ::: "memory");
            ko = (unsigned)min(r0 + ld8_row, last) * krow_bytes + (unsigned)((ld8_chunk ^ (((r0 + ld8_row) >> 1) & 7)) * 16);
            kr = kt;
          }
          copy16(kr, ko, (unsigned)(size_t)((char*)Kd + r0 * 128));
        }
      }
    };
    // Band of bias entries a (query tile, key tile) pair can touch: index (m - j) + N - 1, staged
    // divided by the score multiplier (alpha; fp8: alpha q_scale k_scale) with plain stores, ordered by the barrier that publishes the tile.
    // In two steps, so that the load's round trip passes under a tile's arithmetic: the load goes
    // out before the tile's copies (the wait for it would otherwise wait for them too), the store
    // follows at the end of the tile.
    auto band_load = [&](int it) __attribute__((always_inline)) {
      int idx = q0 - it * BN - (BN - 1) + p.N - 1 + tid;
      idx = idx < 0 ? 0 : (idx >= rab_w ? rab_w - 1 : idx);
      return rabg[idx];  // scaled in band_store: nothing may use the value before the tile's arithmetic is over
    };
    // (it: the tile the band belongs to.  The load clamps its index into the table; a diagonal
    // outside it, possible only in a sequence longer than max_seq_len, gets no bias here)
    auto band_store = [&](auto buf_tag, float val, int it) __attribute__((always_inline)) {
      constexpr int BUF = decltype(buf_tag)::value;
      asm volatile("" : "+v"(val));  // first use of the loaded value: the wait for it stays here
      const bool in_table = (unsigned)(q0 - it * BN - (BN - 1) + p.N - 1 + tid) < (unsigned)rab_w;
      if (tid < BM + BN - 1) (BUF ? rabs1 : rabs0)[(BM + BN - 2) - tid] = in_table ? val * bias_mul : 0.f;
    };
    auto issue_tile_as = [&](int it, auto buf_tag, auto whole_tag) __attribute__((always_inline)) {
#pragma unroll
      for (int part = 0; part <= 8; ++part) issue_part(it, buf_tag, whole_tag, part);
    };
    auto issue_tile = [&](int it, auto buf_tag) __attribute__((always_inline)) {
      issue_tile_as(it, buf_tag, std::false_type{});
    };
    // copies and band where nothing is there to overlap with (tiles this wave skips)
    auto issue_tile_and_band = [&](int it, auto buf_tag) __attribute__((always_inline)) {
      float band = 0.f;
      if (HAS_RAB) band = band_load(it);
      issue_tile(it, buf_tag);
      if (HAS_RAB) band_store(buf_tag, band, it);
    };

    // first tile in flight before anything else is waited for
    // semi-local: key tiles below the window of the workgroup's first row are not walked unless a
    // row of the full-attention tail or a contextual key needs them
    int it0 = 0;
    if (SEMI && si.ctx_eff <= 0 && min(q_end - 1, si.cap) < si.tail0) it0 = max(min(q0, si.cap) - si.win, 0) / BN;
    int it = (has_skip && it0 >= skip_a) ? max(it0, skip_b) : it0;
    float band_first = 0.f;  // stored once the Q rows are in, just before the first barrier
    if (HAS_RAB && it < nkv) band_first = band_load(it);
    if (it < nkv) issue_tile(it, std::integral_constant<int, 0>{});

    // Leading key tiles that are unmasked for every row of the workgroup (64 t + 63 <= q0 and
    // 64 t + 64 <= cap), lie in the first contiguous run of the walk and are followed by a tile that
    // exists and is whole: an even number of them runs the skewed loop further down, all four waves
    // together, since that loop moves K and V in half tiles on a schedule of its own.
    constexpr bool SKEW = HSTU_DL_SKEW && !HAS_RAB && !FP8 && !SEMI;
    int skew_tiles = 0;
    if (SKEW && it == 0) {
      const int run_end = has_skip ? skip_a : nkv;
      const int f = min(min((q0 + 1) / BN, cap0 / BN), min(run_end - 1, si.n / BN - 1));
      skew_tiles = max(f, 0) & ~1;
      if (skew_tiles < DL_SKEW_MIN) skew_tiles = 0;
    }
    // One copy instruction of the skewed loop's trip i (LDS stage BUF = i & 1); this wave moves rows
    // 8 wave + 4 idx .. + 3 of a half tile.  parts 0, 1: K rows 0..31 of tile i + 2 (stage BUF);
    // 2, 3: K rows 32..63 of tile i + 1 (other stage); 4, 5: V rows 0..31 of tile i + 1 (other stage);
    // 6, 7: V rows 32..63 of tile i (stage BUF).  None of the four regions is read during trip i.
    auto skew_copy = [&](int i, auto buf_tag, int part) __attribute__((always_inline)) {
      constexpr int BUF = decltype(buf_tag)::value;
      const int idx = part & 1, sel = part >> 1;
      const bool is_v = sel >= 2, hi = (sel & 1) != 0, to_cur = (sel == 0 || sel == 3);
      const int tile = sel == 0 ? i + 2 : (sel == 3 ? i : i + 1);
      const int stage = to_cur ? BUF : (BUF ^ 1);
      const int jr = 8 * (int)hi + 2 * wave + idx;  // rows 4 jr .. 4 jr + 3 of the tile
      const int r0 = 4 * jr;
      unsigned short* dst = is_v ? (stage ? Vs1 : Vs0) : (stage ? Ks1 : Ks0);
      const char* src = (is_v ? vgb : kgb) + (size_t)(tile * BN + r0) * row_bytes;
      const unsigned off = is_v ? v_off : (k_off ^ (unsigned)(64 * (jr & (KSWZ >> 2))));
      copy16(src, off, (unsigned)(size_t)&dst[r0 * HD]);
    };
    if (SKEW && skew_tiles) {  // K rows 0..31 of tile 1: the first trip's scores of its second tile
      skew_copy(-1, std::integral_constant<int, 1>{}, 0);
      skew_copy(-1, std::integral_constant<int, 1>{}, 1);
    }

    // ---- Q fragments (B operand): lane holds row qw0 + l32 ----
    // bf16: d = 16 kk + 8 half .. +7, as stored;  fp8: d = 64 st + 32 half .. +31 (raw bytes)
    bf16x8 qf[FP8 ? 1 : 8];
    i32x8 q8[FP8 ? 2 : 1];
    {
      const bool valid = m < q_end;
      if constexpr (FP8) {
        const char* qrow = (const char*)p.q + ((size_t)(si.s + (valid ? m : 0)) * p.H + h) * HD;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const u32x4 zero4 = {0u, 0u, 0u, 0u};
          const u32x4 lo = valid ? *(const u32x4*)(qrow + 64 * st + 32 * half) : zero4;
          const u32x4 hi = valid ? *(const u32x4*)(qrow + 64 * st + 32 * half + 16) : zero4;
          q8[st] = (i32x8){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        }
      } else {
        const unsigned short* qrow = (const unsigned short*)p.q + ((size_t)(si.s + (valid ? m : 0)) * p.H + h) * HD;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const u32x4 zero4 = {0u, 0u, 0u, 0u};
          const u32x4 t = valid ? *(const u32x4*)(qrow + kk * 16 + half * 8) : zero4;
          qf[kk] = __builtin_bit_cast(bf16x8, t);
        }
      }
    }

    f32x16 acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

    // silu + mask + bf16 packing of one 32 x 32 score block (accumulator layout) into two B operands
    auto silu_pack = [&](auto masked_tag, const f32x16& sv, int k0, int kvb, unsigned rab_addr, bf16x8& o0,
                         bf16x8& o1) __attribute__((always_inline)) {
      constexpr int MASKED = decltype(masked_tag)::value;  // 0 none, 1 general predicate, 2 range of a history row, 5 nothing kept
      if constexpr (MASKED == 5) {
        const u32x4 z = {0u, 0u, 0u, 0u};
        o0 = __builtin_bit_cast(bf16x8, z);
        o1 = __builtin_bit_cast(bf16x8, z);
        return;
      }
      int rng_base = 0;
      unsigned rng_w = 0;
      if (MASKED == 2) rng_of(k0, rng_base, rng_w);
      f32x16 pv;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int jl = kvb * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        float s = sv[r];
        if (HAS_RAB) s += *(lds_cfloat*)(rab_addr + 4u * (unsigned)(kvb * 32 + 8 * (r >> 2) + (r & 3)));
        const float t = s * neg_c;
        float pe = t * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
        if (MASKED == 1) pe = kept(k0, kvb * 32 + 8 * (r >> 2) + (r & 3)) ? pe : 0.f;
        if (MASKED == 2) pe = (unsigned)(rng_base + (kvb * 32 + 8 * (r >> 2) + (r & 3))) <= rng_w ? pe : 0.f;
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

    // One (32 query rows) x (64 keys) block of this wave in four stages of eight MFMAs; the VALU
    // work of a stage is independent of that stage's MFMAs and the scheduling groups interleave them:
    //   0: S0 = K[0:32] Q^T          |  copies of the next tile are issued
    //   A: S1 = K[32:64] Q^T         |  P0 = silu(S0)
    //   B: O += V^T[:, 0:32] P0      |  P1 = silu(S1)
    //   C: O += V^T[:, 32:64] P1     |
    auto tile_body = [&](auto masked_tag, auto buf_tag, int k0, int nxt, auto fast_tag) __attribute__((always_inline)) {
      constexpr int BUF = decltype(buf_tag)::value;
      constexpr bool FAST = decltype(fast_tag)::value;  // the next tile exists and is whole
      // Tags 3 and 4 are the general predicate (1) decided per 32-key block: 3 keeps every pair of the
      // first block and tests the second, 4 tests the first and keeps none of the second.
      constexpr int TAG = decltype(masked_tag)::value;
      const std::integral_constant<int, TAG == 3 ? 0 : (TAG == 4 ? 1 : TAG)> blk0_tag{};
      const std::integral_constant<int, TAG == 3 ? 1 : (TAG == 4 ? 5 : TAG)> blk1_tag{};
      const char* kb = (const char*)(BUF ? Ks1 : Ks0);
      const char* vb = (const char*)(BUF ? Vs1 : Vs0);
      // LDS byte address of this lane's part of the tile's bias band; opaque per tile, so that the
      // element addresses stay this register plus a constant instead of becoming 64 hoisted registers
      unsigned rab_addr = (unsigned)(size_t)(BUF ? rabs1 : rabs0) + rab_lane;
      if (HAS_RAB) asm volatile("" : "+v"(rab_addr));
      const std::integral_constant<int, BUF ^ 1> other{};
      const f32x16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      auto k_frag = [&](int kvb, int kk) __attribute__((always_inline)) {
        return *(const bf16x8*)(kb + kvb * 32 * HD * 2 + (ks_rd ^ (unsigned)(kk * 32)));
      };
      auto v_frag = [&](int db, int s2) __attribute__((always_inline)) {
        const char* a = vb + (vt_rd ^ (unsigned)(db * 64)) + s2 * 16 * HD * 2;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)a);
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(a + 8 * HD * 2));
        const i16x8 both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        return __builtin_bit_cast(bf16x8, both);
      };
      // The slot schedule: every bf16 tile body but the one with the general mask predicate and no bias
      // (its mask state leaves this schedule too few registers: 7 % slower there); with a bias every
      // body (the other schedule would add the bias in the SiLU arithmetic: 2-3 % slower).
      if constexpr (!FP8 && (TAG != 1 || HAS_RAB)) {
        // Hand-placed schedule, one MFMA per slot with a scheduling fence after each:
        //   slots  0..7   S0 = K[0:32] Q^T            slots  8..15  S1 = K[32:64] Q^T
        //   slots 16..31  O^T[db] += V^T[db, s2] P^T[s2], key step s2 = (slot - 16) / 4, db = slot & 3
        // SiLU of the 32 scores a lane holds runs as 16 units of two scores (one packed word), one
        // unit per slot from slot 9 on, so that every packed word is ready four slots before the
        // MFMA that consumes it; the LDS fragment of slot s + PD is requested in slot s.
        f32x16 sblk[2];
        unsigned pw[2][8];
        bf16x8 F[32];
        int rng_base = 0;
        unsigned rng_w = 0;
        if (decltype(masked_tag)::value == 2) rng_of(k0, rng_base, rng_w);
        // slot in which the LDS fragment of slot s is requested (-1: before slot 0).  Six K fragments
        // open a tile; all sixteen would fit the registers that scores and packed P leave free at
        // that point, but measured 1-3 % slower (configurations 2 and 4).  V fragments run ten slots
        // ahead.  (The bodies that carry mask or clamping state: distance 6 for both.)
        constexpr int PDK = FAST ? (HAS_RAB ? DL_PDK_RAB : DL_PDK) : DL_PD_SLOW, PDV = FAST ? DL_PDV : DL_PD_SLOW;
        auto frag_req = [](int s) constexpr { return s < PDK ? -1 : (s < 16 ? s - PDK : max(s - PDV, 0)); };
        // slot 16 + j of the second contraction: accumulator db, key step s2
        auto pv_db = [](int s) constexpr { return (s - 16) & 3; };
        auto pv_s2 = [](int s) constexpr { return (s - 16) >> 2; };
        auto slot_frag = [&](int s) __attribute__((always_inline)) {
          // stand-ins differ per 32-key block so that the two score blocks stay distinct computations
          return s < 16 ? k_frag(s >> 3, s & 7) : v_frag(pv_db(s), pv_s2(s));
        };
        auto silu_unit = [&](int u) __attribute__((always_inline)) {
          const int blk = u >> 3, e = u & 7;
          const int MASKED = blk ? decltype(blk1_tag)::value : decltype(blk0_tag)::value;  // (folds: u is an unrolled loop's constant)
          if (MASKED == 5) { pw[blk][e] = 0u; return; }
          float pe[2];
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int r = 2 * e + t;
            const int jl = blk * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
            const float sv = sblk[blk][r];  // the bias is already in there, see bias_block
            const float tv = sv * neg_c;
            float pv = tv * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(tv));
            if (MASKED == 1) pv = kept(k0, blk * 32 + 8 * (r >> 2) + (r & 3)) ? pv : 0.f;
            if (MASKED == 2) pv = (unsigned)(rng_base + (blk * 32 + 8 * (r >> 2) + (r & 3))) <= rng_w ? pv : 0.f;
            pe[t] = pv;
          }
          pw[blk][e] = pack_bf16x2(pe[0], pe[1]);
        };
        // The bias enters as the initial value of the score accumulators (no addition in the SiLU
        // units, no register of its own): block 0 is read with the fragments that open the tile,
        // block 1 three slots before its first MFMA (any earlier and it competes with the K
        // fragments in flight).
        auto bias_block = [&](int blk) __attribute__((always_inline)) {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            sblk[blk][r] = *(lds_cfloat*)(rab_addr + 4u * (unsigned)(blk * 32 + 8 * (r >> 2) + (r & 3)));
        };
        if (HAS_RAB) bias_block(0);
#pragma unroll
        for (int s = 0; s < 32; ++s)
          if (frag_req(s) < 0) F[s] = slot_frag(s);
        // the copies of the next tile go out one per slot: a burst of eight would hold this wave's
        // MFMAs back for as long as the address unit takes to accept them
        const bool copy_next = FAST || nxt < nkv;
        auto issue_slot = [&](int part) __attribute__((always_inline)) {
          if constexpr (FAST) issue_part(nxt, other, std::true_type{}, part);
          else if (copy_next) issue_part(nxt, other, std::false_type{}, part);
        };
        // bias band of the next tile: loaded here, stored to LDS in the last slot
        float band_next = 0.f;
        if (HAS_RAB && copy_next) band_next = band_load(nxt);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < 32; ++s) {
#pragma unroll
          for (int t = s + 1; t < 32; ++t)
            if (frag_req(t) == s) F[t] = slot_frag(t);
          if (HAS_RAB && s == DL_B1) bias_block(1);
          __builtin_amdgcn_s_setprio(1);  // while an MFMA waits to issue
          if (s < 16) {
            sblk[s >> 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F[s], qf[s & 7], (!HAS_RAB && (s & 7) == 0) ? zero : sblk[s >> 3], 0, 0, 0);
          } else {
            const int s2 = pv_s2(s), db = pv_db(s);
            const u32x4 w = {pw[s2 >> 1][4 * (s2 & 1) + 0], pw[s2 >> 1][4 * (s2 & 1) + 1], pw[s2 >> 1][4 * (s2 & 1) + 2],
                             pw[s2 >> 1][4 * (s2 & 1) + 3]};
            acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F[s], __builtin_bit_cast(bf16x8, w), acc[db], 0, 0, 0);
          }
          __builtin_amdgcn_s_setprio(0);
          if (s < 8) issue_slot(s);  // one copy instruction of the next tile behind each of the first MFMAs
          if (s >= DL_U0 && s < DL_U0 + 16) silu_unit(s - DL_U0);
          if (HAS_RAB && s == 31 && copy_next) band_store(other, band_next, nxt);
          __builtin_amdgcn_sched_barrier(0);
        }
        return;
      }
      f32x16 s0, s1;
      bf16x8 pb0, pb1, pb2, pb3;
      float band_nxt = 0.f;
      if (HAS_RAB && (FAST || nxt < nkv)) band_nxt = band_load(nxt);
      // The 32 MFMAs of the block run as eight groups of four.  The LDS fragments of group g + 1 are
      // fetched while group g computes (two alternating sets of four registers-quads), so that no
      // MFMA waits for an LDS round trip; only the reads that open the tile are exposed.
      //   groups 0,1: S0 (K rows 0..31)    groups 2,3: S1 (K rows 32..63)   | P0 = silu(S0) over 2,3
      //   groups 4,5: O += V^T[:, 0:32] P0                                  | P1 = silu(S1) over 4,5
      //   groups 6,7: O += V^T[:, 32:64] P1
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
          if (g < 2) {
            const int kk = FP8 ? 0 : g * 4 + i;
            s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i], qf[kk], (g * 4 + i) == 0 ? zero : s0, 0, 0, 0);
          } else if (g < 4) {
            const int kk = FP8 ? 0 : (g - 2) * 4 + i;
            s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i], qf[kk], ((g - 2) * 4 + i) == 0 ? zero : s1, 0, 0, 0);
          } else {
            const int db = ((g & 1) * 2) + (i >> 1);
            const int s2 = ((g - 4) >> 1) * 2 + (i & 1);
            const bf16x8& pb = s2 == 0 ? pb0 : (s2 == 1 ? pb1 : (s2 == 2 ? pb2 : pb3));
            acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i], pb, acc[db], 0, 0, 0);
          }
        }
      };
      bf16x8 fa[4], fb[4];
      if constexpr (FP8) {
        // scores: two K = 64 MFMAs per 32 x 32 block; fragment = two 16-byte reads
        auto k8_frag = [&](int kvb, int st) __attribute__((always_inline)) {
          const char* a = kb + kvb * 32 * 128;
          const u32x4 lo = *(const u32x4*)(a + (k8_rd ^ (unsigned)((4 * st) * 16)));
          const u32x4 hi = *(const u32x4*)(a + (k8_rd ^ (unsigned)((4 * st + 1) * 16)));
          return (i32x8){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        };
        const i32x8 ka0 = k8_frag(0, 0), ka1 = k8_frag(0, 1);
        if constexpr (FAST) issue_tile_as(nxt, other, std::true_type{}); else if (nxt < nkv) issue_tile(nxt, other);
        const i32x8 kb0 = k8_frag(1, 0), kb1 = k8_frag(1, 1);
        s0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ka0, q8[0], zero, 0, 0, 0, 0x7f7f7f7f, 0, 0x7f7f7f7f);
        s0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ka1, q8[1], s0, 0, 0, 0, 0x7f7f7f7f, 0, 0x7f7f7f7f);
        __builtin_amdgcn_sched_barrier(0);
        load_group(4, fa);
        s1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(kb0, q8[0], zero, 0, 0, 0, 0x7f7f7f7f, 0, 0x7f7f7f7f);
        s1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(kb1, q8[1], s1, 0, 0, 0, 0x7f7f7f7f, 0, 0x7f7f7f7f);
        silu_pack(blk0_tag, s0, k0, 0, rab_addr, pb0, pb1);
      } else {
      load_group(0, fa);
      if constexpr (FAST) issue_tile_as(nxt, other, std::true_type{}); else if (nxt < nkv) issue_tile(nxt, other);
      load_group(1, fb);
      mfma_group(0, fa);
      __builtin_amdgcn_sched_barrier(0);
      load_group(2, fa);
      mfma_group(1, fb);
      __builtin_amdgcn_sched_barrier(0);
      // groups 2 and 3 with silu(S0)
      load_group(3, fb);
      mfma_group(2, fa);
      silu_pack(blk0_tag, s0, k0, 0, rab_addr, pb0, pb1);
      load_group(4, fa);
      mfma_group(3, fb);
      // MFMAs issue in pairs: the second of a back-to-back pair costs less issue time than a lone one
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);   // fragment reads of group 3 (8 for V)
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);   // 2 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 10, 0);  // 10 VALU
        __builtin_amdgcn_sched_group_barrier(0x400, 8, 0);   // 8 transcendental
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);   // fragment reads of group 4
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 10, 0);
        __builtin_amdgcn_sched_group_barrier(0x400, 8, 0);
      }
      }
      __builtin_amdgcn_sched_barrier(0);
      // groups 4 and 5 with silu(S1)
      load_group(5, fb);
      mfma_group(4, fa);
      silu_pack(blk1_tag, s1, k0, 1, rab_addr, pb2, pb3);
      load_group(6, fa);
      mfma_group(5, fb);
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 10, 0);
        __builtin_amdgcn_sched_group_barrier(0x400, 8, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 10, 0);
        __builtin_amdgcn_sched_group_barrier(0x400, 8, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      load_group(7, fb);
      mfma_group(6, fa);
      __builtin_amdgcn_sched_barrier(0);
      mfma_group(7, fb);
      if (HAS_RAB && (FAST || nxt < nkv)) band_store(other, band_nxt, nxt);
    };

    // ---- the skewed loop ----
    // Trip i (tile i in LDS stage i & 1), one MFMA per slot, a scheduling fence after each:
    //   slots  0..7   D(i-1): O^T += V^T[:, 32:64] P1(i-1)     second half of the previous tile
    //   slots  8..15  B(i)  : S1 = K(i)[32:64] Q^T
    //   slots 16..23  A(i+1): S0 = K(i+1)[0:32] Q^T            first half of the next tile
    //   slots 24..31  C(i)  : O^T += V^T[:, 0:32] P0(i)
    // so every slot has an MFMA and SiLU work for it to hide: one score enters a five-stage pipeline
    // per slot (t = s neg_c | exp2 | + 1 | rcp | t r and, every other slot, the bf16 pack), the 16 of
    // S0(i) in slots 0..15, the 16 of S1(i) in slots 16..31; the last of them leave it in slots 0..3
    // of the next trip, one slot before D(i) needs them.  The order of the accumulation into O is
    // that of the plain loop.  KIND: 0 first trip (no D), 1 middle, 2 last (no A), 3 the eight slots
    // of D after the last trip.
    f32x16 sk_s0, sk_s1;
    unsigned sk_pw0[8], sk_pw1[8];
    float sk_t[8], sk_r[8];
    auto skew_body = [&](auto buf_tag, auto kind_tag, int i) __attribute__((always_inline)) {
      constexpr int BUF = decltype(buf_tag)::value;
      constexpr int KIND = decltype(kind_tag)::value;
      constexpr int NSLOT = KIND == 3 ? 8 : 32;
      constexpr int PD = DL_SKEW_PD;
      const char* kc = (const char*)(BUF ? Ks1 : Ks0);
      const char* ko = (const char*)(BUF ? Ks0 : Ks1);
      const char* vc = (const char*)(BUF ? Vs1 : Vs0);
      const char* vo = (const char*)(BUF ? Vs0 : Vs1);
      const f32x16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      auto k_frag_at = [&](const char* kb, int kvb, int kk) __attribute__((always_inline)) {
        return *(const bf16x8*)(kb + kvb * 32 * HD * 2 + (ks_rd ^ (unsigned)(kk * 32)));
      };
      auto v_frag_at = [&](const char* vb, int db, int s2) __attribute__((always_inline)) {
        const char* a = vb + (vt_rd ^ (unsigned)(db * 64)) + s2 * 16 * HD * 2;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)a);
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(a + 8 * HD * 2));
        const i16x8 both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        return __builtin_bit_cast(bf16x8, both);
      };
      auto has_mfma = [](int s) constexpr {
        return KIND == 3 ? s < 8 : (KIND == 0 ? s >= 8 : (KIND == 2 ? (s < 16 || s >= 24) : true));
      };
      auto slot_frag = [&](int s) __attribute__((always_inline)) {
        if (s < 8) return v_frag_at(vo, s & 3, 2 + (s >> 2));
        if (s < 16) return k_frag_at(kc, 1, s - 8);
        if (s < 24) return k_frag_at(ko, 0, s - 16);
        return v_frag_at(vc, (s - 24) & 3, (s - 24) >> 2);
      };
      // SiLU pipeline stage `stage` (1..5) of the slot: it works on score n = s - (stage - 1) of this
      // trip, or on score n + 32 of the previous one
      auto silu_stage = [&](int s, int stage) __attribute__((always_inline)) {
        const int n = s - (stage - 1);
        if (n >= 0 ? KIND == 3 : KIND == 0) return;
        const int nn = (n + 32) & 31, e = nn & 7;
        if (stage == 1) sk_t[e] = (nn < 16 ? sk_s0[nn] : sk_s1[nn - 16]) * neg_c;
        else if (stage == 2) sk_r[e] = __builtin_amdgcn_exp2f(sk_t[e]);
        else if (stage == 3) sk_r[e] = 1.0f + sk_r[e];
        else if (stage == 4) sk_r[e] = __builtin_amdgcn_rcpf(sk_r[e]);
        else {
          sk_t[e] = sk_t[e] * sk_r[e];
          if (nn & 1) {
            const unsigned w = pack_bf16x2(sk_t[e - 1], sk_t[e]);
            if (nn < 16) sk_pw0[nn >> 1] = w; else sk_pw1[(nn - 16) >> 1] = w;
          }
        }
      };
      bf16x8 F[32];
#pragma unroll
      for (int s = 0; s < NSLOT; ++s)
        if (has_mfma(s) && s < PD) F[s] = slot_frag(s);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < NSLOT; ++s) {
        if (s + PD < NSLOT && has_mfma(s + PD)) F[s + PD] = slot_frag(s + PD);
        if (has_mfma(s)) {
          if (s < 8) {
            const int w0 = 4 * (s >> 2), db = s & 3;
            const u32x4 w = {sk_pw1[w0], sk_pw1[w0 + 1], sk_pw1[w0 + 2], sk_pw1[w0 + 3]};
            acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F[s], __builtin_bit_cast(bf16x8, w), acc[db], 0, 0, 0);
          } else if (s < 16) {
            sk_s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F[s], qf[s - 8], s == 8 ? zero : sk_s1, 0, 0, 0);
          } else if (s < 24) {
            sk_s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F[s], qf[s - 16], s == 16 ? zero : sk_s0, 0, 0, 0);
          } else {
            const int w0 = 4 * ((s - 24) >> 2), db = (s - 24) & 3;
            const u32x4 w = {sk_pw0[w0], sk_pw0[w0 + 1], sk_pw0[w0 + 2], sk_pw0[w0 + 3]};
            acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F[s], __builtin_bit_cast(bf16x8, w), acc[db], 0, 0, 0);
          }
        }
        if (KIND != 3 && s < 8 && !(KIND == 0 && s >= 6) && !(KIND == 2 && s < 2)) skew_copy(i, buf_tag, s);
#pragma unroll
        for (int stage = 5; stage >= 1; --stage) silu_stage(s, stage);
        __builtin_amdgcn_sched_barrier(0);
      }
    };

    auto compute_tile = [&](int it, auto buf_tag, int nxt) __attribute__((always_inline)) {
      constexpr int BUF = decltype(buf_tag)::value;
      const int k0 = it * BN;
      const int k1 = k0 + BN;
      // wave-level classification of this (32 query rows) x (64 keys) block
      bool any_kept = wave_has_rows && ((k0 <= m_hi && k1 > m_lo) /* diagonal crosses */ ||
                                        (k0 < si.cap && k0 <= m_hi) /* causal history */ ||
                                        (k0 < si.ctx_eff));
      if (SEMI)  // history keys count only inside some row's window
        any_kept = wave_has_rows && ((k0 <= m_hi && k1 > m_lo) || (k0 < si.ctx_eff) ||
                                     (k0 < idhi_w && (wave_has_tail || k1 > idlo_w - si.win)));
      if (!any_kept) {
        if (nxt < nkv) issue_tile_and_band(nxt, std::integral_constant<int, BUF ^ 1>{});  // this wave still copies its share
        return 4;
      }
      bool full = (k1 - 1 <= m_lo) && (k1 <= si.cap);  // implies k1 <= n
      if (SEMI) full = full && (idlo_w >= si.tail0 || k0 >= idhi_w - si.win);  // inside every row's window
      // semi-local, history rows only and no contextual key in the tile: the range form of the mask
      const bool range_mask = SEMI && m_hi < si.cap && k0 >= si.ctx_eff;
      if (full) tile_body(std::integral_constant<int, 0>{}, buf_tag, k0, nxt, std::false_type{});
      else if (SEMI && range_mask) tile_body(std::integral_constant<int, 2>{}, buf_tag, k0, nxt, std::false_type{});
      else if (!SEMI && (k0 + 31 <= m_lo) && (k0 + 32 <= si.cap))  // first 32 keys kept by every row of the wave
        tile_body(std::integral_constant<int, 3>{}, buf_tag, k0, nxt, std::false_type{});
      else if (!SEMI && (k0 + 32 > m_hi) && (k0 + 32 >= si.ctx_eff))  // last 32 keys above every row, none contextual
        tile_body(std::integral_constant<int, 4>{}, buf_tag, k0, nxt, std::false_type{});
      else tile_body(std::integral_constant<int, 1>{}, buf_tag, k0, nxt, std::false_type{});
      return full ? 2 : 3;  // class of the tile for this wave (phase-trace builds): 2 unmasked, 3 partial, 4 skipped
    };

    // Leading tiles this wave runs without classifying them: unmasked for all of its rows
    // (64 t + 63 <= m_lo and 64 t + 64 <= cap), inside the first contiguous run of the walk, and
    // followed by a tile that exists and is whole.  Taken in pairs (stage 0, stage 1).
    int fast_pairs = 0;
    if (!SEMI && wave_has_rows && it == 0) {
      const int run_end = has_skip ? skip_a : nkv;
      int fast_end = min(min((m_lo + 1) / BN, cap0 / BN), min(run_end - 1, si.n / BN - 1));
      fast_pairs = max(fast_end, 0) / 2;
    }

    if (it < nkv) {
      if (HAS_RAB) band_store(std::integral_constant<int, 0>{}, band_first, it);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      HSTU_TR(tr_ready = wall_clock64(); tr_c0_item = clock64(); unsigned long long tr_t = tr_ready;)
      if (SKEW && skew_tiles) {
        const std::integral_constant<int, 0> st0{};
        const std::integral_constant<int, 1> st1{};
        {  // S0 of tile 0
          const f32x16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
          bf16x8 f0[8];
#pragma unroll
          for (int kk = 0; kk < 8; ++kk) {
            f0[kk] = *(const bf16x8*)((const char*)Ks0 + (ks_rd ^ (unsigned)(kk * 32)));
          }
#pragma unroll
          for (int kk = 0; kk < 8; ++kk) sk_s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f0[kk], qf[kk], kk == 0 ? zero : sk_s0, 0, 0, 0);
        }
        __syncthreads();  // the first trip refills the K rows just read
        skew_body(st0, std::integral_constant<int, 0>{}, 0);
        HSTU_DL_TILE_SYNC();
        for (int i = 1; i + 1 < skew_tiles; i += 2) {
          skew_body(st1, std::integral_constant<int, 1>{}, i);
          HSTU_DL_TILE_SYNC();
          skew_body(st0, std::integral_constant<int, 1>{}, i + 1);
          HSTU_DL_TILE_SYNC();
        }
        skew_body(st1, std::integral_constant<int, 2>{}, skew_tiles - 1);
        HSTU_DL_TILE_SYNC();
        // V rows 32..63 of the tile the plain loop takes over with; the second half of the last skewed tile
        skew_copy(skew_tiles, st0, 6);
        skew_copy(skew_tiles, st0, 7);
        skew_body(st0, std::integral_constant<int, 3>{}, skew_tiles);
        HSTU_DL_TILE_SYNC();
        it = skew_tiles;
        fast_pairs = 0;
        HSTU_TR({ const unsigned long long t = wall_clock64(); tr_ticks[0] += t - tr_t; tr_t = t; tr_count[0] += skew_tiles; })
      }
      for (int pi = 0; pi < fast_pairs; ++pi) {
        tile_body(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, it * BN, it + 1, std::true_type{});
        HSTU_DL_TILE_SYNC();
        tile_body(std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{}, (it + 1) * BN, it + 2, std::true_type{});
        HSTU_DL_TILE_SYNC();
        it += 2;
      }
      HSTU_TR(if (fast_pairs) { const unsigned long long t = wall_clock64(); tr_ticks[1] += t - tr_t; tr_t = t; tr_count[1] += 2 * fast_pairs; })
      // two tiles per trip so that the stage index is a compile-time constant
      while (true) {
        int nxt = next_tile(it);
        int cls = compute_tile(it, std::integral_constant<int, 0>{}, nxt);
        if (nxt < nkv) {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's copies of tile nxt have landed
          __syncthreads();                                   // ... and everybody's; tile it is no longer read
        }
        HSTU_TR({ const unsigned long long t = wall_clock64(); tr_ticks[cls] += t - tr_t; tr_t = t; tr_count[cls] += 1; })
        if (nxt >= nkv) break;
        it = nxt;
        nxt = next_tile(it);
        cls = compute_tile(it, std::integral_constant<int, 1>{}, nxt);
        if (nxt < nkv) {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
          __syncthreads();
        }
        HSTU_TR({ const unsigned long long t = wall_clock64(); tr_ticks[cls] += t - tr_t; tr_t = t; tr_count[cls] += 1; })
        if (nxt >= nkv) break;
        it = nxt;
      }
    }

    HSTU_TR(const unsigned long long tr_loop_end = wall_clock64(); const long long tr_c1 = clock64();)
    // ---- epilogue: O^T accumulators -> out[s + m, h, :] ----
    if (m < q_end) {
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
#ifdef HSTU_TRACE
    if (p.trace && lane == 0) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the output rows have left
      unsigned hwid, xcc;
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hwid));
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
      unsigned long long* rec = p.trace + (((size_t)xcd * p.items_cap + slot) * 4 + wave) * TRACE_WORDS;
      rec[0] = tr_start; rec[1] = tr_ready; rec[2] = tr_loop_end; rec[3] = wall_clock64();
      for (int i = 0; i < 5; ++i) rec[4 + i] = tr_ticks[i];
      rec[9] = (unsigned long long)tr_count[0] | ((unsigned long long)tr_count[1] << 8) | ((unsigned long long)tr_count[2] << 16) |
               ((unsigned long long)tr_count[3] << 24) | ((unsigned long long)tr_count[4] << 32);
      rec[10] = ((unsigned long long)xcc << 32) | hwid;
      rec[11] = (unsigned long long)(tr_c1 - tr_c0_item);
    }
#endif
    __syncthreads();  // LDS buffers are reused by the next item
  }  // work items
  // rows behind the last sequence: after the items, so that no workgroup waits for seq_offsets[B] before it starts
  zero_tail_rows<256>(p, (size_t)p.H * HD * 2);
}

}  // namespace recir_hstu
