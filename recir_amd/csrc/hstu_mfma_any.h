// MFMA kernels of the HSTU attention forward and backward for everything the kernels written for
// head dim 128 do not take: any head dims up to 256 (fp32: 128), Dqk and Dv independent; bf16, fp16
// or fp32 values; tensors at any address their element type allows; every mask the operator knows (causal with targets
// and contextual prefix, semi-local, the non-causal forms); a bias with any alpha, and the gradient of
// the bias table.  One template, five modes; nothing here is hand-scheduled: the point is to keep such
// calls on the matrix cores (1.4 to 1.9 times the time of the head-dim-128 kernels at their own shape)
// instead of on the one-wave-per-token kernels (two orders of magnitude slower).
//
// A workgroup (4 waves) owns 128 "stationary" rows of one (sequence, head), 32 per wave, one per lane
// of a 32-lane half; their operands stay in registers.  The other side is streamed through LDS in
// tiles of 64 rows.  With c a stationary row and r a streamed row:
//   FWD  c = query, r = key     S^T[r,c] = K[r,:] . Q[c,:]
//                               O^T[:,c] += V^T[:,r] P^T[r,c]
//   DQ   c = query, r = key     S^T as above, dP^T[r,c] = V[r,:] . dO[c,:]
//                               dQ^T[:,c] += K^T[:,r] dS^T[r,c]
//   DKV  c = key,   r = query   S[r,c] = Q[r,:] . K[c,:],  dP[r,c] = dO[r,:] . V[c,:]
//                               dV^T[:,c] += dO^T[:,r] P[r,c],  dK^T[:,c] += Q^T[:,r] dS[r,c]
//   DV, DK                      the two halves of DKV as passes of their own (the largest padded head
//                               dim, where both accumulators and both operand sets do not fit one
//                               wave's registers)
//   x = alpha S + bias;  P = silu(x) keep;  dS = dP silu'(x) keep   (dO . V is dP)
//   out = scale P V;  dQ = alpha scale dS K;  dK = alpha (scale dS)^T Q;  dV = (scale P)^T dO
// The scale of a query row multiplies a column in FWD and DQ (applied to the accumulators at the
// end) and a streamed row in the key-stationary modes (applied per element when it is per token;
// fp16: times a power of two taken from the largest scale of the item's rows and divided out of the
// accumulators at the end, so that P and dS times a scale of the order of 1 / max_seq_len stay in
// fp16's normal range).
//
// bf16 and fp16: every product is v_mfma_f32_32x32x16 with the streamed tile as the A operand: rows
// of the tile for the score products (ds_read_b128), the transposed tile for the accumulating
// products (ds_read_b64_tr_b16 on the same row-major tile).  The 32 x 32 accumulator layout of a
// score block (lane = c, registers = r) is the B-operand layout of the accumulating product, so P
// and dS go from one MFMA to the next through registers only.
//
// fp32 (DP up to 128) takes the same walk with v_mfma_f32_32x32x2_f32, one element per lane and
// operand: lane half h contracts elements h DP / 2 .. of the head dim in the score products and its
// own streamed rows in the accumulating ones, whose B operand is the score block's register as it
// is and whose A operand is a plain 4-byte LDS read (consecutive lanes, consecutive columns); P and
// dS are not rounded.  A sixteenth of the bf16 rate, and still some twenty times the generic kernel.
//
// Head dims are padded to DP in {32, 64, 128, 256} with zeros (16-byte chunks past Dqk or Dv are not
// loaded or stored); both dims share the larger padding.  ALIGNED: every row of every tensor starts at
// a multiple of 16 bytes (head dims multiples of 8 elements, fp32: 4, and aligned base addresses), and
// rows move in 16-byte pieces that the kernel knows to be aligned; otherwise (a head dim of 25 or 50, a
// view that starts in the middle of a row) in pieces aligned to the element only, the last few elements
// of a row one by one, zeros in the padding, and everything after the staging is the same.
#pragma once
#include <type_traits>

#include "hstu_common.h"

namespace recir_hstu {

typedef __attribute__((ext_vector_type(8))) _Float16 any_f16x8;
typedef __attribute__((ext_vector_type(2))) _Float16 any_f16x2;
typedef __attribute__((ext_vector_type(4))) short any_i16x4;
typedef __attribute__((address_space(3))) any_i16x4 any_lds_i16x4;

#ifndef HSTU_ANY_RING
#define HSTU_ANY_RING 2
#endif
#ifndef HSTU_ANY_READ_AHEAD
#define HSTU_ANY_READ_AHEAD 1  // (0: a measurement build without the fragments read ahead)
#endif

constexpr int ANY_FWD = 0, ANY_DQ = 1, ANY_DKV = 2, ANY_DV = 3, ANY_DK = 4;  // modes (DV, DK: the two halves of DKV as passes of their own)
constexpr int ANY_BF16 = 0, ANY_F16 = 1, ANY_F32 = 2;                        // element types (the template's ELT)
constexpr int ANY_BM = 128;  // stationary rows per workgroup
constexpr int ANY_BN = 64;   // streamed rows per tile
constexpr float kAnyLog2e = 1.4426950408889634f;

template <bool F16>
__device__ __forceinline__ f32x16 any_mfma(const u32x4& a, const u32x4& b, const f32x16& c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(any_f16x8, a), __builtin_bit_cast(any_f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <bool F16>
__device__ __forceinline__ unsigned any_pack2(float lo, float hi) {
  if constexpr (F16) {
    const f32x2 t = {lo, hi};
    const any_f16x2 y = __builtin_convertvector(t, any_f16x2);
    return __builtin_bit_cast(unsigned, y);
  } else {
    return pack_bf16x2(lo, hi);
  }
}

// 16 bytes of a row of D elements from an address aligned to the element only; n = elements left in the
// row from there.  A full piece is one 16-byte load (the hardware's unaligned access mode, which the
// compiler relies on for every under-aligned global access).  The row's last piece, when it holds one
// or two elements (head dims 25, 50), is read element by element; when it holds more, with a 16-byte
// load moved back so that it ends with the row, and the value shifted down, zeros coming in from above
// (distance and shift are the same for every lane: D decides).  Nothing is read outside the row (what
// follows the last row need not be mapped).  Rows shorter than 16 bytes are read element by element.
typedef u32x4 __attribute__((aligned(2))) any_u32x4_a2;
typedef u32x4 __attribute__((aligned(4))) any_u32x4_a4;
typedef u32x2 __attribute__((aligned(2))) any_u32x2_a2;
template <int ES>
__device__ __forceinline__ u32x4 any_load_elems(const char* src, int n, int D) {
  constexpr int EPC = 16 / ES;
  typedef typename std::conditional<ES == 4, any_u32x4_a4, any_u32x4_a2>::type piece;
  typedef typename std::conditional<ES == 4, unsigned, unsigned short>::type elem;
  const elem* s = (const elem*)src;
  u32x4 r = {0u, 0u, 0u, 0u};
  if (D >= EPC) {
    const int last = D % EPC;  // elements of the row's last piece (0: every piece is full)
    if (n >= EPC) {
      r = *(const piece*)src;
    } else if (n > 0) {
      if (last <= 2) {
        const unsigned e0 = s[0], e1 = last > 1 ? (unsigned)s[1] : 0u;
        if constexpr (ES == 4) { r.x = e0; r.y = e1; }
        else r.x = e0 | (e1 << 16);
      } else {
        r = *(const piece*)(src - (EPC - last) * ES);
        r = __builtin_bit_cast(u32x4, __builtin_bit_cast(unsigned __int128, r) >> ((EPC - last) * ES * 8));
      }
    }
  } else {
    unsigned e[EPC];
#pragma unroll
    for (int i = 0; i < EPC - 1; ++i) e[i] = n > i ? (unsigned)s[i] : 0u;
    if constexpr (ES == 4) { r.x = e[0]; r.y = e[1]; r.z = e[2]; }
    else { r.x = e[0] | (e[1] << 16); r.y = e[2] | (e[3] << 16); r.z = e[4] | (e[5] << 16); r.w = e[6]; }
  }
  return r;
}

template <int MODE, int ELT, int DP>
constexpr int any_workgroups_per_cu() {
  return ((ELT != ANY_F32 && ((MODE == ANY_FWD && DP <= 128) || DP <= 64)) || (MODE == ANY_FWD && DP <= 64)) ? 2 : 1;
}

// Two workgroups per CU where the registers allow it (a few spills included: one workgroup per CU
// measured 20-35 % slower at these shapes).
// HAS_RAB: with a bias table (an instantiation of its own: tested per pair the pointer costs seven scalar
// instructions a score, and as a second set of tile bodies inside one kernel it costs registers).
template <int MODE, int ELT, int DP, bool HAS_RAB, bool ALIGNED>
__global__ __launch_bounds__(256, (any_workgroups_per_cu<MODE, ELT, DP>()))
__attribute__((amdgpu_waves_per_eu((any_workgroups_per_cu<MODE, ELT, DP>()), (any_workgroups_per_cu<MODE, ELT, DP>())))) void hstu_mfma_any(BwdParams bp) {
  const Params& p = bp.f;
  constexpr bool F16 = ELT == ANY_F16;
  constexpr bool F32 = ELT == ANY_F32;  // v_mfma_f32_32x32x2_f32: one element per lane and operand, see below
  constexpr int ES = F32 ? 4 : 2;       // bytes per element
  constexpr bool KEYS = MODE >= ANY_DKV;                                  // the stationary rows are keys
  constexpr bool HAS_DP = MODE == ANY_DQ || MODE == ANY_DKV || MODE == ANY_DK;   // dP, dS and the product that dS feeds
  constexpr bool HAS_P = MODE == ANY_FWD || MODE == ANY_DKV || MODE == ANY_DV;   // the product that P feeds
  constexpr int NK = DP * ES / 32;  // 16-byte registers-quads of a stationary row per lane (bf16, fp16: steps of 16 along the head dim)
  constexpr int NB = DP / 32;       // 32-row blocks of a transposed accumulator
  constexpr int RS = DP * ES + 16;  // bytes between tile rows in LDS (the 16 spread the rows over the banks)
  constexpr int CPR = DP * ES / 16; // 16-byte chunks per tile row
  constexpr int NCH = DP * ES / 64; // chunks of one tile that one thread stages
  constexpr int EPC = 16 / ES;      // elements per chunk
  // Forward without a bias in bf16 or fp32: P / alpha = s sigmoid(alpha s) goes into the second product and
  // alpha onto the output rows (one multiplication less per score; not in fp16, whose range P / alpha could leave)
  constexpr bool FOLD_ALPHA = MODE == ANY_FWD && !HAS_RAB && !F16;
  // LDS fragments read a step ahead of the products that take them, kept in that order by scheduling barriers:
  // 3 % where the fragments of a step are few; at padded head dims above 64 their registers cost more
  constexpr bool READ_AHEAD = HSTU_ANY_READ_AHEAD && DP <= 64;
  // above that, in the backward modes: each fragment requested this many products ahead of its own (0: read
  // where it is used; the forward with a bias measured 3 % slower with it, without one 2 % faster)
  constexpr int RING = (READ_AHEAD || MODE == ANY_FWD) ? 0 : HSTU_ANY_RING;
  // The accumulating products stand once, behind the three kinds of tile body, instead of inside each:
  // as the results of several bodies the accumulators were copied once a tile (8-14 % of the time where
  // they are few); where they are many the packed P and dS kept across the bodies' end cost more in spills.
  constexpr bool ACC_APART = (MODE == ANY_FWD && DP <= 128) || DP <= 64;
  static_assert(DP == 32 || DP == 64 || DP == 128 || DP == 256, "padded head dim");
  static_assert(!F32 || DP <= 128, "fp32 tiles of 256 columns do not fit the LDS");
  __shared__ __attribute__((aligned(16))) unsigned char Y1s[2][ANY_BN * RS];
  __shared__ __attribute__((aligned(16))) unsigned char Y2s[2][ANY_BN * RS];
  __shared__ float bias_s[2][ANY_BM + ANY_BN];
  __shared__ float scale_s[2][ANY_BN];
  __shared__ float red_s[4];
  // DQ with the gradient of the bias table: dS of a tile summed along its 191 diagonals as fixed-point
  // integers, one band per LDS stage (integer LDS atomics; float ones run a lane at a time and tripled the
  // backward); the band of tile t goes out to the head's 64-bit table while tile t + 1 is computed.  Integer
  // additions commute: the gradient does not depend on the order of the workgroups.
  __shared__ int dband_s[2][MODE == ANY_DQ ? ANY_BM + ANY_BN : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // (a scalar: what depends on the wave alone then branches without lane masks)
  const int l32 = lane & 31;
  const int half = lane >> 5;
  // row fragment (A operand, 32 rows x 16 elements): lane reads row l32 (+ 32 blk), elements 16 kk + 8 half .. + 7
  const unsigned row_rd = (unsigned)l32 * RS + (unsigned)half * 16u;
  // transposed fragment (A operand, 32 columns of the tile x 16 rows): lane s = lane & 15 of a 16-lane
  // group supplies the 8 bytes at row 4 half + (s >> 2) (+ 16 s2, + 8 for the second read), column
  // 32 db + 16 group + 4 (s & 3) .. + 3; the lanes receive rows {4 half .. + 3, 8 + 4 half .. + 3} of
  // column 32 db + l32, which is the row order of the accumulator registers that feed the B operand
  const int tr_s = lane & 15;
  const unsigned tr_rd = (unsigned)(4 * half + (tr_s >> 2)) * RS + (unsigned)(32 * ((lane >> 4) & 1) + 8 * (tr_s & 3));

  if (MODE == ANY_FWD) zero_tail_rows_of<256>(p, p.out, (size_t)p.H * p.Dv * ES);
  if (MODE == ANY_DQ) zero_tail_rows_of<256>(p, bp.dq, (size_t)p.H * p.Dqk * ES);
  if (KEYS && HAS_DP) zero_tail_rows_of<256>(p, bp.dk, (size_t)p.H * p.Dqk * ES);
  if (KEYS && HAS_P) zero_tail_rows_of<256>(p, bp.dv, (size_t)p.H * p.Dv * ES);

  const bool noncausal = (p.flags & RECIR_HSTU_FLAG_MASK_NONCAUSAL) != 0;
  const bool per_token = p.attn_scale && (p.flags & RECIR_HSTU_FLAG_SCALE_PER_TOKEN);
  const bool semi = p.max_attn_len > 0;
  const float neg_log2e = -kAnyLog2e;
  const float neg_alpha_log2e = -kAnyLog2e * p.alpha;
  const int rab_w = 2 * p.N - 1;
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  const f32x16 zero16 = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // 16 bytes of a row of D elements from element d0 on (src points at that element); zeros past D
  auto ld16 = [&](const char* src, int d0, int D) __attribute__((always_inline)) {
    if constexpr (ALIGNED) return d0 < D ? *(const u32x4*)src : zero4;
    else return any_load_elems<ES>(src, D - d0, D);
  };

  const int xcd = blockIdx.x % NUM_XCD;
  const int list_len = p.ws_counts[xcd];
  const WorkItem* __restrict__ list = p.ws_items + (size_t)xcd * p.items_cap;
  for (int slot = blockIdx.x / NUM_XCD; slot < list_len; slot += p.grid_slots) {
    const WorkItem wi = list[slot];
    SeqInfo si;
    si.s = wi.s; si.n = wi.n; si.cap = wi.cap; si.ctx_eff = wi.ctx_eff;
    mask_window(p, si.cap, si.win, si.tail0);
    const int c0 = wi.q0, c_end = wi.q_end, h = wi.h;  // stationary rows [c0, c_end) of the sequence
    const int cap0 = si.cap > 0 ? si.cap : 0;

    // tensors by role: *1 has Dqk elements per row, *2 has Dv
    const char* __restrict__ X1g = (const char*)(KEYS ? p.k : p.q);
    const char* __restrict__ X2g = (const char*)(KEYS ? p.v : bp.dout);
    const char* __restrict__ Y1g = (const char*)(KEYS ? p.q : p.k);
    const char* __restrict__ Y2g = (const char*)(KEYS ? bp.dout : p.v);
    const size_t rb1 = (size_t)p.H * p.Dqk * ES, rb2 = (size_t)p.H * p.Dv * ES;
    const size_t hb1 = (size_t)h * p.Dqk * ES, hb2 = (size_t)h * p.Dv * ES;
    const float* __restrict__ rabg = HAS_RAB ? p.rab + (size_t)h * rab_w : nullptr;
    long long* __restrict__ drabg = (HAS_RAB && MODE == ANY_DQ && bp.drab_fx) ? bp.drab_fx + (size_t)h * rab_w : nullptr;

    // ---- stationary operands (B operand of the score products): lane holds row c ----
    const int cw0 = c0 + wave * 32;
    const int c = cw0 + l32;
    const bool c_valid = c < c_end;
    const int c_lo = cw0, c_hi = min(cw0 + 31, c_end - 1);
    const bool wave_has_rows = c_lo < c_end;
    u32x4 x1[NK], x2[HAS_DP ? NK : 1];
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      // bf16, fp16: elements 16 kk + 8 half .. + 7 (one MFMA step);  fp32: lane half h owns elements
      // h DP / 2 .. + DP / 2 - 1, four per register quad (one MFMA step each)
      const int d0 = F32 ? half * (DP / 2) + 4 * kk : kk * 16 + half * 8;
      x1[kk] = c_valid ? ld16(X1g + (size_t)(si.s + c) * rb1 + hb1 + (size_t)d0 * ES, d0, p.Dqk) : zero4;
      if constexpr (HAS_DP) x2[kk] = c_valid ? ld16(X2g + (size_t)(si.s + c) * rb2 + hb2 + (size_t)d0 * ES, d0, p.Dv) : zero4;
    }

    f32x16 acc1[HAS_DP ? NB : 1];  // DQ: dQ^T   DKV, DK: dK^T
    f32x16 acc2[HAS_P ? NB : 1];   // FWD: O^T   DKV, DV: dV^T
#pragma unroll
    for (int i = 0; i < (HAS_DP ? NB : 1); ++i) acc1[i] = zero16;
#pragma unroll
    for (int i = 0; i < (HAS_P ? NB : 1); ++i) acc2[i] = zero16;

    // ---- streamed rows: tiles [t_begin, t_end) of 64, minus the run [skip_a, skip_b) ----
    int t_begin = 0, t_end = 0, skip_a = 0, skip_b = 0;
    if (noncausal) {
      // mirrored window on the target-clamped ids (the diagonal alone without a window); a contextual
      // key or a row of the full-attention tail opens the whole sequence
      const bool tail_set = si.tail0 != 0x7fffffff;
      const int idc_lo = min(c0, si.cap), idc_hi = min(c_end - 1, si.cap);
      const bool whole = KEYS ? (c0 < si.ctx_eff || tail_set) : (si.ctx_eff > 0 || (tail_set && idc_hi >= si.tail0));
      int r_begin = 0, r_end = si.n;
      if (!whole) {
        if (si.win == WIN_ALL) {
          r_begin = c0;
          r_end = c_end;
        } else {
          r_begin = max(idc_lo - si.win, 0);
          r_end = idc_hi + si.win >= si.cap ? si.n : idc_hi + si.win + 1;
        }
      }
      t_begin = r_begin / ANY_BN;
      t_end = (r_end + ANY_BN - 1) / ANY_BN;
    } else if (!KEYS) {  // keys
      const int r_end = min(si.n, max(c_end, si.ctx_eff));
      t_end = (r_end + ANY_BN - 1) / ANY_BN;
      // semi-local: keys below the window of the first row, unless a row of the full-attention
      // tail or a contextual key needs them
      if (semi && si.ctx_eff <= 0 && min(c_end - 1, si.cap) < si.tail0) t_begin = max(min(c0, si.cap) - si.win, 0) / ANY_BN;
      // tiles that hold only target keys off this item's diagonal (and no contextual key)
      skip_a = (max(cap0, si.ctx_eff) + ANY_BN - 1) / ANY_BN;
      skip_b = c0 / ANY_BN;
    } else {  // queries
      const int r_begin = c0 < si.ctx_eff ? 0 : c0;  // a key is seen by its own and later rows (a contextual key by all)
      const int r_end = c0 >= max(cap0, si.ctx_eff) ? c_end : si.n;  // target keys: only by their own rows
      t_begin = r_begin / ANY_BN;
      t_end = (r_end + ANY_BN - 1) / ANY_BN;
    }
    // fp16 with a per-token scale, DKV: 2^-e with 2^(e-1) <= largest |scale| of the streamed rows < 2^e
    float pow2_up = 1.0f, pow2_down = 1.0f;
    if constexpr (KEYS && F16) {
      if (per_token) {
        float mx = 0.f;
        for (int r = t_begin * ANY_BN + tid; r < min(t_end * ANY_BN, si.n); r += 256) mx = fmaxf(mx, fabsf(p.attn_scale[si.s + r]));
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) mx = fmaxf(mx, __shfl_xor(mx, d, 64));
        if (lane == 0) red_s[wave] = mx;
        __syncthreads();
        mx = fmaxf(fmaxf(red_s[0], red_s[1]), fmaxf(red_s[2], red_s[3]));
        const int e = (int)((__float_as_uint(mx) >> 23) & 0xffu) - 126;  // mx < 2^e
        if (mx > 0.f && mx < 3.0e38f) {
          const int ec = min(max(e, -100), 100);
          pow2_up = __uint_as_float((unsigned)(127 - ec) << 23);
          pow2_down = __uint_as_float((unsigned)(127 + ec) << 23);
        }
      }
    }
    float uni = 1.0f / (float)p.N;  // the scale where it is the same for every row
    if (p.attn_scale && !per_token) uni = p.attn_scale[0];
    // scale of this lane's stationary row (queries), or what is left to apply to the key rows' sums
    const float col_scale = KEYS ? (per_token ? pow2_down : uni) : ((per_token && c_valid) ? p.attn_scale[si.s + c] : uni);
    // DQ: what dS is multiplied by on its way into the bias table's gradient: the head's fixed-point scale (a
    // power of two from a bound on |dS|, hstu_common.h) and a per-token scale of its row (a scale that is the
    // same for every row is applied when the table is converted back)
    float dscale = 0.f;
    if constexpr (MODE == ANY_DQ && HAS_RAB) {
      if (drabg) {
        float fx_scale, fx_inv;
        drab_fx_scales(drab_fx_bound(bp, h, per_token), fx_scale, fx_inv);
        dscale = c_valid ? (per_token ? col_scale : 1.0f) * fx_scale : 0.f;
      }
    }

    const bool has_skip = skip_a < skip_b;
    auto next_tile = [&](int t) { return (has_skip && t + 1 == skip_a) ? skip_b : t + 1; };

    // ---- staging: global -> registers -> LDS ----
    struct Staged {
      u32x4 y1[NCH], y2[NCH];
      float bias, scale;
    };
    auto load_tiles = [&](int t, Staged& st) __attribute__((always_inline)) {
      const int r0 = t * ANY_BN;
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int idx = tid + 256 * i;
        const int row = idx / CPR, ch = idx % CPR;
        const int rr = min(r0 + row, si.n - 1);  // rows past the sequence re-read its last row; the mask drops them
        st.y1[i] = ld16(Y1g + (size_t)(si.s + rr) * rb1 + hb1 + (size_t)ch * 16, ch * EPC, p.Dqk);
        st.y2[i] = ld16(Y2g + (size_t)(si.s + rr) * rb2 + hb2 + (size_t)ch * 16, ch * EPC, p.Dv);
      }
      st.bias = 0.f;
      if (HAS_RAB && tid < ANY_BM + ANY_BN - 1) {
        // entry e of the band holds the bias of m - j = dmin + e
        const int dmin = KEYS ? r0 - c0 - (ANY_BM - 1) : c0 - r0 - (ANY_BN - 1);
        // (a diagonal outside the table, possible only in a sequence longer than max_seq_len, has no bias)
        const int idx = dmin + tid + p.N - 1;
        st.bias = (idx >= 0 && idx < rab_w) ? rabg[idx] : 0.f;
      }
      st.scale = 1.0f;
      if (KEYS && per_token && tid < ANY_BN) st.scale = p.attn_scale[si.s + min(r0 + tid, si.n - 1)] * pow2_up;
    };
    auto store_tiles = [&](int buf, const Staged& st) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int idx = tid + 256 * i;
        const int row = idx / CPR, ch = idx % CPR;
        *(u32x4*)(&Y1s[buf][row * RS + ch * 16]) = st.y1[i];
        *(u32x4*)(&Y2s[buf][row * RS + ch * 16]) = st.y2[i];
      }
      if (HAS_RAB && tid < ANY_BM + ANY_BN - 1) bias_s[buf][tid] = st.bias;
      if (KEYS && tid < ANY_BN) scale_s[buf][tid] = st.scale;
    };

    auto row_frag = [&](const unsigned char* y, int blk, int kk) __attribute__((always_inline)) {
      return *(const u32x4*)(y + blk * 32 * RS + row_rd + kk * 32);
    };
    auto tr_frag = [&](const unsigned char* y, int db, int s2) __attribute__((always_inline)) {
      const unsigned char* a = y + tr_rd + s2 * 16 * RS + db * 64;
      const any_i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((any_lds_i16x4*)a);
      const any_i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((any_lds_i16x4*)(a + 8 * RS));
      u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
      return (u32x4){l2.x, l2.y, h2.x, h2.y};
    };

    // scores of one 32-row block of a tile against the stationary rows: y rows as the A operand
    auto row_product = [&](const unsigned char* y, int blk, const u32x4 (&x)[NK]) __attribute__((always_inline)) {
      f32x16 acc;
      if constexpr (F32) {
        // lane (row l32, half h) reads elements h DP / 2 + 4 kk .. + 3 of its row: four MFMA steps of one element each
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) {
          const u32x4 a = *(const u32x4*)(y + (blk * 32 + l32) * RS + (half * (DP / 2) + 4 * kk) * 4);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a[e]), __uint_as_float(x[kk][e]), (kk == 0 && e == 0) ? zero16 : acc, 0, 0, 0);
        }
      } else {
        if constexpr (!READ_AHEAD && RING > 0) {
          u32x4 a[NK];
#pragma unroll
          for (int kk = 0; kk < RING; ++kk) a[kk] = row_frag(y, blk, kk);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int kk = 0; kk < NK; ++kk) {
            if (kk + RING < NK) a[kk + RING] = row_frag(y, blk, kk + RING);
            acc = any_mfma<F16>(a[kk], x[kk], kk == 0 ? zero16 : acc);
            __builtin_amdgcn_sched_barrier(0);
          }
          return acc;
        }
        // fragments read ahead in groups of up to eight (left in one loop the compiler reads and waits one at a time)
        constexpr int G = NK < 8 ? NK : 8;
#pragma unroll
        for (int k0 = 0; k0 < NK; k0 += G) {
          u32x4 a[G];
#pragma unroll
          for (int kk = 0; kk < G; ++kk) a[kk] = row_frag(y, blk, k0 + kk);
          if constexpr (READ_AHEAD) __builtin_amdgcn_sched_barrier(0);  // (or the reads sink back to their products, one wait each)
#pragma unroll
          for (int kk = 0; kk < G; ++kk) acc = any_mfma<F16>(a[kk], x[k0 + kk], (k0 + kk) == 0 ? zero16 : acc);
        }
      }
      return acc;
    };

    // MASKED: 0 every pair kept, 1 the causal / semi-local predicate per pair, 2 the non-causal one.
    // The predicates are written with bitwise operators on 0 / 1 values: the short-circuit forms of
    // hstu_common.h compile to a divergent branch per pair here.
    // P and dS of a tile, packed as the B operands of the accumulating products (bf16, fp16; fp32 feeds
    // its accumulating products from the score registers inside tile_body)
    struct Packed {
      unsigned pw[2][8], dsw[HAS_DP ? 2 : 1][8];
    };
    // accumulating products of a tile (bf16, fp16): step s2 covers streamed rows 16 s2 .. + 15 = registers
    // 8 (s2 & 1) .. + 7 of block s2 >> 1
    auto accumulate = [&](int buf, const Packed& pk) __attribute__((always_inline)) {
      const unsigned char* y1 = &Y1s[buf][0];
      const unsigned char* y2 = &Y2s[buf][0];
      if constexpr (READ_AHEAD) {
        // the transposed fragments of step s2 + 1 are read before the products of step s2 are issued (the
        // scheduling barriers keep that order: left alone the compiler reads each fragment right before its
        // product and waits for it)
        u32x4 f2[2][HAS_P ? NB : 1], f1[2][HAS_DP ? NB : 1];
        auto read_step = [&](int s2) __attribute__((always_inline)) {
#pragma unroll
          for (int db = 0; db < NB; ++db) {
            if constexpr (HAS_P) f2[s2 & 1][db] = tr_frag(y2, db, s2);
            if constexpr (HAS_DP) f1[s2 & 1][db] = tr_frag(y1, db, s2);
          }
        };
        read_step(0);
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
          if (s2 + 1 < 4) read_step(s2 + 1);
          __builtin_amdgcn_sched_barrier(0);
          const int blk = s2 >> 1, w0 = 4 * (s2 & 1);
          const u32x4 pb = {pk.pw[blk][w0], pk.pw[blk][w0 + 1], pk.pw[blk][w0 + 2], pk.pw[blk][w0 + 3]};
          u32x4 db_ = zero4;
          if constexpr (HAS_DP) db_ = (u32x4){pk.dsw[blk][w0], pk.dsw[blk][w0 + 1], pk.dsw[blk][w0 + 2], pk.dsw[blk][w0 + 3]};
#pragma unroll
          for (int db = 0; db < NB; ++db) {
            if constexpr (HAS_P) acc2[db] = any_mfma<F16>(f2[s2 & 1][db], pb, acc2[db]);
            if constexpr (HAS_DP) acc1[db] = any_mfma<F16>(f1[s2 & 1][db], db_, acc1[db]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      } else if constexpr (RING > 0) {
        // the products of the tile in one sequence, each fragment requested RING products ahead of its own
        constexpr int K = (HAS_P ? 1 : 0) + (HAS_DP ? 1 : 0);  // products per (step, column block)
        constexpr int NPROD = 4 * NB * K;
        auto frag = [&](int i) __attribute__((always_inline)) {
          const int s2 = i / (NB * K), db = (i / K) % NB;
          const bool second = HAS_P && HAS_DP && (i % K) == 1;  // with both: the P-side product, then the dS-side one
          return tr_frag((HAS_P && !second) ? y2 : y1, db, s2);
        };
        u32x4 F[NPROD];
#pragma unroll
        for (int i = 0; i < RING; ++i) F[i] = frag(i);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NPROD; ++i) {
          if (i + RING < NPROD) F[i + RING] = frag(i + RING);
          const int s2 = i / (NB * K), db = (i / K) % NB, blk = s2 >> 1, w0 = 4 * (s2 & 1);
          const bool second = HAS_P && HAS_DP && (i % K) == 1;
          if (HAS_P && !second) {
            const u32x4 pb = {pk.pw[blk][w0], pk.pw[blk][w0 + 1], pk.pw[blk][w0 + 2], pk.pw[blk][w0 + 3]};
            acc2[db] = any_mfma<F16>(F[i], pb, acc2[db]);
          } else {
            const u32x4 db_ = {pk.dsw[blk][w0], pk.dsw[blk][w0 + 1], pk.dsw[blk][w0 + 2], pk.dsw[blk][w0 + 3]};
            acc1[db] = any_mfma<F16>(F[i], db_, acc1[db]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
          const int blk = s2 >> 1, w0 = 4 * (s2 & 1);
          const u32x4 pb = {pk.pw[blk][w0], pk.pw[blk][w0 + 1], pk.pw[blk][w0 + 2], pk.pw[blk][w0 + 3]};
          u32x4 db_ = zero4;
          if constexpr (HAS_DP) db_ = (u32x4){pk.dsw[blk][w0], pk.dsw[blk][w0 + 1], pk.dsw[blk][w0 + 2], pk.dsw[blk][w0 + 3]};
#pragma unroll
          for (int db = 0; db < NB; ++db) {
            if constexpr (HAS_P) acc2[db] = any_mfma<F16>(tr_frag(y2, db, s2), pb, acc2[db]);
            if constexpr (HAS_DP) acc1[db] = any_mfma<F16>(tr_frag(y1, db, s2), db_, acc1[db]);
          }
        }
      }
    };
    // Streamed rows [ra, rb) against this wave's stationary rows: 0 no pair kept, 1 every pair kept (causal or
    // semi-local history inside every row's window: no predicate needed), 2 the predicate per pair.  Asked
    // once per tile and wave, and again per 32-row block inside the tiles that need the predicate.
    auto classify = [&](int ra, int rb) __attribute__((always_inline)) {
      if (ra >= si.n) return 0;
      // (m_lo, m_hi) and (j_lo, j_hi): query rows and keys, inclusive
      const int m_lo = KEYS ? ra : c_lo, m_hi = KEYS ? min(rb, si.n) - 1 : c_hi;
      const int j_lo = KEYS ? c_lo : ra, j_hi = KEYS ? c_hi : min(rb, si.n) - 1;
      const int id_lo = min(m_lo, si.cap), id_hi = min(m_hi, si.cap);
      const bool diagonal = m_lo <= j_hi && j_lo <= m_hi;
      bool full = false;
      if (!noncausal) {
        const bool history = j_lo < id_hi && (id_hi >= si.tail0 || id_lo - j_hi <= si.win);
        if (!(diagonal || history || j_lo < si.ctx_eff)) return 0;
        // every pair kept: history keys below every row, and under a window inside it for every row
        full = j_hi < m_lo && j_hi < si.cap && rb <= si.n && (!semi || id_lo >= si.tail0 || id_hi - j_lo <= si.win);
      } else {
        const int idj_lo = min(j_lo, si.cap), idj_hi = min(j_hi, si.cap);
        bool window = false, tail = false;
        if (si.win != WIN_ALL) {
          window = idj_lo - id_hi <= si.win && id_lo - idj_hi <= si.win;  // the two id ranges come within the window
          if (si.tail0 != 0x7fffffff) tail = id_hi >= si.tail0 && (idj_lo < si.tail0 ? 0 : idj_lo) < id_hi;
        }
        if (!(diagonal || window || tail || j_lo < si.ctx_eff)) return 0;
        // every pair kept: the two id ranges lie within the window of each other all along
        full = si.win != WIN_ALL && id_hi - idj_lo <= si.win && idj_hi - id_lo <= si.win && rb <= si.n;
      }
      return full ? 1 : 2;
    };
    auto tile_body = [&](auto masked_tag, int r0, int buf, Packed& pk) __attribute__((always_inline)) {
      constexpr int MASKED = decltype(masked_tag)::value;
      const unsigned char* y1 = &Y1s[buf][0];
      const unsigned char* y2 = &Y2s[buf][0];
      // first streamed row of this lane half; opaque, so that the rows of the 32 registers are derived
      // from it inside the tile instead of being kept in 32 registers across the loop
      int rbase = r0 + 4 * half;
      if (MASKED) asm volatile("" : "+v"(rbase));
      // one 32-row block of scores at a time (both at once cost the masked bodies their registers)
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        // a tile that needs the predicate: its two blocks on their own (along the diagonal one of them keeps
        // no pair, or every pair)
        int block_class = 1;
        if constexpr (MASKED != 0) {
          block_class = classify(r0 + 32 * blk, r0 + 32 * blk + 32);
          if (block_class == 0) {
            if constexpr (!F32) {
#pragma unroll
              for (int i = 0; i < 8; ++i) {
                pk.pw[blk][i] = 0u;
                if constexpr (HAS_DP) pk.dsw[blk][i] = 0u;
              }
            }
            continue;
          }
        }
        f32x16 Sb = row_product(y1, blk, x1), dPb;
        if constexpr (HAS_DP) dPb = row_product(y2, blk, x2);
        float pv[16], dsv[HAS_DP ? 16 : 1];
        // (the per-token scale of the key-stationary modes, and the bias table's gradient of the dQ mode, as
        // a compile-time tag of the loop: tested per score they put a branch behind every score, and nothing
        // was scheduled across them)
        auto score_loop = [&](auto tag, auto predicate_tag) __attribute__((always_inline)) {
          constexpr bool ROW_SCALES = KEYS && decltype(tag)::value;
          constexpr bool WITH_DRAB = MODE == ANY_DQ && decltype(tag)::value;
          // 0: every pair kept; 1: the causal / semi-local predicate; 2: the non-causal mask without a window
          // (diagonal and contextual keys); 3: the non-causal mask with a window
          constexpr int PRED = decltype(predicate_tag)::value;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int rl = 32 * blk + 8 * (r >> 2) + 4 * half + (r & 3);  // streamed row of this register
            float x = FOLD_ALPHA ? Sb[r] : Sb[r] * p.alpha;
            if constexpr (HAS_RAB) x += bias_s[buf][KEYS ? rl - (c - c0) + (ANY_BM - 1) : (c - c0) - rl + (ANY_BN - 1)];
            const float sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * (FOLD_ALPHA ? neg_alpha_log2e : neg_log2e)));
            float pe = x * sig;
            float de = 0.f;
            if constexpr (HAS_DP) de = dPb[r] * (sig + pe * (1.0f - sig));  // silu'(x) = sig (1 + x (1 - sig))
            if constexpr (ROW_SCALES) {
              const float rs = scale_s[buf][rl];
              pe *= rs;
              de *= rs;
            }
            if constexpr (PRED != 0) {
              const int rr = rbase + (32 * blk + 8 * (r >> 2) + (r & 3));
              const int m = KEYS ? rr : c, j = KEYS ? c : rr;
              const int idm = min(m, si.cap);
              int kp = (int)(m == j) | (int)(j < si.ctx_eff);
              if (PRED == 1) {
                kp |= (int)(j < idm) & ((int)(idm - j <= si.win) | (int)(idm >= si.tail0));
              } else if (PRED == 3) {
                // (without a full-attention tail tail0 is INT_MAX: both ids below count as 0 and the last term is never true)
                const int idj = min(j, si.cap);
                const int gr = idm < si.tail0 ? 0 : idm, gc = idj < si.tail0 ? 0 : idj;
                kp |= (int)(abs(idm - idj) <= si.win) | (int)(gr - gc > 0);
              }
              kp &= (int)(rr < si.n) & (int)(c < si.n);
              pe = kp ? pe : 0.f;
              de = kp ? de : 0.f;
            }
            pv[r] = pe;
            if constexpr (HAS_DP) dsv[r] = de;
            if constexpr (WITH_DRAB) {
              // d score / d bias = 1: the pair's dS (with its row's scale) goes to its diagonal
              const int iv = __float2int_rn(de * dscale);
              if (iv != 0) __hip_atomic_fetch_add(&dband_s[buf][(c - c0) - rl + (ANY_BN - 1)], iv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            // the masked bodies four pairs at a time: left to itself the scheduler interleaves all 32 and spills
            if (PRED != 0 && (r & 3) == 3) __builtin_amdgcn_sched_barrier(0);
          }
        };
        constexpr bool TAGGED = KEYS || (MODE == ANY_DQ && HAS_RAB);
        auto scores = [&](auto predicate_tag) __attribute__((always_inline)) {
          if (TAGGED && (KEYS ? per_token : drabg != nullptr)) score_loop(std::true_type{}, predicate_tag);
          else score_loop(std::false_type{}, predicate_tag);
        };
        if (MASKED == 0 || block_class == 1) scores(std::integral_constant<int, 0>{});
        else if (MASKED == 2 && si.win != WIN_ALL) scores(std::integral_constant<int, 3>{});
        else scores(std::integral_constant<int, MASKED>{});
        if constexpr (F32) {
          // accumulating products of this block, one streamed row per lane half and step: register r of
          // the score block is the B operand as it is; the A operand is column 32 db + l32 of that row
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = 32 * blk + 8 * (r >> 2) + 4 * half + (r & 3);
#pragma unroll
            for (int db = 0; db < NB; ++db) {
              if constexpr (HAS_P)
                acc2[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(*(const float*)(y2 + row * RS + (32 * db + l32) * 4), pv[r], acc2[db], 0, 0, 0);
              if constexpr (HAS_DP)
                acc1[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(*(const float*)(y1 + row * RS + (32 * db + l32) * 4), dsv[r], acc1[db], 0, 0, 0);
            }
          }
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            pk.pw[blk][i] = any_pack2<F16>(pv[2 * i], pv[2 * i + 1]);
            if constexpr (HAS_DP) pk.dsw[blk][i] = any_pack2<F16>(dsv[2 * i], dsv[2 * i + 1]);
          }
        }
      }
      if constexpr (!F32 && !ACC_APART) accumulate(buf, pk);
    };
    auto compute_tile = [&](int t, int buf) __attribute__((always_inline)) {
      if (!wave_has_rows) return;
      const int r0 = t * ANY_BN;
      const int cls = classify(r0, r0 + ANY_BN);
      if (cls == 0) return;
      const bool full = cls == 1;
      Packed pk;
      if (full) tile_body(std::integral_constant<int, 0>{}, r0, buf, pk);
      else if (!noncausal) tile_body(std::integral_constant<int, 1>{}, r0, buf, pk);
      else tile_body(std::integral_constant<int, 2>{}, r0, buf, pk);
      if constexpr (!F32 && ACC_APART) accumulate(buf, pk);
    };

    // band of tile `tile` (LDS stage b) -> the head's row of the table, and the stage cleared for the
    // tile after the next; float additions in whatever order the workgroups arrive
    auto flush_band = [&](int tile, int b) __attribute__((always_inline)) {
      if constexpr (MODE == ANY_DQ) {
        if (drabg && tid < ANY_BM + ANY_BN - 1) {
          const int v = dband_s[b][tid];
          dband_s[b][tid] = 0;
          const int idx = c0 - tile * ANY_BN - (ANY_BN - 1) + tid + p.N - 1;  // entry e is the diagonal m - j = dmin + e
          if (v != 0 && idx >= 0 && idx < rab_w) atomicAdd((unsigned long long*)&drabg[idx], (unsigned long long)(long long)v);
        }
      }
    };
    if constexpr (MODE == ANY_DQ) {
      if (drabg && tid < ANY_BM + ANY_BN) dband_s[0][tid] = dband_s[1][tid] = 0;  // (published by the first tile's barrier)
    }

    Staged st;
    int t = (has_skip && t_begin >= skip_a) ? max(t_begin, skip_b) : t_begin;
    int buf = 0;
    if (t < t_end) {
      load_tiles(t, st);
      store_tiles(0, st);
      __syncthreads();
      int nxt = next_tile(t);
      if (nxt < t_end) load_tiles(nxt, st);
      while (true) {
        compute_tile(t, buf);
        if (nxt >= t_end) break;
        store_tiles(buf ^ 1, st);
        __syncthreads();
        flush_band(t, buf);  // every wave is through tile t
        t = nxt;
        buf ^= 1;
        nxt = next_tile(t);
        if (nxt < t_end) load_tiles(nxt, st);
      }
      if constexpr (MODE == ANY_DQ) {
        if (drabg) {
          __syncthreads();
          flush_band(t, buf);
        }
      }
    }

    // ---- epilogue: transposed accumulators -> rows of the outputs ----
    if (c_valid) {
      auto store_rows = [&](void* base, int D, const f32x16* acc, float f) __attribute__((always_inline)) {
        char* orow = (char*)base + ((size_t)(si.s + c) * p.H + h) * D * ES;
#pragma unroll
        for (int db = 0; db < NB; ++db) {
#pragma unroll
          for (int rq = 0; rq < 4; ++rq) {
            const int d0 = db * 32 + 8 * rq + 4 * half;
            if constexpr (!ALIGNED) {
              // four elements at once where the row holds them, the row's last few one by one
              if (d0 + 4 <= D) {
                if constexpr (F32) {
                  const u32x4 o = {__float_as_uint(acc[db][4 * rq + 0] * f), __float_as_uint(acc[db][4 * rq + 1] * f),
                                   __float_as_uint(acc[db][4 * rq + 2] * f), __float_as_uint(acc[db][4 * rq + 3] * f)};
                  *(any_u32x4_a4*)(orow + d0 * 4) = o;
                } else {
                  u32x2 o;
                  o.x = any_pack2<F16>(acc[db][4 * rq + 0] * f, acc[db][4 * rq + 1] * f);
                  o.y = any_pack2<F16>(acc[db][4 * rq + 2] * f, acc[db][4 * rq + 3] * f);
                  *(any_u32x2_a2*)(orow + d0 * 2) = o;
                }
              } else {
#pragma unroll
                for (int e = 0; e < 3; ++e) {
                  if (d0 + e < D) {
                    if constexpr (F32) *(float*)(orow + (d0 + e) * 4) = acc[db][4 * rq + e] * f;
                    else *(unsigned short*)(orow + (d0 + e) * 2) = (unsigned short)any_pack2<F16>(acc[db][4 * rq + e] * f, 0.f);
                  }
                }
              }
            } else if (d0 < D) {
              if constexpr (F32) {
                const u32x4 o = {__float_as_uint(acc[db][4 * rq + 0] * f), __float_as_uint(acc[db][4 * rq + 1] * f),
                                 __float_as_uint(acc[db][4 * rq + 2] * f), __float_as_uint(acc[db][4 * rq + 3] * f)};
                *(u32x4*)(orow + d0 * 4) = o;
              } else {
                u32x2 o;
                o.x = any_pack2<F16>(acc[db][4 * rq + 0] * f, acc[db][4 * rq + 1] * f);
                o.y = any_pack2<F16>(acc[db][4 * rq + 2] * f, acc[db][4 * rq + 3] * f);
                *(u32x2*)(orow + d0 * 2) = o;
              }
            }
          }
        }
      };
      if constexpr (MODE == ANY_FWD) store_rows(p.out, p.Dv, acc2, FOLD_ALPHA ? col_scale * p.alpha : col_scale);
      if constexpr (MODE == ANY_DQ) store_rows(bp.dq, p.Dqk, acc1, col_scale * p.alpha);
      if constexpr (KEYS && HAS_DP) store_rows(bp.dk, p.Dqk, acc1, col_scale * p.alpha);
      if constexpr (KEYS && HAS_P) store_rows(bp.dv, p.Dv, acc2, col_scale);
    }
    __syncthreads();  // the LDS tiles are reused by the next item
  }
}

// Launchers.  dtype: RECIR_HSTU_DTYPE_BF16, _FP16 or _FP32; dp: padded head dim (32, 64, 128 or 256).
// aligned: every row of every tensor starts at a multiple of 16 bytes.  Return false when the combination
// has no instantiation.  The instantiations with and without a bias table, for aligned rows and for
// any, live in four translation units (hstu_mfma_any*.hip) that compile side by side.
bool launch_mfma_any_fwd(int dtype, int dp, bool aligned, dim3 grid, hipStream_t stream, const Params& p);
bool launch_mfma_any_bwd(int dtype, int dp, bool aligned, dim3 grid_q, dim3 grid_k, hipStream_t stream, const BwdParams& bq, const BwdParams& bk);
template <bool HAS_RAB, bool ALIGNED>
bool launch_mfma_any_fwd_as(int dtype, int dp, dim3 grid, hipStream_t stream, const BwdParams& bp);
template <bool HAS_RAB, bool ALIGNED>
bool launch_mfma_any_bwd_as(int dtype, int dp, dim3 grid_q, dim3 grid_k, hipStream_t stream, const BwdParams& bq, const BwdParams& bk);

}  // namespace recir_hstu
