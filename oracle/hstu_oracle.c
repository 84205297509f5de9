/*
 * CPU oracle for the HSTU jagged attention forward and backward.  TEST INFRASTRUCTURE ONLY.
 *
 * This file is a plain-C restatement of the reference algorithm.  It exists so
 * that tests, the smoke check and the benchmark's CPU-baseline leg have an
 * independent answer to compare the HIP kernels with.  The product library
 * never links, loads or calls it.
 *
 * Reference lines each function follows (paths relative to the upstream tree):
 *   hstu_oracle_keep            recir/ops/helion/jagged_hstu_attention.py:185-208, :346
 *   hstu_oracle_keep_clamp_id   recir/ops/kjt_split_per_feature.cpp:639-674,
 *                               recir/ops/pallas/hstu_attention.py:86-112, :404-430
 *   hstu_oracle_keep_sl, hstu_oracle_keep_sl_clamp_id
 *                               the semi-local mask (max_attn_len, full_attn_size) of
 *                               recir/ops/kjt_split_per_feature.cpp:654-668 and
 *                               recir/ops/helion/jagged_hstu_attention.py:124-147
 *   hstu_oracle_keep_nc, hstu_oracle_keep_nc_clamp_id
 *                               the mask of any invalid_attn_mask_type other than "lower_triangular"
 *                               (recir/ops/kjt_split_per_feature.cpp:650-671: absolute distance of the
 *                               clamped ids; without max_attn_len only the diagonal is kept)
 *   hstu_oracle_attn_fwd        recir/ops/kjt_split_per_feature.cpp:602-693 (per-sequence loop,
 *                               alpha on the scores, x*sigmoid(x), attn_scale or 1/max_seq_len,
 *                               mask multiply, weights @ v) with the packed [T,H,Dv] output and
 *                               zeroed tail of recir/ops/pallas/jagged_hstu_attention.py:323-344
 *   hstu_oracle_attn_bwd        the gradient formulas of recir/ops/helion/jagged_hstu_attention.py:16-27
 *                               (dP = dO V^T, dV = P^T dO, dS = dP keep scale silu'(S),
 *                               dQ = alpha dS K, dK = alpha dS^T Q, silu'(x) = sig(x)(1 + x(1 - sig(x))))
 *                               with the zeroed tail rows of :916-920
 *   hstu_oracle_e4m3_encode     recir/ops/kjt_split_per_feature.cpp:493-502 (clamp to +-448 then
 *                               round-to-nearest-even cast to float8_e4m3fn)
 *
 * Parity pins (see tests/): the reference's compiled C++ op on seeded inputs
 * (golden fixtures), the reference's own zero-query known-answer test, two
 * independent closed forms of the mask compared exhaustively, closed-form
 * special cases (single token, all-target, constant score => kept-key count),
 * and torch's own float8_e4m3fn cast for the encoder.
 * The gradient of the bias table (hstu_oracle_attn_bwd_rab) has no counterpart in the reference
 * either; it is pinned by torch autograd through the dense float64 restatement in
 * tests/test_oracle_bwd.py and by finite differences of the forward oracle.
 * The backward is pinned the way the reference pins its own kernels
 * (recir/ops/helion/jagged_hstu_attention.py:260-280, autograd through the forward): against
 * torch autograd through the reference's compiled C++ forward op, against torch autograd through
 * a dense torch restatement, and against central finite differences of the forward oracle.
 * Parity unpinned by the reference: the relative attention bias term (the
 * reference has no such argument) and contextual_seq_len > 1 in "prefix" mode
 * (the reference C++ only ever unmasks key 0).  Both are pinned only by the
 * dense closed form in tests/test_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define HSTU_CTX_PREFIX 0  /* keys j < ctx visible to every query               */
#define HSTU_CTX_REFCPP 1  /* reference C++: keys whose clamped id is 0 visible  */
#define HSTU_MASK_NONCAUSAL 2 /* added to the ctx mode: the mask of a mask type other than "lower_triangular" */

/* keep(m, j) in the "causal and key-is-history, or diagonal" form. */
int hstu_oracle_keep(int64_t m, int64_t j, int64_t n, int64_t t, int64_t ctx, int ctx_mode) {
  if (m < 0 || j < 0 || m >= n || j >= n) return 0;
  const int64_t cap = n - t;
  int keep = (m == j) || (m >= j && j < cap);
  if (ctx > 0) {
    if (ctx_mode == HSTU_CTX_PREFIX) {
      keep = keep || (j < ctx);
    } else {
      /* the reference compares the *clamped* key id with zero */
      const int64_t idj = j < cap ? j : cap;
      keep = keep || (idj == 0);
    }
  }
  return keep;
}

/* Same predicate written the way the C++ fallback and the dense JAX reference
 * build it: ids clamped to the history length, distance > 0 or identity. */
int hstu_oracle_keep_clamp_id(int64_t m, int64_t j, int64_t n, int64_t t, int64_t ctx,
                              int ctx_mode) {
  if (m < 0 || j < 0 || m >= n || j >= n) return 0;
  const int64_t bound = n - t;
  const int64_t idm = m < bound ? m : bound;
  const int64_t idj = j < bound ? j : bound;
  int keep = (m == j) || (idm - idj > 0);
  if (ctx > 0) {
    if (ctx_mode == HSTU_CTX_PREFIX) keep = keep || (j < ctx);
    else keep = keep || (idj == 0);
  }
  return keep;
}

/*
 * Mask of a mask type other than "lower_triangular", as the reference builds it
 * (kjt_split_per_feature.cpp:639-674): clamped ids, their absolute distance, a window only when
 * max_attn_len > 0 (without one nothing but the diagonal is kept), the "global" rows of
 * full_attn_size unchanged from the causal case, and the contextual switch.
 */
int hstu_oracle_keep_nc_clamp_id(int64_t m, int64_t j, int64_t n, int64_t t, int64_t ctx,
                                 int ctx_mode, int64_t A, int64_t F) {
  if (m < 0 || j < 0 || m >= n || j >= n) return 0;
  const int64_t bound = n - t;
  const int64_t idm = m < bound ? m : bound;
  const int64_t idj = j < bound ? j : bound;
  int64_t distance = idm - idj;
  if (distance < 0) distance = -distance;
  int keep = (m == j);
  if (A > 0) {
    keep = keep || (distance >= -A && distance <= A);
    if (F > 0) {
      const int64_t boundary = bound - F;
      const int64_t gr = idm < boundary ? 0 : idm;
      const int64_t gc = idj < boundary ? 0 : idj;
      keep = keep || (gr - gc > 0);
    }
  }
  if (ctx > 0) {
    if (ctx_mode & HSTU_CTX_REFCPP) keep = keep || (idj == 0);
    else keep = keep || (j < ctx);
  }
  return keep;
}

/* The same mask said in words: with a window, a pair is kept when the two positions (targets all
 * standing at the first target's position) are at most A apart, either way round, or when the query
 * stands in the last F history positions or beyond and the key stands strictly before it; the
 * diagonal and the contextual keys always. */
int hstu_oracle_keep_nc(int64_t m, int64_t j, int64_t n, int64_t t, int64_t ctx, int ctx_mode,
                        int64_t A, int64_t F) {
  if (m < 0 || j < 0 || m >= n || j >= n) return 0;
  const int64_t cap = n - t;
  const int64_t pm = m < cap ? m : cap, pj = j < cap ? j : cap;
  int keep = (m == j);
  if (A > 0) {
    const int near = (pm >= pj ? pm - pj : pj - pm) <= A;
    /* below the boundary a key counts as position 0: before every tail row but row 0 itself */
    const int tail = F > 0 && pm >= cap - F && (pj < cap - F ? pm > 0 : pj < pm);
    keep = keep || near || tail;
  }
  if (ctx > 0) {
    if (ctx_mode & HSTU_CTX_REFCPP) keep = keep || (pj == 0);
    else keep = keep || (j < ctx);
  }
  return keep;
}

/*
 * Semi-local variant (max_attn_len A > 0): a history key is visible to a query when it lies within
 * the last A positions before the query's target-clamped id, or -- with full_attn_size F > 0 --
 * when the query's clamped id is in the last F history positions or beyond (those rows keep full
 * causal attention).  A == 0 is the plain causal mask (F is then ignored, as in the reference).
 * Written as "history key, and near or full-tail row".
 */
int hstu_oracle_keep_sl(int64_t m, int64_t j, int64_t n, int64_t t, int64_t ctx, int ctx_mode,
                        int64_t A, int64_t F) {
  if (ctx_mode & HSTU_MASK_NONCAUSAL) return hstu_oracle_keep_nc(m, j, n, t, ctx, ctx_mode, A, F);
  if (A <= 0) return hstu_oracle_keep(m, j, n, t, ctx, ctx_mode);
  if (m < 0 || j < 0 || m >= n || j >= n) return 0;
  const int64_t cap = n - t;
  const int64_t idm = m < cap ? m : cap;
  const int hist = j < idm; /* implies j < cap */
  const int near = idm - j <= A;
  const int tail = F > 0 && idm >= cap - F;
  int keep = (m == j) || (hist && (near || tail));
  if (ctx > 0) {
    if (ctx_mode == HSTU_CTX_PREFIX) {
      keep = keep || (j < ctx);
    } else {
      const int64_t idj = j < cap ? j : cap;
      keep = keep || (idj == 0);
    }
  }
  return keep;
}

/* The same mask built the way the reference C++ builds it (kjt_split_per_feature.cpp:639-674):
 * clamped ids, distance window, and the "global" rows/columns zeroed below the boundary. */
int hstu_oracle_keep_sl_clamp_id(int64_t m, int64_t j, int64_t n, int64_t t, int64_t ctx,
                                 int ctx_mode, int64_t A, int64_t F) {
  if (ctx_mode & HSTU_MASK_NONCAUSAL) return hstu_oracle_keep_nc_clamp_id(m, j, n, t, ctx, ctx_mode, A, F);
  if (m < 0 || j < 0 || m >= n || j >= n) return 0;
  const int64_t bound = n - t;
  const int64_t idm = m < bound ? m : bound;
  const int64_t idj = j < bound ? j : bound;
  const int64_t distance = idm - idj;
  int keep = (m == j);
  if (A > 0) {
    keep = keep || (distance > 0 && distance <= A);
    if (F > 0) {
      const int64_t boundary = bound - F;
      const int64_t gr = idm < boundary ? 0 : idm;
      const int64_t gc = idj < boundary ? 0 : idj;
      keep = keep || (gr - gc > 0);
    }
  } else {
    keep = keep || (distance > 0);
  }
  if (ctx > 0) {
    if (ctx_mode == HSTU_CTX_PREFIX) keep = keep || (j < ctx);
    else keep = keep || (idj == 0);
  }
  return keep;
}

int64_t hstu_oracle_count_pairs_sl(int64_t n, int64_t t, int64_t ctx, int ctx_mode, int64_t A,
                                   int64_t F) {
  int64_t c = 0;
  for (int64_t m = 0; m < n; ++m)
    for (int64_t j = 0; j < n; ++j) c += hstu_oracle_keep_sl(m, j, n, t, ctx, ctx_mode, A, F);
  return c;
}

/* Number of kept (m, j) pairs of one sequence, by brute force. */
int64_t hstu_oracle_count_pairs(int64_t n, int64_t t, int64_t ctx, int ctx_mode) {
  int64_t c = 0;
  for (int64_t m = 0; m < n; ++m)
    for (int64_t j = 0; j < n; ++j) c += hstu_oracle_keep(m, j, n, t, ctx, ctx_mode);
  return c;
}

static float round_to_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return x; /* NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  memcpy(&x, &u, 4);
  return x;
}

/*
 * attn_scale_kind: 0 -> 1/max_seq_len, 1 -> attn_scale[0], 2 -> attn_scale[token of the query row].
 * p_round: 0 keeps P in double; 1 rounds P (after the scale) to bf16 like a bf16 value tensor would
 *          force in the reference (weights.to(v.dtype)).
 * Returns 0, or -1 on a malformed offsets array (same condition the reference rejects).
 */
int hstu_oracle_attn_fwd_sl(const float* q, const float* k, const float* v, float* out,
                            const int64_t* seq_offsets, const int64_t* num_targets, const float* rab,
                            int attn_scale_kind, const float* attn_scale, int64_t T, int64_t B,
                            int64_t H, int64_t Dqk, int64_t Dv, int64_t max_seq_len, int64_t ctx,
                            int ctx_mode, double alpha, int p_round, int64_t max_attn_len,
                            int64_t full_attn_size) {
  for (int64_t b = 0; b < B; ++b) {
    const int64_t s = seq_offsets[b], e = seq_offsets[b + 1];
    if (!(0 <= s && s <= e && e <= T)) return -1;
  }
  memset(out, 0, sizeof(float) * (size_t)(T * H * Dv));
  const int64_t rab_w = 2 * max_seq_len - 1;

#pragma omp parallel
  {
    double* acc = (double*)malloc(sizeof(double) * (size_t)(Dv > 0 ? Dv : 1));
    for (int64_t b = 0; b < B; ++b) {
      const int64_t s = seq_offsets[b], e = seq_offsets[b + 1], n = e - s;
      const int64_t t = num_targets ? num_targets[b] : 0;
#pragma omp for collapse(2) schedule(dynamic, 8) nowait
      for (int64_t m = 0; m < n; ++m) {
        for (int64_t h = 0; h < H; ++h) {
          const float* qr = q + ((s + m) * H + h) * Dqk;
          for (int64_t d = 0; d < Dv; ++d) acc[d] = 0.0;
          double scale;
          if (attn_scale_kind == 0) scale = 1.0 / (double)max_seq_len;
          else if (attn_scale_kind == 1) scale = (double)attn_scale[0];
          else scale = (double)attn_scale[s + m];
          for (int64_t j = 0; j < n; ++j) {
            if (!hstu_oracle_keep_sl(m, j, n, t, ctx, ctx_mode, max_attn_len, full_attn_size)) continue;
            const float* kr = k + ((s + j) * H + h) * Dqk;
            double dot = 0.0;
#pragma omp simd reduction(+ : dot)
            for (int64_t d = 0; d < Dqk; ++d) dot += (double)qr[d] * (double)kr[d];
            double x = dot * alpha;
            if (rab) {
              const int64_t idx = m - j + max_seq_len - 1;
              if (idx >= 0 && idx < rab_w) x += (double)rab[h * rab_w + idx];
            }
            double p = x / (1.0 + exp(-x)) * scale;
            if (p_round) p = (double)round_to_bf16((float)p);
            const float* vr = v + ((s + j) * H + h) * Dv;
#pragma omp simd
            for (int64_t d = 0; d < Dv; ++d) acc[d] += p * (double)vr[d];
          }
          float* orow = out + ((s + m) * H + h) * Dv;
          for (int64_t d = 0; d < Dv; ++d) orow[d] = (float)acc[d];
        }
      }
    }
    free(acc);
  }
  return 0;
}

/*
 * Gradients of hstu_oracle_attn_fwd with respect to q, k and v for an upstream gradient dout
 * [T,H,Dv].  attn_scale_kind as in the forward.  Accumulation in double; dq, dk, dv are written in
 * full (rows at and after seq_offsets[B] are zero).  The score bias rab enters S but no gradient is
 * produced for it.
 * p_round: 1 rounds P and dS to bf16 before they are used as matmul operands (what a bf16 kernel
 *          does); 0 keeps them in double.
 */
/* drab (may be NULL): gradient of the bias table, [H, 2 * max_seq_len - 1] doubles, the sum of
 * dS(m, j) over all kept pairs of all sequences with m - j + max_seq_len - 1 equal to the column
 * (the score is alpha q.k + rab, so d score / d rab = 1).  No counterpart in the reference. */
int hstu_oracle_attn_bwd_rab(const float* dout, const float* q, const float* k, const float* v, float* dq,
                             float* dk, float* dv, double* drab, const int64_t* seq_offsets,
                             const int64_t* num_targets, const float* rab, int attn_scale_kind,
                             const float* attn_scale, int64_t T, int64_t B, int64_t H, int64_t Dqk,
                             int64_t Dv, int64_t max_seq_len, int64_t ctx, int ctx_mode, double alpha,
                             int p_round, int64_t max_attn_len, int64_t full_attn_size) {
  for (int64_t b = 0; b < B; ++b) {
    const int64_t s = seq_offsets[b], e = seq_offsets[b + 1];
    if (!(0 <= s && s <= e && e <= T)) return -1;
  }
  memset(dq, 0, sizeof(float) * (size_t)(T * H * Dqk));
  memset(dk, 0, sizeof(float) * (size_t)(T * H * Dqk));
  memset(dv, 0, sizeof(float) * (size_t)(T * H * Dv));
  const int64_t rab_w = 2 * max_seq_len - 1;
  if (drab) memset(drab, 0, sizeof(double) * (size_t)(H * rab_w));

  /* one (sequence, head) per task: every output row is owned by exactly one task */
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t h = 0; h < H; ++h) {
      const int64_t s = seq_offsets[b], e = seq_offsets[b + 1], n = e - s;
      const int64_t t = num_targets ? num_targets[b] : 0;
      if (n <= 0) continue;
      double* adrab = drab ? (double*)calloc((size_t)rab_w, sizeof(double)) : NULL;
      double* adq = (double*)calloc((size_t)(n * Dqk), sizeof(double));
      double* adk = (double*)calloc((size_t)(n * Dqk), sizeof(double));
      double* adv = (double*)calloc((size_t)(n * Dv), sizeof(double));
      for (int64_t m = 0; m < n; ++m) {
        const float* qr = q + ((s + m) * H + h) * Dqk;
        const float* gr = dout + ((s + m) * H + h) * Dv;
        double scale;
        if (attn_scale_kind == 0) scale = 1.0 / (double)max_seq_len;
        else if (attn_scale_kind == 1) scale = (double)attn_scale[0];
        else scale = (double)attn_scale[s + m];
        for (int64_t j = 0; j < n; ++j) {
          if (!hstu_oracle_keep_sl(m, j, n, t, ctx, ctx_mode, max_attn_len, full_attn_size)) continue;
          const float* kr = k + ((s + j) * H + h) * Dqk;
          const float* vr = v + ((s + j) * H + h) * Dv;
          double dot = 0.0;
          for (int64_t d = 0; d < Dqk; ++d) dot += (double)qr[d] * (double)kr[d];
          double x = dot * alpha;
          if (rab) {
            const int64_t idx = m - j + max_seq_len - 1;
            if (idx >= 0 && idx < rab_w) x += (double)rab[h * rab_w + idx];
          }
          const double sig = 1.0 / (1.0 + exp(-x));
          double p = x * sig * scale;
          double dp = 0.0;
          for (int64_t d = 0; d < Dv; ++d) dp += (double)gr[d] * (double)vr[d];
          double ds = dp * scale * sig * (1.0 + x * (1.0 - sig));
          if (p_round) {
            p = (double)round_to_bf16((float)p);
            ds = (double)round_to_bf16((float)ds);
          }
          if (adrab) {
            const int64_t idx = m - j + max_seq_len - 1;
            if (idx >= 0 && idx < rab_w) adrab[idx] += ds;
          }
          for (int64_t d = 0; d < Dv; ++d) adv[j * Dv + d] += p * (double)gr[d];
          for (int64_t d = 0; d < Dqk; ++d) {
            adq[m * Dqk + d] += ds * (double)kr[d];
            adk[j * Dqk + d] += ds * (double)qr[d];
          }
        }
      }
      for (int64_t m = 0; m < n; ++m) {
        for (int64_t d = 0; d < Dqk; ++d) {
          dq[((s + m) * H + h) * Dqk + d] = (float)(alpha * adq[m * Dqk + d]);
          dk[((s + m) * H + h) * Dqk + d] = (float)(alpha * adk[m * Dqk + d]);
        }
        for (int64_t d = 0; d < Dv; ++d) dv[((s + m) * H + h) * Dv + d] = (float)adv[m * Dv + d];
      }
      if (adrab) {
        /* sequences of one head add into the same row: one at a time */
#pragma omp critical(hstu_oracle_drab)
        for (int64_t i = 0; i < rab_w; ++i) drab[h * rab_w + i] += adrab[i];
        free(adrab);
      }
      free(adq);
      free(adk);
      free(adv);
    }
  }
  return 0;
}

int hstu_oracle_attn_bwd_sl(const float* dout, const float* q, const float* k, const float* v, float* dq,
                            float* dk, float* dv, const int64_t* seq_offsets,
                            const int64_t* num_targets, const float* rab, int attn_scale_kind,
                            const float* attn_scale, int64_t T, int64_t B, int64_t H, int64_t Dqk,
                            int64_t Dv, int64_t max_seq_len, int64_t ctx, int ctx_mode, double alpha,
                            int p_round, int64_t max_attn_len, int64_t full_attn_size) {
  return hstu_oracle_attn_bwd_rab(dout, q, k, v, dq, dk, dv, NULL, seq_offsets, num_targets, rab, attn_scale_kind,
                                  attn_scale, T, B, H, Dqk, Dv, max_seq_len, ctx, ctx_mode, alpha, p_round,
                                  max_attn_len, full_attn_size);
}

/* Causal forms (max_attn_len = full_attn_size = 0). */
int hstu_oracle_attn_fwd(const float* q, const float* k, const float* v, float* out,
                         const int64_t* seq_offsets, const int64_t* num_targets, const float* rab,
                         int attn_scale_kind, const float* attn_scale, int64_t T, int64_t B,
                         int64_t H, int64_t Dqk, int64_t Dv, int64_t max_seq_len, int64_t ctx,
                         int ctx_mode, double alpha, int p_round) {
  return hstu_oracle_attn_fwd_sl(q, k, v, out, seq_offsets, num_targets, rab, attn_scale_kind, attn_scale,
                                 T, B, H, Dqk, Dv, max_seq_len, ctx, ctx_mode, alpha, p_round, 0, 0);
}

int hstu_oracle_attn_bwd(const float* dout, const float* q, const float* k, const float* v, float* dq,
                         float* dk, float* dv, const int64_t* seq_offsets,
                         const int64_t* num_targets, const float* rab, int attn_scale_kind,
                         const float* attn_scale, int64_t T, int64_t B, int64_t H, int64_t Dqk,
                         int64_t Dv, int64_t max_seq_len, int64_t ctx, int ctx_mode, double alpha,
                         int p_round) {
  return hstu_oracle_attn_bwd_sl(dout, q, k, v, dq, dk, dv, seq_offsets, num_targets, rab, attn_scale_kind,
                                 attn_scale, T, B, H, Dqk, Dv, max_seq_len, ctx, ctx_mode, alpha, p_round,
                                 0, 0);
}

/* float -> OCP float8 e4m3fn byte: saturate to +-448 first (the reference clamps before the cast),
 * round to nearest even, keep subnormals, NaN -> 0x7f. */
uint8_t hstu_oracle_e4m3_encode(float x) {
  if (x != x) return 0x7f;
  const uint8_t sign = signbit(x) ? 0x80 : 0x00;
  double a = fabs((double)x);
  if (a > 448.0) a = 448.0;
  if (a == 0.0) return sign;
  int ex;
  double mant = frexp(a, &ex); /* a = mant * 2^ex, mant in [0.5, 1) */
  int E = ex - 1;              /* a = (2*mant) * 2^E, 2*mant in [1, 2) */
  if (E < -6) {
    /* subnormal: multiples of 2^-9 */
    double qv = nearbyint(a * 512.0); /* ties to even under the default rounding mode */
    if (qv >= 8.0) return sign | 0x08; /* rounds up to the smallest normal 2^-6 */
    return sign | (uint8_t)qv;
  }
  double frac = (2.0 * mant - 1.0) * 8.0; /* in [0, 8) */
  double qf = nearbyint(frac);
  int m3 = (int)qf;
  if (m3 == 8) { m3 = 0; E += 1; }
  int be = E + 7;
  if (be > 15 || (be == 15 && m3 > 6)) { be = 15; m3 = 6; } /* 448 = 1.75 * 2^8 */
  return sign | (uint8_t)(be << 3) | (uint8_t)m3;
}

float hstu_oracle_e4m3_decode(uint8_t b) {
  const int sgn = b >> 7, be = (b >> 3) & 0xf, m3 = b & 7;
  double val;
  if (be == 15 && m3 == 7) return NAN;
  if (be == 0) val = (double)m3 / 8.0 * ldexp(1.0, -6);
  else val = (1.0 + (double)m3 / 8.0) * ldexp(1.0, be - 7);
  return (float)(sgn ? -val : val);
}

/* Per-head symmetric quantisation of a packed [T,H,D] tensor: scale[h] = max(amax_h, 1e-12)/448,
 * codes = e4m3(clamp(x / scale[h], +-448)).  Granularity is per head (not per row as in the
 * reference helper); the arithmetic is the reference's. */
void hstu_oracle_quant_e4m3_per_head(const float* x, uint8_t* codes, float* scale, int64_t T,
                                     int64_t H, int64_t D) {
  for (int64_t h = 0; h < H; ++h) {
    float amax = 0.f;
    for (int64_t r = 0; r < T; ++r)
      for (int64_t d = 0; d < D; ++d) {
        const float a = fabsf(x[(r * H + h) * D + d]);
        if (a > amax) amax = a;
      }
    if (amax < 1e-12f) amax = 1e-12f;
    scale[h] = amax / 448.0f;
  }
  for (int64_t r = 0; r < T; ++r)
    for (int64_t h = 0; h < H; ++h)
      for (int64_t d = 0; d < D; ++d) {
        float y = x[(r * H + h) * D + d] / scale[h];
        if (y > 448.f) y = 448.f;
        if (y < -448.f) y = -448.f;
        codes[(r * H + h) * D + d] = hstu_oracle_e4m3_encode(y);
      }
}
