// Work-list construction for the tiled kernels.
//
// Goals: (1) every query tile of one (sequence, head) runs on the same XCD, so that the K and V rows
// of that pair are fetched into exactly one L2; (2) the eight per-XCD lists carry equal work;
// (3) inside a list the query tiles with the longest causal prefix come first, so that the tail of
// the launch consists of short work.
//
// Sequences are ranked by their number of query tiles (descending); pair (rank r, head h) gets the
// running index pr = r * H + h and is dealt to the XCDs in boustrophedon order
// (0..7, 7..0, 0..7, ...), which keeps the list sums within one pair's work of each other.  Inside a
// list, items are ordered by query-tile index descending, ties in dealing order.
//
// With PLAN_REVERSE the item at the position of tile index t carries tile nt - 1 - t instead: the
// backward's key-tile kernel, whose work grows towards the start of a sequence, gets the same
// heaviest-first order.
#pragma once
#include "hstu_common.h"

namespace recir_hstu {

#ifndef HSTU_PLAN_THREADS
#define HSTU_PLAN_THREADS 1024
#endif
constexpr int PLAN_THREADS = HSTU_PLAN_THREADS;
static_assert(PLAN_THREADS >= NUM_XCD * 64 && PLAN_THREADS % 64 == 0, "one wave per XCD list sums that list");
constexpr int PLAN_MAX_B = 1024;      // fast path: sequences ...
constexpr int PLAN_MAX_PAIRS = 4096;  // ... (sequence, head) pairs ...
constexpr int PLAN_MAX_TILES = 256;   // ... and query tiles per sequence that fit the LDS tables

__device__ __forceinline__ int snake_xcd(int pr) {
  const int pos = pr % NUM_XCD;
  return ((pr / NUM_XCD) & 1) ? NUM_XCD - 1 - pos : pos;
}
// position of pair pr inside its XCD list (pairs 16 k + x and 16 k + 15 - x, in that order)
__device__ __forceinline__ int snake_slot(int pr) {
  return 2 * (pr / (2 * NUM_XCD)) + ((pr % (2 * NUM_XCD)) >= NUM_XCD ? 1 : 0);
}

constexpr int PLAN_REVERSE = 1;     // item at the position of tile t carries tile nt - 1 - t
constexpr int PLAN_SHIFT_ODD = 2;   // see tile_rows
constexpr int PLAN_NO_SPREAD = 4;   // always deal whole (sequence, head) pairs
constexpr int PLAN_GROUP = 8;       // order a list by groups of PLAN_GROUP_PAIRS pairs (see plan_one_block)
constexpr int PLAN_GROUP_PAIRS = 8;
constexpr int PLAN_PAIR_CU = 16;    // see pair_pos
constexpr int CUS_PER_XCD = 32;

// A launch with two workgroups per CU places list positions s and s + 32 of an XCD on the same CU
// (read off the hardware ids of a 512-workgroup launch: the first 32 workgroups of an XCD take one
// CU each, the next 32 the same CUs in the same order; later workgroups go wherever a slot frees).
// With PLAN_PAIR_CU the second run of 32 positions is reversed, so that the heaviest item shares its
// CU with the lightest of the first 64 instead of the 33rd heaviest.  Worth 1-5 % where 64 heavy
// items open a list (long sequences), nothing at configuration 2.
__device__ __forceinline__ int pair_pos(int pos, int list_len, int mode) {
  if (!(mode & PLAN_PAIR_CU) || pos < CUS_PER_XCD) return pos;
  const int hi = min(list_len, 2 * CUS_PER_XCD);
  return pos < hi ? CUS_PER_XCD + (hi - 1 - pos) : pos;
}
#ifndef HSTU_PLAN_SPREAD_AT
#define HSTU_PLAN_SPREAD_AT 1.05f
#endif
constexpr float PLAN_SPREAD_AT = HSTU_PLAN_SPREAD_AT;  // heaviest list / mean list beyond which tiles are dealt

// Rows [q0, q_end) of tile t of a sequence of n rows cut into tiles of bm rows.  Plain cut:
// [t bm, t bm + bm).  With PLAN_SHIFT_ODD and an odd number of half tiles, tile 0 holds the first
// half tile only and the others follow it: the half-empty workgroup is then the one with the
// shortest causal prefix instead of the one with the longest.
__device__ __forceinline__ void tile_rows(int n, int bm, int t, int mode, int& q0, int& q_end) {
  const int half = bm >> 1;
  if ((mode & PLAN_SHIFT_ODD) && (((n + half - 1) / half) & 1)) {
    q0 = t == 0 ? 0 : half + (t - 1) * bm;
    q_end = t == 0 ? half : q0 + bm;
  } else {
    q0 = t * bm;
    q_end = q0 + bm;
  }
  q_end = min(q_end, n);
}

__device__ __forceinline__ void fill_item(WorkItem& w, const SeqInfo& si, int bm, int t, int nt, int mode, int h, int b) {
  w.s = si.s; w.n = si.n; w.cap = si.cap; w.ctx_eff = si.ctx_eff;
  w.h = h; w.b = b;
  tile_rows(si.n, bm, (mode & PLAN_REVERSE) ? nt - 1 - t : t, mode, w.q0, w.q_end);
}

// Fast path: everything in LDS, one block.
__device__ __forceinline__ void plan_one_block(const Params& p, int bm, int mode) {
  __shared__ int nt[PLAN_MAX_B];          // query tiles of sequence b
  __shared__ int seq_of_rank[PLAN_MAX_B];
  __shared__ int nt_by_rank[PLAN_MAX_B];
  __shared__ int xnt[NUM_XCD][PLAN_MAX_PAIRS / NUM_XCD + 2];  // tiles of the k-th pair of list x
  __shared__ int above[NUM_XCD][PLAN_MAX_TILES + 1];          // tiles of list x with index > t
  __shared__ int gbase[NUM_XCD][PLAN_MAX_PAIRS / NUM_XCD / PLAN_GROUP_PAIRS + 2];  // items of list x ahead of its group g
  __shared__ float list_work[NUM_XCD];
  __shared__ int list_total[NUM_XCD];
  __shared__ int seq_s[PLAN_MAX_B], seq_n[PLAN_MAX_B], seq_cap[PLAN_MAX_B], seq_ctx[PLAN_MAX_B];
  const int tid = threadIdx.x;
  const int B = p.B, H = p.H;
  const int pairs = B * H;
  const int per_list = (pairs + NUM_XCD - 1) / NUM_XCD + 1;  // upper bound on pairs per list

  // The kernel is a chain of short phases on one CU, so its time is the number of barriers and the
  // longest thing a single thread does between two of them: no phase has a loop over the batch or
  // over a list in one thread that the others wait for.
  for (int i = tid; i < NUM_XCD * per_list; i += PLAN_THREADS) xnt[i / per_list][i - (i / per_list) * per_list] = 0;
  for (int b = tid; b < B; b += PLAN_THREADS) {
    const SeqInfo si = seq_info(p, b);  // kept in LDS: the item phase needs it again
    seq_s[b] = si.s; seq_n[b] = si.n; seq_cap[b] = si.cap; seq_ctx[b] = si.ctx_eff;
    nt[b] = (si.n + bm - 1) / bm;
  }
  __syncthreads();
  for (int b = tid; b < B; b += PLAN_THREADS) {
    const int mine = nt[b];
    int r = 0;
    for (int b2 = 0; b2 < B; ++b2) {
      const int o = nt[b2];
      r += (o > mine) || (o == mine && b2 < b);
    }
    seq_of_rank[r] = b;
    nt_by_rank[r] = mine;
  }
  __syncthreads();
  for (int i = tid; i < pairs; i += PLAN_THREADS) xnt[snake_xcd(i)][snake_slot(i)] = nt_by_rank[i / H];
  __syncthreads();
  const int tmax = B > 0 ? nt_by_rank[0] : 0;
  // Work of a pair with v tiles ~ v (v + 1) / 2 (tile t meets t + 1 key tiles).  When dealing whole
  // pairs leaves the lists unequal (few pairs, or one sequence far longer than the rest), tiles are
  // dealt instead: see below.  Wave x sums list x.
  if (tid < NUM_XCD * 64) {
    const int x = tid >> 6;
    float w = 0.f;
    int total = 0;
    for (int k = tid & 63; k < per_list; k += 64) { const int v = xnt[x][k]; w += (float)v * ((float)v + 1.f); total += v; }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) { w += __shfl_xor(w, d, 64); total += __shfl_xor(total, d, 64); }
    if ((tid & 63) == 0) { list_work[x] = w; list_total[x] = total; }
  }
  // (the tables of the whole-pair order do not depend on that decision and are filled in the same phase)
  auto tiles_above = [&](int x, int t) {
    int a = 0;
    for (int k = 0; k < per_list; ++k) a += max(0, xnt[x][k] - 1 - t);
    return a;
  };
  const int ttab = min(tmax, PLAN_MAX_TILES) + 1;  // tabulated tile indices; beyond: computed in place
  // Grouped order (PLAN_GROUP): a list is walked group by group of PLAN_GROUP_PAIRS pairs, tile index
  // descending inside a group.  All pairs at once is the better order for balance (2-4 % at
  // configuration 2), but their K and V rows together are several times an XCD's L2; once the tensors
  // of a call no longer fit the last-level cache either, the re-fetches cost more than the balance
  // (four times configuration 2: 348 -> 317 us).  The caller decides by the size of the tensors.
  const bool grouped = (mode & PLAN_GROUP) != 0;
  const int ngroups = (per_list + PLAN_GROUP_PAIRS - 1) / PLAN_GROUP_PAIRS;
  if (grouped) {
    // items of list x in its groups before g: one thread per (list, group)
    for (int i = tid; i < NUM_XCD * (ngroups + 1); i += PLAN_THREADS) {
      const int x = i / (ngroups + 1), g = i - x * (ngroups + 1);
      int run = 0;
      for (int k = 0; k < g * PLAN_GROUP_PAIRS && k < per_list; ++k) run += xnt[x][k];
      gbase[x][g] = run;
    }
  } else {
    for (int i = tid; i < NUM_XCD * ttab; i += PLAN_THREADS) {
      const int x = i / ttab, t = i - x * ttab;
      above[x][t] = tiles_above(x, t);
    }
  }
  __syncthreads();
  bool spread = false;
  int n_items = 0;
  {
    float mx = 0.f, sum = 0.f;
    for (int x = 0; x < NUM_XCD; ++x) { mx = fmaxf(mx, list_work[x]); sum += list_work[x]; n_items += list_total[x]; }
    spread = !(mode & PLAN_NO_SPREAD) && (mx * NUM_XCD > sum * PLAN_SPREAD_AT);
  }
  if (spread) {
    // All tiles of all pairs in one order, tile index descending and pair rank ascending inside one
    // index, dealt to the lists in the same boustrophedon order: every list is still heaviest
    // first, the list sums differ by at most one tile's work, and a pair's K and V rows are read
    // through several L2s, which costs little when few pairs carry the work.
    auto all_above = [&](int t) {
      int a = 0;
      for (int r = 0; r < B; ++r) a += max(0, nt_by_rank[r] - 1 - t);
      return a * H;
    };
    for (int t = tid; t < ttab; t += PLAN_THREADS) above[0][t] = all_above(t);
    __syncthreads();
    // length of list x when n_items are dealt in boustrophedon order
    auto dealt_len = [&](int x) {
      const int part = n_items % (2 * NUM_XCD);
      return 2 * (n_items / (2 * NUM_XCD)) + (x < part ? 1 : 0) + (x >= 2 * NUM_XCD - part ? 1 : 0);
    };
    const int per_rank = tmax * H;
    for (int i = tid; i < B * per_rank; i += PLAN_THREADS) {
      const int r = i / per_rank, rem = i - r * per_rank;
      const int t = rem / H, h = rem - t * H;
      const int my_nt = nt_by_rank[r];
      if (t >= my_nt) continue;
      const int b = seq_of_rank[r];
      SeqInfo si;
      si.s = seq_s[b]; si.n = seq_n[b]; si.cap = seq_cap[b]; si.ctx_eff = seq_ctx[b];
      // the r ranks ahead have at least as many tiles, so each of their pairs owns a tile t
      const int g = (t < ttab ? above[0][t] : all_above(t)) + r * H + h;
      WorkItem w;
      fill_item(w, si, bm, t, my_nt, mode, h, b);
      const int x = snake_xcd(g);
      p.ws_items[(size_t)x * p.items_cap + pair_pos(snake_slot(g), dealt_len(x), mode)] = w;
    }
    if (tid < NUM_XCD) {
      p.ws_counts[tid] = dealt_len(tid);
      p.ws_counts[NUM_XCD + tid] = p.grid_slots;  // first list position a persistent kernel's workgroups draw
    }
    return;
  }
  // one thread per (rank, tile, head)
  const int per_rank = tmax * H;
  for (int i = tid; i < B * per_rank; i += PLAN_THREADS) {
    const int r = i / per_rank, rem = i - r * per_rank;
    const int t = rem / H, h = rem - t * H;
    const int my_nt = nt_by_rank[r];
    if (t >= my_nt) continue;
    const int b = seq_of_rank[r];
    SeqInfo si;
    si.s = seq_s[b]; si.n = seq_n[b]; si.cap = seq_cap[b]; si.ctx_eff = seq_ctx[b];
    const int pr = r * H + h;
    const int x = snake_xcd(pr), k = snake_slot(pr);
    // pairs enter a list in rank order, so the k pairs ahead of this one in its list have at least
    // as many tiles: each of them owns a tile t, and all of those come first
    int pos;
    if (grouped) {
      const int g = k / PLAN_GROUP_PAIRS, k0 = g * PLAN_GROUP_PAIRS;
      pos = gbase[x][g] + (k - k0);
      for (int kk = k0; kk < k0 + PLAN_GROUP_PAIRS && kk < per_list; ++kk) pos += max(0, xnt[x][kk] - 1 - t);
    } else {
      pos = pair_pos((t < ttab ? above[x][t] : tiles_above(x, t)) + k, list_total[x], mode);
    }
    WorkItem w;
    fill_item(w, si, bm, t, my_nt, mode, h, b);
    p.ws_items[(size_t)x * p.items_cap + pos] = w;
  }
  if (tid < NUM_XCD) {
    p.ws_counts[tid] = list_total[tid];
    p.ws_counts[NUM_XCD + tid] = p.grid_slots;
  }
}

__global__ __launch_bounds__(PLAN_THREADS) void hstu_plan_kernel(Params p, int bm, int mode) {
  plan_one_block(p, bm, mode);
}

// Two lists over the same sequences in one launch (the backward's query-tile and key-tile lists):
// block 0 builds the first, block 1 the second.
__global__ __launch_bounds__(PLAN_THREADS) void hstu_plan_pair_kernel(Params pa, int mode_a, Params pb, int mode_b, int bm) {
  if (blockIdx.x == 0) plan_one_block(pa, bm, mode_a);
  else plan_one_block(pb, bm, mode_b);
}

// General path for batches beyond the LDS tables: no ranking, pairs dealt in input order, list
// positions computed from global memory.  Slow (quadratic in the number of pairs) but only used for
// batches whose attention work dwarfs it.
__global__ __launch_bounds__(256) void hstu_plan_kernel_general(Params p, int bm, int mode) {
  const int H = p.H;
  const int pairs = p.B * H;
  const int rounds = (pairs + 2 * NUM_XCD - 1) / (2 * NUM_XCD);
  for (int pr = blockIdx.x * blockDim.x + threadIdx.x; pr < pairs; pr += gridDim.x * blockDim.x) {
    const int b = pr / H, h = pr - b * H;
    const SeqInfo si = seq_info(p, b);
    const int my_nt = (si.n + bm - 1) / bm;
    const int x = snake_xcd(pr);
    for (int t = 0; t < my_nt; ++t) {
      int pos = 0;
      for (int k16 = 0; k16 < rounds; ++k16) {
        for (int side = 0; side < 2; ++side) {
          const int o = k16 * 2 * NUM_XCD + (side ? 2 * NUM_XCD - 1 - x : x);
          if (o >= pairs) continue;
          const int nt2 = (seq_info(p, o / H).n + bm - 1) / bm;
          pos += max(0, nt2 - 1 - t) + ((o < pr && nt2 > t) ? 1 : 0);
        }
      }
      WorkItem w;
      fill_item(w, si, bm, t, my_nt, mode, h, b);
      p.ws_items[(size_t)x * p.items_cap + pos] = w;
    }
  }
  const int x = blockIdx.x * blockDim.x + threadIdx.x;
  if (x < NUM_XCD) {
    int total = 0;
    for (int pr = 0; pr < pairs; ++pr)
      if (snake_xcd(pr) == x) total += (seq_info(p, pr / H).n + bm - 1) / bm;
    p.ws_counts[x] = total;
    p.ws_counts[NUM_XCD + x] = p.grid_slots;
  }
}

}  // namespace recir_hstu
