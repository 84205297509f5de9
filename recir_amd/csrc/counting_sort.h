// Stable counting sort of small non-negative integer keys with their indices, for the two index
// lists of the timestamp / position embedding add (position rows < P, time buckets <= 2048): the
// keys of list x come out ascending in out_keys, out_idx[j] is the token the j-th key came from,
// and equal keys keep token order -- what a stable argsort gives
// (recir/ops/kjt_split_per_feature.cpp:401-417).  Three launches for both lists together, where a
// general-purpose radix or merge sort of 40,000 keys takes a dozen dependent launches per list.
//
// The tokens are cut into NW contiguous chunks, one per wave:
//   count    wave w counts its chunk's keys (LDS histogram)                 counts[w][k]
//   scan     counts[w][k] := keys k in chunks before w; starts[k] := keys k in all chunks
//   scatter  every block turns starts into "keys below k" (a block scan in LDS); then wave w walks
//            its chunk in token order, 64 tokens a step: lanes holding the same key
//            find each other with one ballot per key bit, the lowest of them advances the key's
//            cursor (its own LDS copy, so no other wave interferes) and all take consecutive slots
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace recir_jagged {

constexpr int CSORT_MAX_K = 8192;        // keys per list the LDS histograms hold (one wave: 32 KB)
constexpr int CSORT_BATCH = 16;          // steps of 64 tokens whose keys a wave loads at once
constexpr int CSORT_MAX_CHUNKS = 1024;   // waves the tokens are cut for, at most

struct CsortList {
  const int* keys;   // [L], values in [0, K)
  int* out_keys;     // [L]
  int* out_idx;      // [L]
  int* counts;       // [NW][K] scratch
  int* starts;       // [K] scratch: keys k in all chunks
  int K, bits;       // bits: number of key bits that can be set
};
struct CsortParams {
  CsortList list[2];
  long long L;
  int NW, CW;        // chunks and tokens per chunk (a multiple of 64)
  int kmax;          // larger K of the two lists: stride of a wave's LDS histogram
};

__global__ __launch_bounds__(256) void csort_count(CsortParams p) {
  extern __shared__ int csort_lds[];
  const CsortList& l = p.list[blockIdx.y];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int w = blockIdx.x * (blockDim.x >> 6) + wave;
  if (w >= p.NW) return;
  int* hist = csort_lds + (size_t)wave * p.kmax;  // touched by this wave only
  for (int k = lane; k < l.K; k += 64) hist[k] = 0;
  const long long begin = (long long)w * p.CW, end = begin + p.CW < p.L ? begin + p.CW : p.L;
  for (long long s0 = begin; s0 < end; s0 += 64 * CSORT_BATCH) {
    int key[CSORT_BATCH];  // the loads of a batch of steps go out together
#pragma unroll
    for (int r = 0; r < CSORT_BATCH; ++r) {
      const long long i = s0 + r * 64 + lane;
      key[r] = i < end ? l.keys[i] : -1;
    }
#pragma unroll
    for (int r = 0; r < CSORT_BATCH; ++r)
      if (key[r] >= 0) atomicAdd(&hist[key[r] > l.K - 1 ? l.K - 1 : key[r]], 1);
  }
  for (int k = lane; k < l.K; k += 64) l.counts[(size_t)w * l.K + k] = hist[k];
}

// counts[w][k] := keys k in chunks before w; starts[k] := keys k in all chunks (summed over the keys
// by the scatter kernel).  One thread per key, the chunk loop reads eight counts ahead of the stores.
__global__ __launch_bounds__(256) void csort_scan(CsortParams p) {
  const CsortList& l = p.list[blockIdx.y];
  const int k = blockIdx.x * 256 + threadIdx.x;
  if (k >= l.K) return;
  int* col = l.counts + k;
  int run = 0;
  for (int w0 = 0; w0 < p.NW; w0 += 8) {
    int c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = w0 + j < p.NW ? col[(size_t)(w0 + j) * l.K] : 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (w0 + j < p.NW) col[(size_t)(w0 + j) * l.K] = run;
      run += c[j];
    }
  }
  l.starts[k] = run;
}

__global__ __launch_bounds__(256) void csort_scatter(CsortParams p) {
  extern __shared__ int csort_lds[];
  const CsortList& l = p.list[blockIdx.y];
  const int tid = threadIdx.x, nthreads = blockDim.x;
  const int lane = tid & 63, wave = tid >> 6;
  // exclusive prefix of the per-key totals, by the whole block, in LDS: first[k] = keys below k
  int* first = csort_lds;
  __shared__ int partial[256];
  const int per = (l.K + nthreads - 1) / nthreads;
  int sum = 0;
#pragma unroll 8
  for (int j = 0; j < per; ++j) {
    const int k = tid * per + j;
    sum += k < l.K ? l.starts[k] : 0;
  }
  partial[tid] = sum;
  __syncthreads();
  for (int step = 1; step < nthreads; step <<= 1) {
    const int add = tid >= step ? partial[tid - step] : 0;
    __syncthreads();
    partial[tid] += add;
    __syncthreads();
  }
  int run = partial[tid] - sum;
  for (int j = 0; j < per; ++j) {
    const int k = tid * per + j;
    if (k < l.K) {
      first[k] = run;
      run += l.starts[k];
    }
  }
  __syncthreads();
  const int w = blockIdx.x * (nthreads >> 6) + wave;
  if (w >= p.NW) return;
  volatile int* cursor = csort_lds + (size_t)(1 + wave) * p.kmax;  // this wave's next slot of every key
  {
    const int* mine = l.counts + (size_t)w * l.K;
    for (int k0 = lane; k0 < l.K; k0 += 64 * 8) {
      int c[8];  // eight loads ahead of the stores
#pragma unroll
      for (int j = 0; j < 8; ++j) c[j] = k0 + 64 * j < l.K ? mine[k0 + 64 * j] : 0;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (k0 + 64 * j < l.K) cursor[k0 + 64 * j] = c[j] + first[k0 + 64 * j];
    }
  }
  const long long begin = (long long)w * p.CW, end = begin + p.CW < p.L ? begin + p.CW : p.L;
  const unsigned long long below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  for (long long s0 = begin; s0 < end; s0 += 64 * CSORT_BATCH) {
    int keys[CSORT_BATCH];  // the loads of a batch of steps go out together
#pragma unroll
    for (int r = 0; r < CSORT_BATCH; ++r) {
      const long long i = s0 + r * 64 + lane;
      keys[r] = i < end ? l.keys[i] : -1;
    }
#pragma unroll
    for (int r = 0; r < CSORT_BATCH; ++r) {
      const long long i = s0 + r * 64 + lane;
      const bool valid = keys[r] >= 0;
      const int key = keys[r] > l.K - 1 ? l.K - 1 : (keys[r] < 0 ? 0 : keys[r]);
      unsigned long long same = __ballot(valid);
      if (same == 0) break;  // past the end of the chunk (uniform)
      for (int b = 0; b < l.bits; ++b) {
        const bool bit = (key >> b) & 1;
        const unsigned long long m = __ballot(bit);
        same &= bit ? m : ~m;
      }
      if (!valid) same = 1ull << lane;  // keeps the arithmetic below defined; nothing is written
      const int rank = __popcll(same & below);
      const int leader = __ffsll((long long)same) - 1;
      int base = 0;
      if (valid && lane == leader) {
        base = cursor[key];
        cursor[key] = base + __popcll(same);
      }
      base = __shfl(base, leader);
      if (valid) {
        l.out_keys[base + rank] = key;
        l.out_idx[base + rank] = (int)i;
      }
    }
  }
}

}  // namespace recir_jagged
