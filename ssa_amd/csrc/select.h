// Wave-level selection of the K largest keys (one entry per lane and slot j: entry lane + 64 j),
// shared by the router's select kernels and the fused decode route.
#pragma once

#include "common.h"

namespace ssa {

// The K-th largest of a wave's entries (lane l, slot j: entry l + 64 j; non-candidates hold
// key 0), found bit by bit from the top (count of keys >= T | bit by ballots), or the first
// prefix with exactly K keys >= T -- then no tie straddles the cut. Requires 0 < K < #candidates.
// The search starts below the leading bits that every nonzero key shares (the K-th largest
// shares them when at least K keys are nonzero).
template <int J>
__device__ inline unsigned int wave_kth_key(const unsigned int (&key)[J], int64_t K) {
  unsigned int all = 0xffffffffu, any = 0u;
  int nz = 0;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    all &= key[j] ? key[j] : 0xffffffffu;
    any |= key[j];
    nz += __popcll(__ballot(key[j] != 0u));
  }
  if (nz < K) return 0u;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    all &= lane_xor(all, off);
    any |= lane_xor(any, off);
  }
  const unsigned int diff = all ^ any;  // bits on which nonzero keys differ
  if (diff == 0u) return all;           // one distinct nonzero key
  const int top = 31 - __clz(diff);
  unsigned int T = top == 31 ? 0u : all & ~((2u << top) - 1u);
  for (int bit = top; bit >= 0; --bit) {
    const unsigned int t = T | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) cnt += __popcll(__ballot(key[j] >= t));
    if (cnt >= K) {
      T = t;
      if (cnt == K) break;  // wave-uniform
    }
  }
  return T;
}

// The K largest of a wave's candidates (bit j of the lane's mask cm: entry lane + 64 j is one;
// non-candidates must hold key 0) under the order (key desc, entry asc), as a per-lane mask:
// keys > T (the K-th largest) are taken, and keys == T in increasing entry order until K are
// taken. ncand is the number of candidates.
// With kth != NULL, *kth = T (0 when every candidate is taken or K <= 0).
template <int J>
__device__ inline unsigned int wave_select_top(const unsigned int (&key)[J], unsigned int cm,
                                               int64_t K, int64_t ncand,
                                               unsigned int* kth = nullptr) {
  const int lane = threadIdx.x & 63;
  const unsigned long long lt = (1ull << lane) - 1ull;
  if (kth) *kth = 0u;
  if (K >= ncand) return cm;
  if (K <= 0) return 0u;
  const unsigned int T = wave_kth_key<J>(key, K);
  if (kth) *kth = T;
  int above = 0;
#pragma unroll
  for (int j = 0; j < J; ++j) above += __popcll(__ballot(((cm >> j) & 1u) && key[j] > T));
  int need = (int)K - above;  // keys equal to T to take, lowest entry first
  unsigned int selm = 0u;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const bool cd = (cm >> j) & 1u;
    const bool eq = cd && key[j] == T;
    const unsigned long long be = __ballot(eq);
    // (int) casts: __popcll is unsigned, and need turns negative once the ties are taken
    const bool take = (cd && key[j] > T) || (eq && (int)__popcll(be & lt) < need);
    selm |= (take ? 1u : 0u) << j;
    need -= (int)__popcll(be);
  }
  return selm;
}

// Bitonic sort of one (key, block) pair per lane across the wave: descending keys, ties by
// ascending block (the router's order); lane j ends with the (j+1)-th.
__device__ inline void wave_sort_desc(unsigned int& key, unsigned int& blk) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
    for (int j = k >> 1; j >= 1; j >>= 1) {
      const unsigned int ok = lane_xor(key, j), ob = lane_xor(blk, j);
      // does the partner rank before this lane's pair?
      const bool before = ok > key || (ok == key && ob < blk);
      const bool lower = (lane & j) == 0, desc = (lane & k) == 0;
      // the lower lane of a descending pair keeps the better pair, and so on
      const bool take = (lower == desc) ? before : !before;
      if (take) {
        key = ok;
        blk = ob;
      }
    }
}

// Block-wide exclusive scan of one int per thread (NT threads); returns the exclusive prefix
// and writes the total to *total.
template <int NT>
__device__ inline int block_exclusive_scan(int v, int* wave_sums, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  if (lane == 63) wave_sums[wave] = incl;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    if (w < wave) base += wave_sums[w];
    tot += wave_sums[w];
  }
  __syncthreads();
  *total = tot;
  return base + incl - v;
}

}  // namespace ssa
