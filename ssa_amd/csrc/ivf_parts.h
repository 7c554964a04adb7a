// Device pieces shared by the IVF router (ivf.hip) and the certified causal cascade (ccc.hip):
// ordering keys, fp64 inner products, workgroup scans, radix top-K threshold and compaction over
// LDS, and the inverted-list build (assignment keys, per-tile ranks, list scatter, centroid
// update). Everything is deterministic: inner products accumulate in fp64 in dimension order and
// round once to fp32, ties go to the lower index, list members stay in ascending order.
#pragma once
#include <math.h>

#include "common.h"

namespace ssa {
namespace {
constexpr int kIvfMaxD = 256;      // head dim: a multiple of 32, at most this
constexpr int kIvfCap = 2048;      // LDS keys per route pass (coarse keys, candidates, the union)
constexpr int kIvfMaxSearch = kIvfCap / 2;
constexpr int kAssignC = 16;       // centroids staged in LDS per assignment pass
constexpr int kTile = 256;         // block means per rank / scatter workgroup
constexpr int kScoreTile = 64;     // block means per scoring workgroup (one wave)

inline size_t r256(size_t x) { return (x + 255) & ~size_t(255); }

// Unique, order-preserving key of (score, index): larger score first, then lower index.
__device__ inline unsigned long long ivf_key(float s, int64_t idx) {
  return ((unsigned long long)score_key(s) << 32) |
         (unsigned long long)(0xffffffffu - (unsigned int)idx);
}

__device__ inline int64_t ivf_key_index(unsigned long long k) {
  return (int64_t)(0xffffffffu - (unsigned int)(k & 0xffffffffull));
}

// <q, x> with q in LDS and x[t] at col[t * stride] (d a multiple of 32), accumulated in fp64 in
// dimension order (a product of two fp32 values is exact in fp64, so each step rounds once) and
// rounded once to fp32. Each 32-element chunk of x is loaded in one burst before its fmas.
__device__ inline float dot_strided(const float* q, const float* col, int64_t stride,
                                    int64_t d) {
  double acc = 0.0;
  for (int64_t t0 = 0; t0 < d; t0 += 32) {
    float x[32];
#pragma unroll
    for (int u = 0; u < 32; ++u) x[u] = col[(t0 + u) * stride];
#pragma unroll
    for (int u = 0; u < 32; u += 4) {
      const float4 qq = *reinterpret_cast<const float4*>(q + t0 + u);
      acc = fma((double)qq.x, (double)x[u], acc);
      acc = fma((double)qq.y, (double)x[u + 1], acc);
      acc = fma((double)qq.z, (double)x[u + 2], acc);
      acc = fma((double)qq.w, (double)x[u + 3], acc);
    }
  }
  return (float)acc;
}

// Exclusive prefix of v over a 256-thread workgroup; *total = the sum. ws holds 4 ints.
__device__ inline int ivf_block_scan(int v, int* ws, int* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) ws[w] = x;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (k < w) base += ws[k];
    tot += ws[k];
  }
  __syncthreads();
  *total = tot;
  return base + x - v;
}

// A threshold T with exactly K of the n keys in LDS >= T (0 < K <= n, the K largest keys
// distinct), by an MSB-first radix walk over 8-bit digits that stops once the digit's whole bin
// is taken (T then ends in zero bits). 256 threads; shv holds 3 ints.
__device__ unsigned long long block_kth_largest(const unsigned long long* keys, int n, int K,
                                                unsigned int* hist, unsigned int* shv) {
  const int tid = threadIdx.x, lane = tid & 63;
  unsigned long long prefix = 0ull;
  int need = K;
  for (int shift = 56; shift >= 0; shift -= 8) {
    hist[tid] = 0u;
    __syncthreads();
    const unsigned long long hi = shift == 56 ? 0ull : (~0ull << (shift + 8));
    for (int e = tid; e < n; e += 256) {
      const unsigned long long k = keys[e];
      if ((k & hi) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      const unsigned int c0 = hist[4 * lane], c1 = hist[4 * lane + 1];
      const unsigned int c2 = hist[4 * lane + 2], c3 = hist[4 * lane + 3];
      const unsigned int s = c0 + c1 + c2 + c3;
      unsigned int suf = s;  // sum over lanes >= this one
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const unsigned int y = __shfl_down(suf, o);
        if (lane + o < 64) suf += y;
      }
      unsigned int above = suf - s;  // keys in the bins above this lane's four
      const unsigned int cb[4] = {c0, c1, c2, c3};
#pragma unroll
      for (int b = 3; b >= 0; --b) {
        if (above < (unsigned int)need && (unsigned int)need <= above + cb[b]) {
          shv[0] = 4u * lane + b;
          shv[1] = (unsigned int)need - above;
          shv[2] = (unsigned int)need == above + cb[b];
        }
        above += cb[b];
      }
    }
    __syncthreads();
    prefix |= (unsigned long long)shv[0] << shift;
    need = (int)shv[1];
    const bool whole = shv[2] != 0u;
    __syncthreads();
    if (whole) break;  // uniform: every key of the bin is taken
  }
  return prefix;
}

// ---- build --------------------------------------------------------------------------------------
// One wave per (tile of 128 block means, centroid group): the key of the best centroid of the
// group for each block mean (largest inner product, ties to the lower centroid). Each lane owns
// block means j and j + 64, so every staged centroid value (widened to fp64 once, when staged in
// LDS, 2 per 16-byte read) feeds two fp64 chains with no conversion in the loop. Dynamic LDS:
// kAssignC * d doubles.
__global__ __launch_bounds__(kScoreTile) void ivf_score_kernel(
    const float* __restrict__ mu, const float* __restrict__ cent, int64_t nb, int64_t d,
    int64_t nlist, int64_t per_group, unsigned long long* __restrict__ pbest) {
  extern __shared__ double scd[];  // d x kAssignC: element t of centroid c0 + c at t * kAssignC + c
  const int tid = threadIdx.x;
  const int64_t bh = blockIdx.y, tile = blockIdx.x, g = blockIdx.z;
  int64_t j[2];
  bool live[2];
  const float* row[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    j[h] = tile * 2 * kScoreTile + h * kScoreTile + tid;
    live[h] = j[h] < nb;
    row[h] = mu + (bh * nb + (live[h] ? j[h] : nb - 1)) * d;  // idle lanes read a valid row
  }
  const float* cb = cent + bh * nlist * d;
  const int64_t cbeg = g * per_group;
  const int64_t cend = cbeg + per_group < nlist ? cbeg + per_group : nlist;
  unsigned long long best[2] = {0ull, 0ull};
  for (int64_t c0 = cbeg; c0 < cend; c0 += kAssignC) {
    const int cc = (int)(cend - c0 < kAssignC ? cend - c0 : kAssignC);
    __syncthreads();
    for (int e = tid; e < kAssignC * (int)d; e += kScoreTile) {
      const int c = e / (int)d, t = e - c * (int)d;
      scd[t * kAssignC + c] = c < cc ? (double)cb[(c0 + c) * d + t] : 0.0;
    }
    __syncthreads();
    double acc[2][kAssignC];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int c = 0; c < kAssignC; ++c) acc[h][c] = 0.0;
    for (int64_t t0 = 0; t0 < d; t0 += 16) {
      float r[2][16];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float4 x = *reinterpret_cast<const float4*>(row[h] + t0 + 4 * u);
          r[h][4 * u] = x.x;
          r[h][4 * u + 1] = x.y;
          r[h][4 * u + 2] = x.z;
          r[h][4 * u + 3] = x.w;
        }
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const double2* s2 = reinterpret_cast<const double2*>(scd + (t0 + t) * kAssignC);
        double cv[kAssignC];
#pragma unroll
        for (int q = 0; q < kAssignC / 2; ++q) {
          const double2 x = s2[q];
          cv[2 * q] = x.x;
          cv[2 * q + 1] = x.y;
        }
        const double r0 = r[0][t], r1 = r[1][t];
#pragma unroll
        for (int c = 0; c < kAssignC; ++c) {
          acc[0][c] = fma(r0, cv[c], acc[0][c]);
          acc[1][c] = fma(r1, cv[c], acc[1][c]);
        }
      }
    }
#pragma unroll
    for (int c = 0; c < kAssignC; ++c) {
      if (c < cc) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const unsigned long long k = ivf_key((float)acc[h][c], c0 + c);
          best[h] = k > best[h] ? k : best[h];
        }
      }
    }
  }
#pragma unroll
  for (int h = 0; h < 2; ++h)
    if (live[h]) pbest[(bh * gridDim.z + g) * nb + j[h]] = best[h];
}

// One workgroup per tile: each block mean joins the best of its groups' centroids; rank = its
// position among the tile's members of that centroid, and the tile's member count of every
// centroid goes to its tcount row (0 for absent ones).
__global__ __launch_bounds__(256) void ivf_rank_kernel(
    const unsigned long long* __restrict__ pbest, int64_t nb, int64_t nlist, int64_t ntiles,
    int64_t groups, int32_t* __restrict__ assign, int32_t* __restrict__ rank,
    int32_t* __restrict__ tcount) {
  __shared__ int sa[kTile];
  const int tid = threadIdx.x;
  const int64_t bh = blockIdx.y, tile = blockIdx.x;
  const int64_t j = tile * kTile + tid;
  const bool live = j < nb;
  int32_t* trow = tcount + (bh * ntiles + tile) * nlist;
  for (int64_t c = tid; c < nlist; c += kTile) trow[c] = 0;
  unsigned long long best = 0ull;
  const unsigned long long* pb = pbest + bh * groups * nb + (live ? j : 0);
  for (int64_t g0 = 0; g0 < groups; g0 += 8) {  // 8 loads in flight (clamped to a valid group)
    unsigned long long k[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) k[u] = pb[(g0 + u < groups ? g0 + u : groups - 1) * nb];
#pragma unroll
    for (int u = 0; u < 8; ++u) best = k[u] > best ? k[u] : best;
  }
  const int a = live ? (int)ivf_key_index(best) : -1;
  sa[tid] = a;
  __syncthreads();  // also orders the zeroing of trow before the counts below
  if (live) {
    int r = 0;
    bool last = true;
    for (int t = 0; t < kTile; ++t) {
      const int x = sa[t];
      if (t < tid) r += (x == a);
      else if (t > tid && x == a) last = false;
    }
    assign[bh * nb + j] = a;
    rank[bh * nb + j] = r;
    if (last) trow[a] = r + 1;
  }
}

// One workgroup per (centroid, head): tcount[t] <- the centroid's members in the tiles before t
// (an exclusive prefix over the tiles, in place, 256 tiles per pass) and count = its members in
// all tiles. Work O(tiles x centroids). With gate set, nothing runs unless *gate != 0.
__global__ __launch_bounds__(256) void ivf_tile_prefix_kernel(int32_t* __restrict__ tcount,
                                                               int64_t ntiles, int64_t nlist,
                                                               int32_t* __restrict__ count,
                                                               const int32_t* __restrict__ gate) {
  __shared__ int ws[4];
  if (gate != nullptr && *gate == 0) return;
  const int64_t bh = blockIdx.y, c = blockIdx.x;
  int32_t* col = tcount + bh * ntiles * nlist + c;
  int running = 0;
  for (int64_t t0 = 0; t0 < ntiles; t0 += 256) {
    const int64_t t = t0 + threadIdx.x;
    const int v = t < ntiles ? col[t * nlist] : 0;
    int tot;
    const int ex = ivf_block_scan(v, ws, &tot);
    if (t < ntiles) col[t * nlist] = running + ex;
    running += tot;
  }
  if (threadIdx.x == 0) count[bh * nlist + c] = running;
}

// One workgroup per head: off[c] = the members of the centroids before c, off[nlist] = all.
__global__ __launch_bounds__(256) void ivf_offsets_kernel(const int32_t* __restrict__ count,
                                                           int64_t nlist,
                                                           int32_t* __restrict__ off) {
  __shared__ int ws[4];
  const int64_t bh = blockIdx.x;
  const int tid = threadIdx.x;
  int running = 0;
  for (int64_t c0 = 0; c0 < nlist; c0 += 256) {
    const int64_t c = c0 + tid;
    const int v = c < nlist ? count[bh * nlist + c] : 0;
    int tot;
    const int ex = ivf_block_scan(v, ws, &tot);
    if (c < nlist) off[bh * (nlist + 1) + c] = running + ex;
    running += tot;
  }
  if (tid == 0) off[bh * (nlist + 1) + nlist] = running;
}

// One thread per block mean: its slot in ids = offset of its list + members of the list in
// earlier tiles (tbase, the prefix of ivf_tile_prefix_kernel) + its rank in its tile. With muL set
// (the last assignment), the mean is also copied to its list's transposed storage: element t of
// member k of list p at d * off[p] + t * size[p] + k.
__global__ __launch_bounds__(256) void ivf_scatter_kernel(
    const int32_t* __restrict__ assign, const int32_t* __restrict__ rank,
    const int32_t* __restrict__ tbase, int64_t nb, int64_t nlist, int64_t ntiles,
    const int32_t* __restrict__ count, const int32_t* __restrict__ off, int32_t* __restrict__ ids,
    const float* __restrict__ mu, int64_t d, float* __restrict__ muL) {
  const int64_t bh = blockIdx.y, tile = blockIdx.x;
  const int64_t j = tile * kTile + threadIdx.x;
  if (j >= nb) return;
  const int a = assign[bh * nb + j];
  const int o = off[bh * (nlist + 1) + a];
  const int pos = o + tbase[(bh * ntiles + tile) * nlist + a] + rank[bh * nb + j];
  ids[bh * nb + pos] = (int32_t)j;
  if (muL != nullptr) {
    const int64_t L = count[bh * nlist + a];
    const float* src = mu + (bh * nb + j) * d;
    float* dst = muL + bh * nb * d + d * (int64_t)o + (pos - o);
    for (int64_t t = 0; t < d; ++t) dst[t * L] = src[t];
  }
}

// The lists of an assignment whose per-tile ranks and counts (tcount) are set: sizes, offsets,
// member ids in ascending order and, with muL, the transposed member storage. tcount is
// overwritten with its prefix over the tiles.
inline int ivf_lists(const int32_t* assign, const int32_t* rank, int32_t* tcount, int64_t BH,
                     int64_t nb, int64_t nlist, int64_t ntiles, int32_t* count, int32_t* off,
                     int32_t* ids, const float* mu, int64_t d, float* muL, hipStream_t s) {
  ivf_tile_prefix_kernel<<<dim3((unsigned)nlist, (unsigned)BH), 256, 0, s>>>(tcount, ntiles,
                                                                             nlist, count, nullptr);
  SSA_TRY(launch_status("ivf_tile_prefix_kernel"));
  ivf_offsets_kernel<<<(unsigned)BH, 256, 0, s>>>(count, nlist, off);
  SSA_TRY(launch_status("ivf_offsets_kernel"));
  ivf_scatter_kernel<<<dim3((unsigned)ntiles, (unsigned)BH), 256, 0, s>>>(
      assign, rank, tcount, nb, nlist, ntiles, count, off, ids, mu, d, muL);
  return launch_status("ivf_scatter_kernel");
}

// centT (BH, d, nlist) = the centroids transposed.
__global__ __launch_bounds__(64) void ivf_transpose_cent_kernel(const float* __restrict__ cent,
                                                                 int64_t d, int64_t nlist,
                                                                 float* __restrict__ centT) {
  const int64_t bh = blockIdx.y, c = blockIdx.x;
  for (int64_t t = threadIdx.x; t < d; t += 64)
    centT[(bh * d + t) * nlist + c] = cent[(bh * nlist + c) * d + t];
}

// Centroid c <- normalised sum of its members (fp64, ascending member order; SPHERICAL), or
// fl32(sum / count), the members' mean (!SPHERICAL); unchanged when it has no members (or, when
// SPHERICAL, their sum is zero). Lane l owns dimensions l + 64 u, u < NU (d <= 64 NU); every load
// is unconditional (clamped to a valid address) so a batch of them is in flight before the
// in-order adds.
template <int NU, bool SPHERICAL = true>
__global__ __launch_bounds__(64) void ivf_update_kernel(
    const float* __restrict__ mu, const int32_t* __restrict__ count,
    const int32_t* __restrict__ off, const int32_t* __restrict__ ids, int64_t nb, int64_t d,
    int64_t nlist, float* __restrict__ cent) {
  __shared__ double sd[kIvfMaxD];
  __shared__ double snrm;
  const int64_t bh = blockIdx.y, c = blockIdx.x;
  const int lane = threadIdx.x;
  const int L = count[bh * nlist + c];
  if (L == 0) return;
  const int32_t* mem = ids + bh * nb + off[bh * (nlist + 1) + c];
  const float* mb = mu + bh * nb * d;
  int64_t tt[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) tt[u] = lane + 64 * u < d ? lane + 64 * u : 0;
  double acc[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) acc[u] = 0.0;
  constexpr int kB = 16;  // members whose values are loaded before they are added in order
  for (int k0 = 0; k0 < L; k0 += kB) {
    float v[kB][NU];
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      const int64_t j = mem[k0 + b < L ? k0 + b : L - 1];
#pragma unroll
      for (int u = 0; u < NU; ++u) v[b][u] = mb[j * d + tt[u]];
    }
    const int nbat = L - k0 < kB ? L - k0 : kB;
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      if (b < nbat) {
#pragma unroll
        for (int u = 0; u < NU; ++u) acc[u] = __dadd_rn(acc[u], (double)v[b][u]);
      }
    }
  }
  if constexpr (!SPHERICAL) {
    float* dst = cent + (bh * nlist + c) * d;
#pragma unroll
    for (int u = 0; u < NU; ++u)
      if (lane + 64 * u < d) dst[lane + 64 * u] = (float)(acc[u] / (double)L);
    return;
  }
#pragma unroll
  for (int u = 0; u < NU; ++u)
    if (lane + 64 * u < d) sd[lane + 64 * u] = acc[u];
  __syncthreads();
  if (lane == 0) {
    double nrm = 0.0;
    for (int64_t t = 0; t < d; ++t) nrm = __dadd_rn(nrm, __dmul_rn(sd[t], sd[t]));
    snrm = nrm;
  }
  __syncthreads();
  const double nrm = snrm;
  if (!(nrm > 0.0)) return;
  const double r = sqrt(nrm);
  float* dst = cent + (bh * nlist + c) * d;
  for (int64_t t = lane; t < d; t += 64) dst[t] = (float)(sd[t] / r);
}

// ---- route --------------------------------------------------------------------------------------
// Compacts the entries of v[0..n) (LDS, at most 8 per thread) for which take(entry) holds to
// dst[0..), in any order; returns how many. 256 threads.
template <typename T, typename F>
__device__ inline int block_compact(const T* v, int n, T* dst, int* ws, F take) {
  T mine[kIvfCap / 256];
  bool keep[kIvfCap / 256];
  int cnt = 0;
#pragma unroll
  for (int u = 0; u < kIvfCap / 256; ++u) {
    const int e = threadIdx.x + 256 * u;
    keep[u] = e < n && take(v[e]);
    mine[u] = e < n ? v[e] : T(0);
    cnt += keep[u];
  }
  int total;
  int pos = ivf_block_scan(cnt, ws, &total);  // its barriers order the reads before the writes
#pragma unroll
  for (int u = 0; u < kIvfCap / 256; ++u)
    if (keep[u]) dst[pos++] = mine[u];
  __syncthreads();
  return total;
}

}  // namespace
}  // namespace ssa
