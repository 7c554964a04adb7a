// IVF router over block means: a deterministic, faiss-free restatement of the GpuIndexIVFFlat
// block router of ssa/ivf_kernel.py:63-119 (build_ivf, _route_head, ivf_route).
//
// Build (ssa_ivf_build; build_ivf = faiss train + add, ssa/ivf_kernel.py:63-69):
//   each head's nlist centroids start at the normalised key-block means mu[c * nb / nlist] and run
//   niter rounds of spherical k-means (the clustering faiss runs for an inner-product IVF index):
//   every block mean joins the centroid of largest inner product, then each centroid becomes the
//   normalised sum of its members (a centroid without members keeps its value). A last assignment
//   fills the inverted lists, each holding its members in ascending block order.
// Route (ssa_ivf_route; _route_head, ssa/ivf_kernel.py:72-99), per query block i:
//   the nprobe lists of largest <qb_i, centroid>, the search_k members of those lists of largest
//   <qb_i, mu_j>, the first top_c of them (by score) with j <= i, OR the own block and `local`
//   predecessors; ascending in kv_idx, padded with 0, counted in kv_num.
// Every inner product is accumulated in fp64 in dimension order and rounded once to fp32; ties go
// to the lower centroid / block index. Member sums run in ascending member order, so the whole
// index is deterministic and reproducible on the CPU.
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

// Byte offsets of the index regions (see ssa_ivf_index_size in ssa_hip.h). After the four
// documented regions: the centroids transposed (BH, d, nlist) and the block means of every list
// stored list by list, each list transposed (d, size) -- the route reads both with coalesced
// loads -- then the build's scratch. The assignment splits the centroids into `groups` ranges so
// that the scoring launch holds about 2048 waves.
struct IvfLayout {
  size_t cent, count, off, ids, centT, muL, assign, rank, tcount, pbest, total;
  int64_t ntiles, stiles, groups, per_group;
};

IvfLayout ivf_layout(int64_t BH, int64_t nb, int64_t nlist, int64_t d) {
  IvfLayout L;
  L.ntiles = (nb + kTile - 1) / kTile;
  const int64_t gmax = (nlist + kAssignC - 1) / kAssignC;
  L.stiles = (nb + 2 * kScoreTile - 1) / (2 * kScoreTile);
  int64_t g = (2048 + L.stiles * BH - 1) / (L.stiles * BH);
  L.groups = g < 1 ? 1 : (g > gmax ? gmax : g);
  L.per_group = (nlist + L.groups - 1) / L.groups;
  size_t o = 0;
  L.cent = o;   o += r256(size_t(BH) * nlist * d * 4);
  L.count = o;  o += r256(size_t(BH) * nlist * 4);
  L.off = o;    o += r256(size_t(BH) * (nlist + 1) * 4);
  L.ids = o;    o += r256(size_t(BH) * nb * 4);
  L.centT = o;  o += r256(size_t(BH) * nlist * d * 4);
  L.muL = o;    o += r256(size_t(BH) * nb * d * 4);
  L.assign = o; o += r256(size_t(BH) * nb * 4);
  L.rank = o;   o += r256(size_t(BH) * nb * 4);
  L.tcount = o; o += r256(size_t(BH) * L.ntiles * nlist * 4);
  L.pbest = o;  o += r256(size_t(BH) * L.groups * nb * 8);
  L.total = o;
  return L;
}

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

// Writes fl32(s / sqrt(sum_t s_t^2)) (the squares summed in dimension order), or s itself when
// the norm is zero. s in LDS as fp64; 64 threads, d <= 256.
__device__ inline void store_normalised(const double* s, int64_t d, double* snrm, float* dst) {
  const int lane = threadIdx.x;
  if (lane == 0) {
    double nrm = 0.0;
    for (int64_t t = 0; t < d; ++t) nrm = __dadd_rn(nrm, __dmul_rn(s[t], s[t]));
    *snrm = nrm;
  }
  __syncthreads();
  const double nrm = *snrm;
  const double r = nrm > 0.0 ? sqrt(nrm) : 1.0;
  for (int64_t t = lane; t < d; t += 64) dst[t] = (float)(nrm > 0.0 ? s[t] / r : s[t]);
}

// Centroid c of head bh starts at the normalised key-block mean mu[c * nb / nlist].
__global__ __launch_bounds__(64) void ivf_init_kernel(const float* __restrict__ mu, int64_t nb,
                                                       int64_t d, int64_t nlist,
                                                       float* __restrict__ cent) {
  __shared__ double sd[kIvfMaxD];
  __shared__ double snrm;
  const int64_t bh = blockIdx.y, c = blockIdx.x;
  const int64_t j = c * nb / nlist;
  const float* src = mu + (bh * nb + j) * d;
  for (int64_t t = threadIdx.x; t < d; t += 64) sd[t] = (double)src[t];
  __syncthreads();
  store_normalised(sd, d, &snrm, cent + (bh * nlist + c) * d);
}

// One wave per (tile of 128 block means, centroid group): the key of the best centroid of the
// group for each block mean (largest inner product, ties to the lower centroid). Each lane owns
// block means j and j + 64, so every staged centroid value (fp32 in LDS, 4 per 16-byte read)
// feeds two fp64 chains: LDS traffic, not the fp64 rate, bounds this loop.
__global__ __launch_bounds__(kScoreTile) void ivf_score_kernel(
    const float* __restrict__ mu, const float* __restrict__ cent, int64_t nb, int64_t d,
    int64_t nlist, int64_t per_group, unsigned long long* __restrict__ pbest) {
  extern __shared__ float scf[];  // d x kAssignC: element t of centroid c0 + c at t * kAssignC + c
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
      scf[t * kAssignC + c] = c < cc ? cb[(c0 + c) * d + t] : 0.0f;
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
        const float4* s4 = reinterpret_cast<const float4*>(scf + (t0 + t) * kAssignC);
        double cv[kAssignC];
#pragma unroll
        for (int q = 0; q < kAssignC / 4; ++q) {
          const float4 x = s4[q];
          cv[4 * q] = x.x;
          cv[4 * q + 1] = x.y;
          cv[4 * q + 2] = x.z;
          cv[4 * q + 3] = x.w;
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

// One workgroup per tile: list sizes (count), list offsets (off, nlist + 1 per head) and, for the
// tile's block means, their slots in ids: offset of the list + members in earlier tiles + rank.
// Every workgroup derives the offsets from tcount; tile 0 writes count and off. With muL set
// (the last assignment), each block mean is also copied to its list's transposed storage:
// element t of member k of list p at d * off[p] + t * size[p] + k.
__global__ __launch_bounds__(256) void ivf_scatter_kernel(
    const int32_t* __restrict__ assign, const int32_t* __restrict__ rank,
    const int32_t* __restrict__ tcount, int64_t nb, int64_t nlist, int64_t ntiles,
    int32_t* __restrict__ count, int32_t* __restrict__ off, int32_t* __restrict__ ids,
    const float* __restrict__ mu, int64_t d, float* __restrict__ muL) {
  __shared__ int base[kIvfCap];
  __shared__ int offl[kIvfCap];
  __shared__ int cntl[kIvfCap];
  __shared__ int ws[4];
  const int tid = threadIdx.x;
  const int64_t bh = blockIdx.y, tile = blockIdx.x;
  int running = 0;
  for (int64_t c0 = 0; c0 < nlist; c0 += 256) {
    const int64_t c = c0 + tid;
    int tot = 0, bef = 0;
    if (c < nlist) {
      const int32_t* col = tcount + bh * ntiles * nlist + c;
#pragma unroll 8
      for (int64_t t = 0; t < ntiles; ++t) {
        const int x = col[t * nlist];
        tot += x;
        bef += t < tile ? x : 0;
      }
    }
    int all;
    const int ex = ivf_block_scan(tot, ws, &all);
    if (c < nlist) {
      base[c] = running + ex + bef;
      offl[c] = running + ex;
      cntl[c] = tot;
      if (tile == 0) {
        count[bh * nlist + c] = tot;
        off[bh * (nlist + 1) + c] = running + ex;
      }
    }
    running += all;
  }
  if (tile == 0 && tid == 0) off[bh * (nlist + 1) + nlist] = running;
  __syncthreads();
  const int64_t j = tile * kTile + tid;
  if (j < nb) {
    const int a = assign[bh * nb + j];
    const int pos = base[a] + rank[bh * nb + j];
    ids[bh * nb + pos] = (int32_t)j;
    if (muL != nullptr) {
      const float* src = mu + (bh * nb + j) * d;
      float* dst = muL + bh * nb * d + d * (int64_t)offl[a] + (pos - offl[a]);
      for (int64_t t = 0; t < d; ++t) dst[t * cntl[a]] = src[t];
    }
  }
}

// centT (BH, d, nlist) = the centroids transposed.
__global__ __launch_bounds__(64) void ivf_transpose_cent_kernel(const float* __restrict__ cent,
                                                                 int64_t d, int64_t nlist,
                                                                 float* __restrict__ centT) {
  const int64_t bh = blockIdx.y, c = blockIdx.x;
  for (int64_t t = threadIdx.x; t < d; t += 64)
    centT[(bh * d + t) * nlist + c] = cent[(bh * nlist + c) * d + t];
}

// Centroid c <- normalised sum of its members (fp64, ascending member order); unchanged when it
// has no members or their sum is zero. Lane l owns dimensions l + 64 u, u < NU (d <= 64 NU);
// every load is unconditional (clamped to a valid address) so a batch of them is in flight
// before the in-order adds.
template <int NU>
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

struct IvfRouteArgs {
  const float* centT;
  const float* muL;
  const int32_t* count;
  const int32_t* off;
  const int32_t* ids;
  const float* qb;
  int64_t nb, d, nlist, nprobe, search_k, top_c, local, W, G;
  int32_t* kv_num;
  int32_t* kv_idx;
};

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

// One workgroup per (query block i, query head bh); query head bh searches index head bh / G.
__global__ __launch_bounds__(256) void ivf_route_kernel(IvfRouteArgs a) {
  __shared__ unsigned long long buf[kIvfCap];
  __shared__ int lst[kIvfCap];         // probed lists, then the selected blocks and their union
  __shared__ int aux[kIvfCap + 1];     // member prefix of the probed lists, then the sorted union
  __shared__ __align__(16) float qs[kIvfMaxD];
  __shared__ unsigned int hist[256];
  __shared__ unsigned int shv[3];
  __shared__ int ws[4];
  const int tid = threadIdx.x;
  const int64_t i = blockIdx.x, bh = blockIdx.y, bk = bh / a.G;
  const int64_t nb = a.nb, d = a.d, nlist = a.nlist;
  for (int64_t t = tid; t < d; t += 256) qs[t] = a.qb[(bh * nb + i) * d + t];
  __syncthreads();

  // coarse search: the nprobe centroids of largest <qb_i, c>
  const float* cT = a.centT + bk * d * nlist;
  for (int64_t c = tid; c < nlist; c += 256) buf[c] = ivf_key(dot_strided(qs, cT + c, nlist, d), c);
  __syncthreads();
  unsigned long long T = 0ull;
  if (a.nprobe < nlist) T = block_kth_largest(buf, (int)nlist, (int)a.nprobe, hist, shv);
  int nprobed = 0;
  {
    int running = 0;
    for (int64_t c0 = 0; c0 < nlist; c0 += 256) {
      const int64_t c = c0 + tid;
      const bool take = c < nlist && buf[c] >= T;
      int tot;
      const int ex = ivf_block_scan(take ? 1 : 0, ws, &tot);
      if (take) lst[running + ex] = (int)c;
      running += tot;
    }
    nprobed = running;
  }
  __syncthreads();
  // member prefix over the probed lists
  const int32_t* cnt = a.count + bk * nlist;
  const int32_t* off = a.off + bk * (nlist + 1);
  const int32_t* ids = a.ids + bk * nb;
  {
    int running = 0;
    for (int p0 = 0; p0 < nprobed; p0 += 256) {
      const int p = p0 + tid;
      const int sz = p < nprobed ? cnt[lst[p]] : 0;
      int tot;
      const int ex = ivf_block_scan(sz, ws, &tot);
      if (p < nprobed) aux[p] = running + ex;
      running += tot;
    }
    if (tid == 0) aux[nprobed] = running;
  }
  __syncthreads();
  const int64_t M = aux[nprobed];

  // fine search: stream the members through buf, keeping the search_k largest keys
  const float* mL = a.muL + bk * nb * d;
  int nk = 0;
  for (int64_t m0 = 0; m0 < M;) {
    const int room = kIvfCap - nk;
    const int batch = (int)(M - m0 < room ? M - m0 : room);
    for (int e = tid; e < batch; e += 256) {
      const int64_t m = m0 + e;
      int lo = 0, hi = nprobed - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (aux[mid] <= m) lo = mid;
        else hi = mid - 1;
      }
      const int p = lst[lo];
      const int64_t k = m - aux[lo], L = cnt[p];
      const int64_t j = ids[off[p] + k];
      const float* col = mL + d * (int64_t)off[p] + k;  // member k of list p, transposed
      buf[nk + e] = ivf_key(dot_strided(qs, col, L, d), j);
    }
    __syncthreads();
    const int tot = nk + batch;
    if (tot > a.search_k) {
      const unsigned long long Ts = block_kth_largest(buf, tot, (int)a.search_k, hist, shv);
      nk = block_compact<unsigned long long>(buf, tot, buf, ws,
                                             [Ts](unsigned long long k) { return k >= Ts; });
    } else {
      nk = tot;
    }
    m0 += batch;
  }

  // the first top_c (by score) of the causal hits
  const int ncausal = block_compact<unsigned long long>(
      buf, nk, buf, ws, [i](unsigned long long k) { return ivf_key_index(k) <= i; });
  const int K2 = (int)(a.top_c < ncausal ? a.top_c : ncausal);
  int nsel = 0;
  if (K2 > 0) {
    const unsigned long long T2 =
        K2 < ncausal ? block_kth_largest(buf, ncausal, K2, hist, shv) : 0ull;
    int running = 0;
    for (int e0 = 0; e0 < ncausal; e0 += 256) {
      const int e = e0 + tid;
      const bool take = e < ncausal && buf[e] >= T2;
      int tot;
      const int ex = ivf_block_scan(take ? 1 : 0, ws, &tot);
      if (take) lst[running + ex] = (int)ivf_key_index(buf[e]);
      running += tot;
    }
    nsel = running;
  }
  __syncthreads();

  // OR the own block and `local` predecessors (those not already selected)
  const int64_t nwin = (a.local < i ? a.local : i) + 1;
  int nu = nsel;
  for (int64_t w0 = 0; w0 < nwin; w0 += 256) {
    const int64_t w = w0 + tid;
    bool take = false;
    int jw = 0;
    if (w < nwin) {
      jw = (int)(i - w);
      take = true;
      for (int e = 0; e < nsel; ++e)
        if (lst[e] == jw) { take = false; break; }
    }
    int tot;
    const int ex = ivf_block_scan(take ? 1 : 0, ws, &tot);
    if (take) lst[nu + ex] = jw;
    nu += tot;
  }
  __syncthreads();

  // ascending order (the entries are distinct): the rank of each is its slot
  for (int e = tid; e < nu; e += 256) {
    const int v = lst[e];
    int r = 0;
    for (int f = 0; f < nu; ++f) r += lst[f] < v;
    aux[r] = v;
  }
  __syncthreads();
  if (tid == 0) a.kv_num[bh * nb + i] = nu;
  int32_t* out = a.kv_idx + (bh * nb + i) * a.W;
  for (int64_t r = tid; r < a.W; r += 256) out[r] = r < nu ? aux[r] : 0;
}

}  // namespace
}  // namespace ssa

using ssa::IvfLayout;

extern "C" size_t ssa_ivf_index_size(int64_t BH, int64_t nb, int64_t nlist, int64_t d) {
  if (BH <= 0 || nb <= 0 || nlist <= 0 || d <= 0) return 0;
  return ssa::ivf_layout(BH, nb, nlist, d).total;
}

namespace {

int check_ivf_shape(const char* fn, const float* rows, int64_t BH, int64_t nb, int64_t d,
                    int64_t nlist) {
  SSA_REQUIRE(rows != nullptr && ssa::aligned16(rows), SSA_ERR_INVALID,
              "%s: mu / qb must be a 16-byte aligned device pointer", fn);
  SSA_REQUIRE(BH > 0 && BH <= 65535, SSA_ERR_INVALID, "%s: BH=%lld must be in [1, 65535]", fn,
              (long long)BH);
  SSA_REQUIRE(nb > 0 && nb < (int64_t(1) << 31), SSA_ERR_INVALID, "%s: bad nb=%lld", fn,
              (long long)nb);
  SSA_REQUIRE(d > 0 && d % 32 == 0 && d <= ssa::kIvfMaxD, SSA_ERR_UNSUPPORTED,
              "%s: d=%lld must be a multiple of 32 and at most %d", fn, (long long)d,
              ssa::kIvfMaxD);
  SSA_REQUIRE(nlist > 0 && nlist <= nb && nlist <= ssa::kIvfCap, SSA_ERR_UNSUPPORTED,
              "%s: nlist=%lld must be in [1, min(nb, %d)]", fn, (long long)nlist, ssa::kIvfCap);
  return SSA_OK;
}

}  // namespace

extern "C" int ssa_ivf_build(const float* mu, int64_t BH, int64_t nb, int64_t d, int64_t nlist,
                             int64_t niter, void* index, size_t index_bytes,
                             ssa_stream_t stream) {
  SSA_TRY(check_ivf_shape("ivf_build", mu, BH, nb, d, nlist));
  SSA_REQUIRE(niter >= 0, SSA_ERR_INVALID, "ivf_build: niter must be >= 0");
  const IvfLayout L = ssa::ivf_layout(BH, nb, nlist, d);
  SSA_REQUIRE(index != nullptr && (reinterpret_cast<uintptr_t>(index) & 255u) == 0,
              SSA_ERR_INVALID, "ivf_build: index must be a 256-byte aligned device pointer");
  SSA_REQUIRE(index_bytes >= L.total, SSA_ERR_WORKSPACE,
              "ivf_build: index holds %zu bytes, needs %zu", index_bytes, L.total);
  char* base = static_cast<char*>(index);
  float* cent = reinterpret_cast<float*>(base + L.cent);
  int32_t* count = reinterpret_cast<int32_t*>(base + L.count);
  int32_t* off = reinterpret_cast<int32_t*>(base + L.off);
  int32_t* ids = reinterpret_cast<int32_t*>(base + L.ids);
  int32_t* assign = reinterpret_cast<int32_t*>(base + L.assign);
  int32_t* rank = reinterpret_cast<int32_t*>(base + L.rank);
  int32_t* tcount = reinterpret_cast<int32_t*>(base + L.tcount);
  unsigned long long* pbest = reinterpret_cast<unsigned long long*>(base + L.pbest);
  float* centT = reinterpret_cast<float*>(base + L.centT);
  float* muL = reinterpret_cast<float*>(base + L.muL);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 gc((unsigned)nlist, (unsigned)BH), gt((unsigned)L.ntiles, (unsigned)BH);
  const dim3 gs((unsigned)L.stiles, (unsigned)BH, (unsigned)L.groups);
  ssa::ivf_init_kernel<<<gc, 64, 0, s>>>(mu, nb, d, nlist, cent);
  SSA_TRY(ssa::launch_status("ivf_init_kernel"));
  for (int64_t it = 0; it <= niter; ++it) {
    const bool last = it == niter;  // the last assignment only fills the lists
    ssa::ivf_score_kernel<<<gs, ssa::kScoreTile, ssa::kAssignC * d * sizeof(float), s>>>(
        mu, cent, nb, d, nlist, L.per_group, pbest);
    SSA_TRY(ssa::launch_status("ivf_score_kernel"));
    ssa::ivf_rank_kernel<<<gt, ssa::kTile, 0, s>>>(pbest, nb, nlist, L.ntiles, L.groups, assign,
                                                    rank, tcount);
    SSA_TRY(ssa::launch_status("ivf_rank_kernel"));
    ssa::ivf_scatter_kernel<<<gt, 256, 0, s>>>(assign, rank, tcount, nb, nlist, L.ntiles, count,
                                               off, ids, mu, d, last ? muL : nullptr);
    SSA_TRY(ssa::launch_status("ivf_scatter_kernel"));
    if (last) break;
    switch ((d + 63) / 64) {
      case 1: ssa::ivf_update_kernel<1><<<gc, 64, 0, s>>>(mu, count, off, ids, nb, d, nlist, cent); break;
      case 2: ssa::ivf_update_kernel<2><<<gc, 64, 0, s>>>(mu, count, off, ids, nb, d, nlist, cent); break;
      case 3: ssa::ivf_update_kernel<3><<<gc, 64, 0, s>>>(mu, count, off, ids, nb, d, nlist, cent); break;
      default: ssa::ivf_update_kernel<4><<<gc, 64, 0, s>>>(mu, count, off, ids, nb, d, nlist, cent); break;
    }
    SSA_TRY(ssa::launch_status("ivf_update_kernel"));
  }
  ssa::ivf_transpose_cent_kernel<<<gc, 64, 0, s>>>(cent, d, nlist, centT);
  return ssa::launch_status("ivf_transpose_cent_kernel");
}

extern "C" int ssa_ivf_route(const void* index, const float* qb, int64_t BH, int64_t G,
                             int64_t nb, int64_t d, int64_t nlist, int64_t nprobe,
                             int64_t search_k, int64_t top_c, int64_t local, int32_t* kv_num,
                             int32_t* kv_idx, int64_t W, ssa_stream_t stream) {
  SSA_TRY(check_ivf_shape("ivf_route", qb, BH, nb, d, nlist));
  SSA_REQUIRE(G >= 1 && BH * G <= 65535, SSA_ERR_INVALID,
              "ivf_route: G=%lld must be >= 1 with BH * G <= 65535", (long long)G);
  SSA_REQUIRE(index != nullptr && (reinterpret_cast<uintptr_t>(index) & 255u) == 0,
              SSA_ERR_INVALID, "ivf_route: index must be a 256-byte aligned device pointer");
  SSA_REQUIRE(kv_num != nullptr && kv_idx != nullptr, SSA_ERR_INVALID,
              "ivf_route: kv_num / kv_idx is NULL");
  SSA_REQUIRE(nprobe > 0 && search_k > 0 && top_c >= 0 && local >= 0, SSA_ERR_INVALID,
              "ivf_route: need nprobe > 0, search_k > 0, top_c >= 0, local >= 0");
  const int64_t np = nprobe < nlist ? nprobe : nlist;
  const int64_t sk = search_k < nb ? search_k : nb;
  SSA_REQUIRE(sk <= ssa::kIvfMaxSearch, SSA_ERR_UNSUPPORTED,
              "ivf_route: min(search_k, nb)=%lld exceeds %d", (long long)sk, ssa::kIvfMaxSearch);
  const int64_t keep = top_c < sk ? top_c : sk;
  const int64_t win = (local < nb - 1 ? local : nb - 1) + 1;
  SSA_REQUIRE(keep + win <= ssa::kIvfCap, SSA_ERR_UNSUPPORTED,
              "ivf_route: min(top_c, search_k) + min(local, nb-1) + 1 = %lld exceeds %d",
              (long long)(keep + win), ssa::kIvfCap);
  const int64_t wneed = top_c + local + 1 < nb ? top_c + local + 1 : nb;
  SSA_REQUIRE(W >= wneed, SSA_ERR_INVALID, "ivf_route: W=%lld < min(top_c + local + 1, nb)=%lld",
              (long long)W, (long long)wneed);
  const IvfLayout L = ssa::ivf_layout(BH, nb, nlist, d);
  const char* base = static_cast<const char*>(index);
  ssa::IvfRouteArgs a;
  a.centT = reinterpret_cast<const float*>(base + L.centT);
  a.muL = reinterpret_cast<const float*>(base + L.muL);
  a.count = reinterpret_cast<const int32_t*>(base + L.count);
  a.off = reinterpret_cast<const int32_t*>(base + L.off);
  a.ids = reinterpret_cast<const int32_t*>(base + L.ids);
  a.qb = qb;
  a.nb = nb;
  a.d = d;
  a.nlist = nlist;
  a.nprobe = np;
  a.search_k = sk;
  a.top_c = top_c;
  a.local = local;
  a.W = W;
  a.G = G;
  a.kv_num = kv_num;
  a.kv_idx = kv_idx;
  ssa::ivf_route_kernel<<<dim3((unsigned)nb, (unsigned)(BH * G)), 256, 0,
                          static_cast<hipStream_t>(stream)>>>(a);
  return ssa::launch_status("ivf_route_kernel");
}
