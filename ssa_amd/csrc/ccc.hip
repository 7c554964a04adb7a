// Certified causal cascade (CCC): the streaming, chunked-causal sub-block selector of
// ssa/cascade_router.py:66-442 (CausalCascade, ccc_prefill) on the library's own kernels, with the
// faiss GpuIndexIVFFlat replaced by the inverted lists of ivf_parts.h.
//
// State (held by the caller, see ssa_amd/cascade_router.py): the routing-space sub-block means of
// every appended key (fp32, row-major), how many of them are committed, the outlier keys (fp32
// vectors, parent block, token position) and, once built, one index buffer (ssa_ccc_index_size).
//
// ssa_ccc_stage (append + _extract_outliers, :120-128,:214-231): means of `group` consecutive
//   rows, fp64 sums in row order rounded once; with quota > 0, every row's squared distance to its
//   group mean (fp64, dimension order) and the quota rows of largest distance (ties to the lower
//   row; each tile of 2048 rows keeps its own quota best first), copied out as outlier keys,
//   largest first.
// ssa_ccc_kmeans / ssa_ccc_index_build / ssa_ccc_index_add (_kmeans, _build_index, _commit,
//   _update_radii, :131-198): inner-product Lloyd rounds (each mean joins the centroid of largest
//   inner product, ties to the lower centroid; a centroid with members becomes their mean), the
//   lists of the last assignment with their members in ascending order, and per-cell radii
//   max ||x - c|| (exact at a build, raised by every add).
// ssa_ccc_route (route, _search_committed, _search_staged, _select_topc, _outlier_parents, _pack,
//   _certify, :233-403): one workgroup per query block, escalation rounds inside the kernel.
//
// Every inner product accumulates in fp64 in dimension order and rounds once to fp32, and every
// ranking breaks ties by the lower index, so each step is reproducible on the CPU.
#include "ivf_parts.h"

namespace ssa {
namespace {

// Scalar element i of a row-major array of dtype DT, as fp32 (exact for every DT).
template <int DT>
__device__ inline float ld_elem(const void* p, int64_t i) {
  if constexpr (DT == SSA_F32) {
    return static_cast<const float*>(p)[i];
  } else if constexpr (DT == SSA_F16) {
    return (float)static_cast<const _Float16*>(p)[i];
  } else {
    return __uint_as_float((unsigned int)static_cast<const unsigned short*>(p)[i] << 16);
  }
}

// The fp32 score a score_key came from (score_key is one-to-one on non-NaN values but -0).
__device__ inline float key_score(unsigned long long key) {
  const unsigned int k = (unsigned int)(key >> 32);
  const unsigned int u = (k & 0x80000000u) ? (k ^ 0x80000000u) : ~k;
  return __uint_as_float(u);
}

// <q, row> for a row-major fp32 row (16-byte aligned, d a multiple of 32): the same fp64 chain in
// dimension order as dot_strided, the row read with 16-byte loads.
__device__ inline float dot_row(const float* q, const float* row, int64_t d) {
  double acc = 0.0;
  for (int64_t t0 = 0; t0 < d; t0 += 32) {
    float4 x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = *reinterpret_cast<const float4*>(row + t0 + 4 * u);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float4 qq = *reinterpret_cast<const float4*>(q + t0 + 4 * u);
      acc = fma((double)qq.x, (double)x[u].x, acc);
      acc = fma((double)qq.y, (double)x[u].y, acc);
      acc = fma((double)qq.z, (double)x[u].z, acc);
      acc = fma((double)qq.w, (double)x[u].w, acc);
    }
  }
  return (float)acc;
}

// Smallest of v[0..n) (LDS) over a 256-thread workgroup; slot holds 4 values.
__device__ inline unsigned long long block_min_key(const unsigned long long* v, int n,
                                                   unsigned long long* slot) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  unsigned long long m = ~0ull;
  for (int e = tid; e < n; e += 256) m = v[e] < m ? v[e] : m;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const unsigned long long y = __shfl_xor(m, o);
    m = y < m ? y : m;
  }
  if (lane == 0) slot[w] = m;
  __syncthreads();
  unsigned long long r = slot[0];
#pragma unroll
  for (int k = 1; k < 4; ++k) r = slot[k] < r ? slot[k] : r;
  __syncthreads();
  return r;
}

// Largest of x over a 256-thread workgroup; slot holds 4 values.
__device__ inline float block_max_f32(float x, float* slot) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  if (lane == 0) slot[w] = x;
  __syncthreads();
  const float r = fmaxf(fmaxf(slot[0], slot[1]), fmaxf(slot[2], slot[3]));
  __syncthreads();
  return r;
}

// Streams M candidates through buf (LDS, kIvfCap keys), keeping the K largest (K <= kIvfMaxSearch,
// keys unique); keyof(m) is candidate m's key, or 0 to skip it. Once K keys are kept, a candidate
// below the threshold that kept them (K keys above it already) cannot enter the K largest and is
// dropped on arrival, so later batches fill the buffer slowly. buf[0..nk0) may hold up to K keys
// of earlier candidates (nonzero, visible to the workgroup), ranked with the M new ones. Returns
// how many are kept (in buf[0..), any order). 256 threads.
template <typename F>
__device__ int stream_top(unsigned long long* buf, int64_t M, int K, F keyof, unsigned int* hist,
                          unsigned int* shv, int* ws, int nk0 = 0) {
  int nk = nk0;
  unsigned long long floor_key = 1ull;  // every real key is at least 1
  for (int64_t m0 = 0; m0 < M;) {
    const int room = kIvfCap - nk;
    const int batch = (int)(M - m0 < room ? M - m0 : room);
    for (int e = threadIdx.x; e < batch; e += 512) {  // two candidates per thread per pass
      const bool two = e + 256 < batch;
      const unsigned long long k0 = keyof(m0 + e);
      const unsigned long long k1 = two ? keyof(m0 + e + 256) : 0ull;
      buf[nk + e] = k0 >= floor_key ? k0 : 0ull;
      if (two) buf[nk + e + 256] = k1 >= floor_key ? k1 : 0ull;
    }
    __syncthreads();
    int tot = block_compact<unsigned long long>(buf, nk + batch, buf, ws,
                                                [](unsigned long long k) { return k != 0ull; });
    if (tot > K) {
      const unsigned long long T = block_kth_largest(buf, tot, K, hist, shv);
      tot = block_compact<unsigned long long>(buf, tot, buf, ws,
                                              [T](unsigned long long k) { return k >= T; });
      floor_key = T;
    }
    nk = tot;
    m0 += batch;
  }
  return nk;
}

// ---- stage: group means, distances, outliers ----------------------------------------------------

// One wave per group of g rows: means[grp] = fl32(sum / g) (fp64 sums in row order); with RESID,
// keys[row] = ivf_key(fl32(||x_row - mean||^2), row) (fp64, dimension order).
template <int DT, bool RESID>
__global__ __launch_bounds__(64) void ccc_means_kernel(const void* __restrict__ x, int64_t rs,
                                                        int64_t d, int64_t g,
                                                        float* __restrict__ means,
                                                        unsigned long long* __restrict__ keys) {
  __shared__ float mu[kIvfMaxD];
  const int64_t grp = blockIdx.x, r0 = grp * g;
  const int lane = threadIdx.x;
  for (int64_t t = lane; t < d; t += 64) {
    double acc = 0.0;
    const int64_t base = r0 * rs + t;
    int64_t r = 0;
    for (; r + 8 <= g; r += 8) {  // 8 loads in flight before the in-order adds
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = ld_elem<DT>(x, base + (r + u) * rs);
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = __dadd_rn(acc, (double)v[u]);
    }
    for (; r < g; ++r) acc = __dadd_rn(acc, (double)ld_elem<DT>(x, base + r * rs));
    const float m = (float)(acc / (double)g);
    means[grp * d + t] = m;
    if constexpr (RESID) mu[t] = m;
  }
  if constexpr (RESID) {
    __syncthreads();
    for (int64_t r = lane; r < g; r += 64) {
      const int64_t row = r0 + r;
      double ss = 0.0;
      for (int64_t t = 0; t < d; ++t) {
        const double df = (double)ld_elem<DT>(x, row * rs + t) - (double)mu[t];
        ss = __dadd_rn(ss, __dmul_rn(df, df));
      }
      keys[row] = ivf_key((float)ss, row);
    }
  }
}

// One workgroup per tile of kIvfCap row keys: the tile's K largest (every key of a tile holding
// at most K), written to cand[tile * K ..] and padded with 0 (no key). The K largest of all rows
// are among them.
__global__ __launch_bounds__(256) void ccc_tile_top_kernel(
    const unsigned long long* __restrict__ keys, int64_t m, int K,
    unsigned long long* __restrict__ cand) {
  __shared__ unsigned long long buf[kIvfCap];
  __shared__ unsigned int hist[256];
  __shared__ unsigned int shv[3];
  __shared__ int ws[4];
  const int64_t t0 = (int64_t)blockIdx.x * kIvfCap;
  const int n = (int)(m - t0 < kIvfCap ? m - t0 : kIvfCap);
  for (int e = threadIdx.x; e < n; e += 256) buf[e] = keys[t0 + e];
  __syncthreads();
  int keep = n;
  if (n > K) {
    const unsigned long long T = block_kth_largest(buf, n, K, hist, shv);
    keep = block_compact<unsigned long long>(buf, n, buf, ws,
                                             [T](unsigned long long k) { return k >= T; });
  }
  unsigned long long* out = cand + (int64_t)blockIdx.x * K;
  for (int e = threadIdx.x; e < K; e += 256) out[e] = e < keep ? buf[e] : 0ull;
}

// One workgroup: the K largest of the m candidate keys (at least K of them real, the rest 0),
// largest first, copied out as outlier keys (fp32 vector of the key's row, parent block
// (base + row) / block, position base + row).
template <int DT>
__global__ __launch_bounds__(256) void ccc_outlier_kernel(
    const unsigned long long* __restrict__ keys, int64_t m, int K, const void* __restrict__ x,
    int64_t rs, int64_t d, int64_t base, int64_t block, float* __restrict__ ovec,
    int64_t* __restrict__ opar, int64_t* __restrict__ opos) {
  __shared__ unsigned long long sel[kIvfCap];
  __shared__ unsigned long long srt[kIvfCap];
  __shared__ unsigned int hist[256];
  __shared__ unsigned int shv[3];
  __shared__ int cnt;
  const int tid = threadIdx.x;
  const unsigned long long T = (int64_t)K < m ? block_kth_largest(keys, (int)m, K, hist, shv) : 0ull;
  if (tid == 0) cnt = 0;
  __syncthreads();
  for (int64_t e = tid; e < m; e += 256) {
    const unsigned long long k = keys[e];
    if (k >= T) sel[atomicAdd(&cnt, 1)] = k;  // exactly K keys (unique) pass
  }
  __syncthreads();
  for (int e = tid; e < K; e += 256) {
    const unsigned long long v = sel[e];
    int r = 0;
    for (int f = 0; f < K; ++f) r += sel[f] > v;
    srt[r] = v;
  }
  __syncthreads();
  for (int64_t e = tid; e < (int64_t)K * d; e += 256) {
    const int64_t r = e / d, t = e - r * d;
    ovec[e] = ld_elem<DT>(x, ivf_key_index(srt[r]) * rs + t);
  }
  for (int r = tid; r < K; r += 256) {
    const int64_t row = ivf_key_index(srt[r]);
    opar[r] = (base + row) / block;
    opos[r] = base + row;
  }
}

// ---- index: Lloyd rounds, lists, radii ------------------------------------------------------------

// Byte offsets of the index regions: the centroids (nlist, d), transposed (d, nlist), the radii
// (nlist), the assignment of every committed mean, list sizes, list capacity offsets (nlist + 1),
// list members (ascending) and the members' means, and the scratch of the list build (overflow
// flag, new members per list, ranks, per-tile counts, assignment keys).
//
// List p owns member slots off[p] .. off[p + 1] - 1 (a multiple of 64 of them, off[p] a multiple of
// 64): its capacity, set at its last full layout to roundup64(2 size) + 64, so that incremental
// adds write only the new members. Member k's id is ids[off[p] + k]; its mean sits in tile
// (off[p] + k) / 64 of 64 members, each tile stored transposed (d, 64): element t of member k at
// muL[(off[p] + k - k % 64) d + 64 t + k % 64], 256-byte aligned runs of 64 members per dimension.
struct CccLayout {
  size_t cent, centT, rc, assign, count, off, ids, muL, flag, cnew, rank, tcount, pbest, total;
  int64_t pcap;  // assignment keys the pbest region holds
  int64_t mcap;  // member slots: capacities summing to at most 2 n_cap + 128 nlist
};

__host__ __device__ inline int32_t ccc_list_cap(int32_t size) {
  return ((2 * size + 63) & ~63) + 64;
}

CccLayout ccc_layout(int64_t n_cap, int64_t nlist, int64_t d) {
  CccLayout L;
  const int64_t ntiles = (n_cap + kTile - 1) / kTile;
  L.pcap = n_cap > 262144 ? n_cap : 262144;
  size_t o = 0;
  L.cent = o;   o += r256(size_t(nlist) * d * 4);
  L.centT = o;  o += r256(size_t(nlist) * d * 4);
  L.mcap = 2 * n_cap + 128 * nlist;
  L.rc = o;     o += r256(size_t(nlist) * 4);
  L.assign = o; o += r256(size_t(n_cap) * 4);
  L.count = o;  o += r256(size_t(nlist) * 4);
  L.off = o;    o += r256(size_t(nlist + 1) * 4);
  L.ids = o;    o += r256(size_t(L.mcap) * 4);
  L.muL = o;    o += r256(size_t(L.mcap) * d * 4);
  L.flag = o;   o += 256;
  L.cnew = o;   o += r256(size_t(nlist) * 4);
  L.rank = o;   o += r256(size_t(n_cap) * 4);
  L.tcount = o; o += r256(size_t(ntiles) * nlist * 4);
  L.pbest = o;  o += r256(size_t(L.pcap) * 8);
  L.total = o;
  return L;
}

// Centroid c starts at mean x[c * n / nlist] (cold start).
__global__ __launch_bounds__(64) void ccc_init_kernel(const float* __restrict__ x, int64_t n,
                                                       int64_t d, int64_t nlist,
                                                       float* __restrict__ cent) {
  const int64_t c = blockIdx.x, j = c * n / nlist;
  for (int64_t t = threadIdx.x; t < d; t += 64) cent[c * d + t] = x[j * d + t];
}

__global__ __launch_bounds__(256) void ccc_fill_kernel(float* __restrict__ p, int64_t n, float v) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e < n) p[e] = v;
}

__global__ __launch_bounds__(64) void ccc_copy_kernel(const float* __restrict__ src,
                                                       float* __restrict__ dst, int64_t n) {
  for (int64_t e = (int64_t)blockIdx.x * 64 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 64)
    dst[e] = src[e];
}

// Rows x[0..m) (mean base + j): assign[base + j] = the best of the groups' centroids; with rc,
// rc[c] = max(rc[c], fl32(||x_j - cent[c]||)) for that centroid c (fp64, dimension order).
__global__ __launch_bounds__(256) void ccc_assign_kernel(
    const unsigned long long* __restrict__ pbest, int64_t groups, int64_t m, int64_t base,
    const float* __restrict__ x, const float* __restrict__ cent, int64_t d,
    int32_t* __restrict__ assign, float* __restrict__ rc) {
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= m) return;
  unsigned long long best = 0ull;
  for (int64_t g = 0; g < groups; ++g) {
    const unsigned long long k = pbest[g * m + j];
    best = k > best ? k : best;
  }
  const int c = (int)ivf_key_index(best);
  assign[base + j] = c;
  if (rc != nullptr) {
    const float* xr = x + j * d;
    const float* cr = cent + (int64_t)c * d;
    double ss = 0.0;
    for (int64_t t = 0; t < d; ++t) {
      const double df = (double)xr[t] - (double)cr[t];
      ss = __dadd_rn(ss, __dmul_rn(df, df));
    }
    const float r = (float)sqrt(ss);  // >= 0: its bits order like its value
    atomicMax(reinterpret_cast<unsigned int*>(rc) + c, __float_as_uint(r));
  }
}

// One workgroup per tile of 256 means: rank = position among the tile's members of its centroid;
// the tile's member count of every centroid goes to its tcount row (0 for absent ones).
// With gate set, nothing runs unless *gate != 0.
__global__ __launch_bounds__(256) void ccc_rank_kernel(const int32_t* __restrict__ assign,
                                                        int64_t n, int64_t nlist,
                                                        int32_t* __restrict__ rank,
                                                        int32_t* __restrict__ tcount,
                                                        const int32_t* __restrict__ gate) {
  __shared__ int sa[kTile];
  if (gate != nullptr && *gate == 0) return;
  const int tid = threadIdx.x;
  const int64_t tile = blockIdx.x, j = tile * kTile + tid;
  const bool live = j < n;
  int32_t* trow = tcount + tile * nlist;
  for (int64_t c = tid; c < nlist; c += kTile) trow[c] = 0;
  const int a = live ? assign[j] : -1;
  sa[tid] = a;
  __syncthreads();  // also orders the zeroing of trow before the counts below
  if (live) {
    int r = 0;
    bool last = true;
    for (int t = 0; t < kTile; ++t) {
      const int y = sa[t];
      if (t < tid) r += (y == a);
      else if (t > tid && y == a) last = false;
    }
    rank[j] = r;
    if (last) trow[a] = r + 1;
  }
}

// Assignment of the m means x[0..m) (base = the index of x[0]) to their best centroid: the
// scoring launch splits the centroids into groups so that it holds about 2048 waves.
int ccc_assign_rows(const float* x, int64_t m, int64_t base, int64_t d, const float* cent,
                    int64_t nlist, unsigned long long* pbest, int64_t pcap, int32_t* assign,
                    float* rc, hipStream_t s) {
  if (m <= 0) return SSA_OK;
  const int64_t stiles = (m + 2 * kScoreTile - 1) / (2 * kScoreTile);
  const int64_t gmax = (nlist + kAssignC - 1) / kAssignC;
  int64_t g = (2048 + stiles - 1) / stiles;
  g = g > gmax ? gmax : g;
  g = g > pcap / m ? pcap / m : g;
  g = g < 1 ? 1 : g;
  const int64_t per_group = (nlist + g - 1) / g;
  const int64_t groups = (nlist + per_group - 1) / per_group;
  ivf_score_kernel<<<dim3((unsigned)stiles, 1, (unsigned)groups), kScoreTile,
                     kAssignC * d * sizeof(double), s>>>(x, cent, m, d, nlist, per_group, pbest);
  SSA_TRY(launch_status("ivf_score_kernel"));
  ccc_assign_kernel<<<(unsigned)((m + 255) / 256), 256, 0, s>>>(pbest, groups, m, base, x, cent, d,
                                                                 assign, rc);
  return launch_status("ccc_assign_kernel");
}

// One workgroup: off[c] = the capacity slots (ccc_list_cap of each size) of the lists before c,
// off[nlist] = all of them. With gate set, nothing runs unless *gate != 0.
__global__ __launch_bounds__(256) void ccc_cap_offsets_kernel(const int32_t* __restrict__ count,
                                                               int64_t nlist,
                                                               int32_t* __restrict__ off,
                                                               const int32_t* __restrict__ gate) {
  __shared__ int ws[4];
  if (gate != nullptr && *gate == 0) return;
  int running = 0;
  for (int64_t c0 = 0; c0 < nlist; c0 += 256) {
    const int64_t c = c0 + threadIdx.x;
    const int v = c < nlist ? ccc_list_cap(count[c]) : 0;
    int tot;
    const int ex = ivf_block_scan(v, ws, &tot);
    if (c < nlist) off[c] = running + ex;
    running += tot;
  }
  if (threadIdx.x == 0) off[nlist] = running;
}

// One thread per mean j < m (id base + j, list a = assign[j]): it is member k = start[a] (0 without
// start) + tbase[(j / kTile) nlist + a] + rank[j] of list a, stored at slot off[a] + k: its id and,
// with muL set, its mean in the list's tiled storage. With gate set, runs only if
// (*gate != 0) == gate_on.
__global__ __launch_bounds__(256) void ccc_scatter_kernel(
    const int32_t* __restrict__ assign, const int32_t* __restrict__ rank,
    const int32_t* __restrict__ tbase, int64_t m, int64_t base, int64_t nlist,
    const int32_t* __restrict__ start, const int32_t* __restrict__ off, int32_t* __restrict__ ids,
    const float* __restrict__ x, int64_t d, float* __restrict__ muL,
    const int32_t* __restrict__ gate, int gate_on) {
  if (gate != nullptr && ((*gate != 0) != (gate_on != 0))) return;
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= m) return;
  const int a = assign[j];
  const int64_t k = (start != nullptr ? start[a] : 0) + tbase[(j / kTile) * nlist + a] + rank[j];
  const int64_t slot = off[a] + k;
  ids[slot] = (int32_t)(base + j);
  if (muL != nullptr) {
    float* dst = muL + (slot - (k & 63)) * d + (k & 63);
    const float* src = x + j * d;
    for (int64_t t = 0; t < d; ++t) dst[t * 64] = src[t];
  }
}

// One workgroup: *flag = 1 if some list's size plus its new members exceeds its capacity, else 0.
__global__ __launch_bounds__(256) void ccc_add_check_kernel(const int32_t* __restrict__ count,
                                                             const int32_t* __restrict__ cnew,
                                                             const int32_t* __restrict__ off,
                                                             int64_t nlist,
                                                             int32_t* __restrict__ flag) {
  __shared__ int any;
  if (threadIdx.x == 0) any = 0;
  __syncthreads();
  bool over = false;
  for (int64_t c = threadIdx.x; c < nlist; c += 256)
    over |= (int64_t)count[c] + cnew[c] > (int64_t)off[c + 1] - off[c];
  if (over) atomicOr(&any, 1);
  __syncthreads();
  if (threadIdx.x == 0) flag[0] = any;
}

// count[c] += cnew[c], unless *flag is set (the full layout recounts them).
__global__ __launch_bounds__(256) void ccc_add_count_kernel(int32_t* __restrict__ count,
                                                             const int32_t* __restrict__ cnew,
                                                             int64_t nlist,
                                                             const int32_t* __restrict__ flag) {
  if (*flag != 0) return;
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c < nlist) count[c] += cnew[c];
}

// Full layout of the lists of the means x[0..n) from their assignment in the index: sizes,
// capacity offsets, ascending members and (with_means) the members' means. With gate set, runs
// only if *gate != 0 (every kernel checks it on the device).
int ccc_lists(const float* x, int64_t n, int64_t d, int64_t nlist, const CccLayout& L, char* base,
              bool with_means, const int32_t* gate, hipStream_t s) {
  const int64_t ntiles = (n + kTile - 1) / kTile;
  int32_t* assign = reinterpret_cast<int32_t*>(base + L.assign);
  int32_t* rank = reinterpret_cast<int32_t*>(base + L.rank);
  int32_t* tcount = reinterpret_cast<int32_t*>(base + L.tcount);
  int32_t* count = reinterpret_cast<int32_t*>(base + L.count);
  int32_t* off = reinterpret_cast<int32_t*>(base + L.off);
  ccc_rank_kernel<<<(unsigned)ntiles, kTile, 0, s>>>(assign, n, nlist, rank, tcount, gate);
  SSA_TRY(launch_status("ccc_rank_kernel"));
  ivf_tile_prefix_kernel<<<dim3((unsigned)nlist, 1), 256, 0, s>>>(tcount, ntiles, nlist, count,
                                                                  gate);
  SSA_TRY(launch_status("ivf_tile_prefix_kernel"));
  ccc_cap_offsets_kernel<<<1, 256, 0, s>>>(count, nlist, off, gate);
  SSA_TRY(launch_status("ccc_cap_offsets_kernel"));
  ccc_scatter_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
      assign, rank, tcount, n, 0, nlist, nullptr, off, reinterpret_cast<int32_t*>(base + L.ids),
      x, d, with_means ? reinterpret_cast<float*>(base + L.muL) : nullptr, gate, 1);
  return launch_status("ccc_scatter_kernel");
}

// Incremental add of the means n_old..n-1 (already assigned) to lists laid out over x[0..n_old):
// each list's new members (ascending) go to the slots after its current ones, unless some list
// would exceed its capacity; then (decided on the device) the lists are laid out again in full.
int ccc_lists_add(const float* x, int64_t n_old, int64_t n, int64_t d, int64_t nlist,
                  const CccLayout& L, char* base, hipStream_t s) {
  const int64_t m = n - n_old, ntn = (m + kTile - 1) / kTile;
  const int32_t* assign = reinterpret_cast<const int32_t*>(base + L.assign) + n_old;
  int32_t* rank = reinterpret_cast<int32_t*>(base + L.rank);
  int32_t* tcount = reinterpret_cast<int32_t*>(base + L.tcount);
  int32_t* count = reinterpret_cast<int32_t*>(base + L.count);
  int32_t* off = reinterpret_cast<int32_t*>(base + L.off);
  int32_t* cnew = reinterpret_cast<int32_t*>(base + L.cnew);
  int32_t* flag = reinterpret_cast<int32_t*>(base + L.flag);
  ccc_rank_kernel<<<(unsigned)ntn, kTile, 0, s>>>(assign, m, nlist, rank, tcount, nullptr);
  SSA_TRY(launch_status("ccc_rank_kernel"));
  ivf_tile_prefix_kernel<<<dim3((unsigned)nlist, 1), 256, 0, s>>>(tcount, ntn, nlist, cnew,
                                                                  nullptr);
  SSA_TRY(launch_status("ivf_tile_prefix_kernel"));
  ccc_add_check_kernel<<<1, 256, 0, s>>>(count, cnew, off, nlist, flag);
  SSA_TRY(launch_status("ccc_add_check_kernel"));
  ccc_scatter_kernel<<<(unsigned)((m + 255) / 256), 256, 0, s>>>(
      assign, rank, tcount, m, n_old, nlist, count, off, reinterpret_cast<int32_t*>(base + L.ids),
      x + n_old * d, d, reinterpret_cast<float*>(base + L.muL), flag, 0);
  SSA_TRY(launch_status("ccc_scatter_kernel"));
  ccc_add_count_kernel<<<(unsigned)((nlist + 255) / 256), 256, 0, s>>>(count, cnew, nlist, flag);
  SSA_TRY(launch_status("ccc_add_count_kernel"));
  return ccc_lists(x, n, d, nlist, L, base, true, flag, s);
}

// ---- route ----------------------------------------------------------------------------------------

struct CccRouteArgs {
  const float* qr;
  int64_t nbq, qb_start, d;
  const float* means;
  int64_t committed, n_sub, spb;
  int has_index;
  const float* centT;
  const float* muL;
  const int32_t* count;
  const int32_t* off;
  const int32_t* ids;
  const float* rc;
  int64_t nlist;
  const float* ovec;
  const int64_t* opar;
  int64_t n_out;
  int64_t top_c, local, ocap, ks, sk0, nprobe0, esc, max_esc;
  int certify;
  float margin;
  int32_t* kv_num;
  int32_t* kv_idx;
  int64_t W;
  unsigned char* cert;
  int32_t* rounds;
  unsigned long long* carry;  // (nbq, kkeep) keys, or NULL: see ccc_route_kernel
  int64_t kkeep;
};

// One workgroup per query block i of the chunk (global block qblk = qb_start + i).
// Escalation rounds probe nested sets of lists (the nprobe cells of largest <q, c>, nprobe growing).
// With a carry, each round keeps the kkeep best committed keys of every list probed so far in
// carry row i (kkeep >= every round's search_k), and a later round streams only the lists it adds
// through stream_top seeded with them: the top search_k of (the kkeep best of the earlier lists)
// and (the new lists) is the top search_k of all of them. Each thread reads back only the carry
// entries it wrote. Without a carry every round scans all of its lists.
__global__ __launch_bounds__(256) void ccc_route_kernel(CccRouteArgs a) {
  __shared__ unsigned long long buf[kIvfCap];     // streamed keys, then the merged candidates
  __shared__ unsigned long long stg[kIvfMaxSearch];  // the staged top
  __shared__ int lst[kIvfCap];                    // probed lists, then the block union
  __shared__ int aux[kIvfCap + 1];                // member prefix of the probed lists, then sorted
  __shared__ __align__(16) float qs[kIvfMaxD];
  __shared__ float csv[kIvfCap];                  // <q, centroid> of every cell
  __shared__ unsigned int hist[256];
  __shared__ unsigned int shv[3];
  __shared__ int ws[4];
  __shared__ unsigned long long kslot[4];
  __shared__ float fslot[4];
  __shared__ int nuniq;
  const int tid = threadIdx.x;
  const int64_t i = blockIdx.x, qblk = a.qb_start + i, d = a.d;
  for (int64_t t = tid; t < d; t += 256) qs[t] = a.qr[i * d + t];
  __syncthreads();
  float qn;
  {
    if (tid == 0) {
      double s = 0.0;
      for (int64_t t = 0; t < d; ++t) s = __dadd_rn(s, __dmul_rn((double)qs[t], (double)qs[t]));
      fslot[0] = (float)sqrt(s);
    }
    __syncthreads();
    qn = fslot[0];
    __syncthreads();
  }
  const float* means = a.means;
  const int64_t spb = a.spb, committed = a.committed;

  // the staged sub-means (exhaustive, causally masked: parent strictly before the query block)
  const int64_t ns = a.n_sub - committed;
  const int ks = (int)(a.ks < ns ? a.ks : ns);
  int nst = 0;
  if (ks > 0) {
    nst = stream_top(
        buf, ns, ks,
        [&](int64_t m) -> unsigned long long {
          const int64_t j = committed + m;
          if (j / spb >= qblk) return 0ull;
          return ivf_key(dot_row(qs, means + j * d, d), j);
        },
        hist, shv, ws);
    for (int e = tid; e < nst; e += 256) stg[e] = buf[e];
    __syncthreads();
  }
  const int64_t nlist = a.nlist;
  if (a.has_index) {
    for (int64_t c = tid; c < nlist; c += 256) csv[c] = dot_strided(qs, a.centT + c, nlist, d);
    __syncthreads();
  }

  int64_t nprobe = a.nprobe0, sk = a.sk0;
  unsigned long long* carry = a.carry != nullptr ? a.carry + i * a.kkeep : nullptr;
  int ncarry = 0;
  int64_t mtot = 0;              // members of every list probed so far
  unsigned long long Tprev = 0;  // the previous round's Tc
  for (int rnd = 0;; ++rnd) {
    // committed candidates: exhaustive (flat regime) or the probed lists (index)
    const int64_t kc = sk < committed ? sk : committed;
    int ncm = 0, nprobed = 0;
    float dlast = -INFINITY;
    unsigned long long Tc = 0ull;
    if (committed > 0 && kc > 0) {
      if (!a.has_index) {
        ncm = stream_top(
            buf, committed, (int)kc,
            [&](int64_t m) -> unsigned long long {
              return ivf_key(dot_row(qs, means + m * d, d), m);
            },
            hist, shv, ws);
      } else {
        for (int64_t c = tid; c < nlist; c += 256) buf[c] = ivf_key(csv[c], c);
        __syncthreads();
        if (nprobe < nlist) Tc = block_kth_largest(buf, (int)nlist, (int)nprobe, hist, shv);
        {
          int running = 0;
          for (int64_t c0 = 0; c0 < nlist; c0 += 256) {
            const int64_t c = c0 + tid;
            const bool take = c < nlist && buf[c] >= Tc &&
                              (carry == nullptr || rnd == 0 || buf[c] < Tprev);
            int tot;
            const int ex = ivf_block_scan(take ? 1 : 0, ws, &tot);
            if (take) lst[running + ex] = (int)c;
            running += tot;
          }
          nprobed = running;
        }
        __syncthreads();  // the probed lists (written by any wave) before their sizes are read
        {
          // member prefix of the probed lists in aux; lst[p] becomes list p's member offset (only
          // thread tid reads and rewrites entry p; the scan's barriers order it before other reads)
          int running = 0;
          for (int p0 = 0; p0 < nprobed; p0 += 256) {
            const int p = p0 + tid;
            const int cell = p < nprobed ? lst[p] : 0;
            const int sz = p < nprobed ? a.count[cell] : 0;
            const int of = p < nprobed ? a.off[cell] : 0;
            int tot;
            const int ex = ivf_block_scan(sz, ws, &tot);
            if (p < nprobed) {
              aux[p] = running + ex;
              lst[p] = of;
            }
            running += tot;
          }
          if (tid == 0) aux[nprobed] = running;
        }
        __syncthreads();
        const int64_t M = aux[nprobed];
        const int np = nprobed;
        mtot += M;
        for (int e = tid; e < ncarry; e += 256) buf[e] = carry[e];
        __syncthreads();
        ncm = stream_top(
            buf, M, carry != nullptr ? (int)a.kkeep : (int)kc,
            [&](int64_t m) -> unsigned long long {
              int lo = 0, hi = np - 1;
              while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (aux[mid] <= m) lo = mid;
                else hi = mid - 1;
              }
              const int64_t o = lst[lo], k = m - aux[lo];  // o: a multiple of 64
              const int64_t j = a.ids[o + k];
              return ivf_key(dot_strided(qs, a.muL + (o + (k & ~int64_t(63))) * d + (k & 63), 64, d),
                             j);
            },
            hist, shv, ws, ncarry);
        if (carry != nullptr) {
          for (int e = tid; e < ncm; e += 256) carry[e] = buf[e];
          ncarry = ncm;
          if (ncm > kc) {  // this round's kc best of the kkeep kept
            const unsigned long long T = block_kth_largest(buf, ncm, (int)kc, hist, shv);
            ncm = block_compact<unsigned long long>(buf, ncm, buf, ws,
                                                    [T](unsigned long long k) { return k >= T; });
          }
        }
        // a search that filled its kc slots reports its smallest score; a starved one (fewer
        // members than kc) reports -inf: nothing was cut by truncation
        if (mtot >= kc) dlast = key_score(block_min_key(buf, ncm, kslot));
      }
    }

    // merge with the staged top; each parent keeps its best sub-block; the top_c best parents
    const int n = ncm + nst;
    for (int e = tid; e < nst; e += 256) buf[ncm + e] = stg[e];
    __syncthreads();
    bool drop[kIvfCap / 256];
#pragma unroll
    for (int u = 0; u < kIvfCap / 256; ++u) {
      const int e = tid + 256 * u;
      drop[u] = false;
      if (e < n) {
        const unsigned long long v = buf[e];
        const int64_t p = ivf_key_index(v) / spb;
        for (int f = 0; f < n; ++f) {
          const unsigned long long y = buf[f];
          if (y > v && ivf_key_index(y) / spb == p) {
            drop[u] = true;
            break;
          }
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kIvfCap / 256; ++u)
      if (drop[u]) buf[tid + 256 * u] = 0ull;
    __syncthreads();
    const int nd = block_compact<unsigned long long>(buf, n, buf, ws,
                                                     [](unsigned long long k) { return k != 0ull; });
    const int K = (int)(a.top_c < nd ? a.top_c : nd);
    float tau = -INFINITY;
    if (K > 0) {
      if (K < nd) {
        const unsigned long long T = block_kth_largest(buf, nd, K, hist, shv);
        block_compact<unsigned long long>(buf, nd, buf, ws,
                                          [T](unsigned long long k) { return k >= T; });
      }
      tau = key_score(block_min_key(buf, K, kslot));
      for (int e = tid; e < K; e += 256) lst[e] = (int)(ivf_key_index(buf[e]) / spb);
      __syncthreads();
    }

    // outlier keys of past blocks scoring above tau: the ocap best, their parents
    int nop = 0;
    const int cap = (int)(a.ocap < a.n_out ? a.ocap : a.n_out);
    if (cap > 0) {
      const float* ov = a.ovec;
      const int64_t* op = a.opar;
      nop = stream_top(
          buf, a.n_out, cap,
          [&](int64_t r) -> unsigned long long {
            if (op[r] >= qblk) return 0ull;
            const float s = dot_row(qs, ov + r * d, d);
            return s > tau ? ivf_key(s, r) : 0ull;
          },
          hist, shv, ws);
      for (int e = tid; e < nop; e += 256) lst[K + e] = (int)op[ivf_key_index(buf[e])];
    }
    // the own block and `local` predecessors
    const int nloc = (int)((a.local < qblk ? a.local : qblk) + 1);
    for (int e = tid; e < nloc; e += 256) lst[K + nop + e] = (int)(qblk - e);
    __syncthreads();

    // distinct blocks, ascending
    const int nu = K + nop + nloc;
    bool dup[kIvfCap / 256];
#pragma unroll
    for (int u = 0; u < kIvfCap / 256; ++u) {
      const int e = tid + 256 * u;
      dup[u] = false;
      if (e < nu) {
        const int v = lst[e];
        for (int f = 0; f < e; ++f)
          if (lst[f] == v) {
            dup[u] = true;
            break;
          }
      }
    }
    if (tid == 0) nuniq = 0;
    __syncthreads();
    int mine = 0;
#pragma unroll
    for (int u = 0; u < kIvfCap / 256; ++u) {
      if (dup[u]) lst[tid + 256 * u] = 0x7fffffff;
      mine += (tid + 256 * u < nu) && !dup[u];
    }
    atomicAdd(&nuniq, mine);
    __syncthreads();
    for (int e = tid; e < nu; e += 256) {
      const int v = lst[e];
      if (v == 0x7fffffff) continue;
      int r = 0;
      for (int f = 0; f < nu; ++f) r += lst[f] < v;
      aux[r] = v;
    }
    __syncthreads();
    const int cnt = nuniq;
    if (tid == 0) a.kv_num[i] = cnt;
    int32_t* out = a.kv_idx + i * a.W;
    for (int64_t r = tid; r < a.W; r += 256) out[r] = r < cnt ? aux[r] : 0;

    // certificate: a full budget above -inf, no unprobed cell bound and no truncated search
    // reaching tau - margin
    bool ok = false;
    if (a.certify) {
      const int64_t want = a.top_c < qblk ? a.top_c : qblk;
      const bool full = (int64_t)K >= want;
      const bool has_tau = tau > -INFINITY;
      if (!a.has_index) {
        ok = full && (has_tau || qblk == 0);
      } else {
        const float lim = __fsub_rn(tau, a.margin);
        float mx = -INFINITY;
        for (int64_t c = tid; c < nlist; c += 256) {
          const bool probed = nprobe >= nlist || ivf_key(csv[c], c) >= Tc;
          if (!probed) mx = fmaxf(mx, __fadd_rn(csv[c], __fmul_rn(qn, a.rc[c])));
        }
        mx = block_max_f32(mx, fslot);
        ok = full && has_tau && mx < lim && dlast < lim;
      }
      if (tid == 0) {
        a.cert[i] = ok ? 1 : 0;
        a.rounds[i] = rnd;
      }
    } else if (tid == 0) {
      a.cert[i] = 0;
      a.rounds[i] = 0;
    }
    if (!a.certify || ok || !a.has_index || rnd >= a.max_esc) break;
    nprobe = nprobe * a.esc < nlist ? nprobe * a.esc : nlist;
    sk = sk * 2 < committed ? sk * 2 : committed;
    Tprev = Tc;
    __syncthreads();  // the next round rewrites buf / lst / aux
  }
}

}  // namespace
}  // namespace ssa

using ssa::CccLayout;

extern "C" size_t ssa_ccc_index_size(int64_t n_cap, int64_t nlist, int64_t d) {
  if (n_cap <= 0 || nlist <= 0 || d <= 0 || 2 * n_cap + 128 * nlist >= (int64_t(1) << 31)) return 0;
  return ssa::ccc_layout(n_cap, nlist, d).total;
}

namespace {

// The index addresses its list slots (2 n_cap + 128 nlist of them) with 32-bit offsets.
int check_ccc_cap(const char* fn, int64_t n_cap, int64_t nlist) {
  SSA_REQUIRE(2 * n_cap + 128 * nlist < (int64_t(1) << 31), SSA_ERR_UNSUPPORTED,
              "%s: n_cap=%lld with nlist=%lld exceeds the 32-bit list slots", fn,
              (long long)n_cap, (long long)nlist);
  return SSA_OK;
}

int check_ccc_rows(const char* fn, const float* x, int64_t n, int64_t d, int64_t nlist) {
  SSA_REQUIRE(x != nullptr && ssa::aligned16(x), SSA_ERR_INVALID,
              "%s: the means must be a 16-byte aligned device pointer", fn);
  SSA_REQUIRE(n > 0 && n < (int64_t(1) << 31), SSA_ERR_INVALID, "%s: bad n=%lld", fn,
              (long long)n);
  SSA_REQUIRE(d > 0 && d % 32 == 0 && d <= ssa::kIvfMaxD, SSA_ERR_UNSUPPORTED,
              "%s: d=%lld must be a multiple of 32 and at most %d", fn, (long long)d,
              ssa::kIvfMaxD);
  SSA_REQUIRE(nlist > 0 && nlist <= ssa::kIvfCap, SSA_ERR_UNSUPPORTED,
              "%s: nlist=%lld must be in [1, %d]", fn, (long long)nlist, ssa::kIvfCap);
  return SSA_OK;
}

int check_ccc_buffer(const char* fn, const void* buf, size_t bytes, size_t need) {
  SSA_REQUIRE(buf != nullptr && (reinterpret_cast<uintptr_t>(buf) & 255u) == 0, SSA_ERR_INVALID,
              "%s: the index / workspace must be a 256-byte aligned device pointer", fn);
  SSA_REQUIRE(bytes >= need, SSA_ERR_WORKSPACE, "%s: buffer holds %zu bytes, needs %zu", fn,
              bytes, need);
  return SSA_OK;
}

template <int DT>
int ccc_stage_impl(const void* x, int64_t m, int64_t d, int64_t rs, int64_t group, float* means,
                   int64_t quota, int64_t base, int64_t block, float* ovec, int64_t* opar,
                   int64_t* opos, unsigned long long* keys, hipStream_t s) {
  const int64_t ng = m / group;
  if (quota > 0) {
    ssa::ccc_means_kernel<DT, true><<<(unsigned)ng, 64, 0, s>>>(x, rs, d, group, means, keys);
    SSA_TRY(ssa::launch_status("ccc_means_kernel"));
    const int K = (int)(quota < m ? quota : m);
    const int64_t ntiles = (m + ssa::kIvfCap - 1) / ssa::kIvfCap;
    unsigned long long* cand = keys + m;
    ssa::ccc_tile_top_kernel<<<(unsigned)ntiles, 256, 0, s>>>(keys, m, K, cand);
    SSA_TRY(ssa::launch_status("ccc_tile_top_kernel"));
    ssa::ccc_outlier_kernel<DT><<<1, 256, 0, s>>>(cand, ntiles * K, K, x, rs, d, base, block,
                                                  ovec, opar, opos);
    return ssa::launch_status("ccc_outlier_kernel");
  }
  if (ng == 0) return SSA_OK;
  ssa::ccc_means_kernel<DT, false><<<(unsigned)ng, 64, 0, s>>>(x, rs, d, group, means, nullptr);
  return ssa::launch_status("ccc_means_kernel");
}

}  // namespace

extern "C" int ssa_ccc_stage(const void* x, int dtype, int64_t m, int64_t d, int64_t row_stride,
                             int64_t group, float* means, int64_t quota, int64_t base_tok,
                             int64_t block, float* out_vec, int64_t* out_parent,
                             int64_t* out_pos, void* ws, size_t ws_bytes, ssa_stream_t stream) {
  SSA_REQUIRE(x != nullptr && means != nullptr, SSA_ERR_INVALID, "ccc_stage: x / means is NULL");
  SSA_REQUIRE(ssa::dtype_size(dtype) > 0, SSA_ERR_INVALID, "ccc_stage: bad dtype %d", dtype);
  SSA_REQUIRE(d > 0 && d <= ssa::kIvfMaxD, SSA_ERR_UNSUPPORTED,
              "ccc_stage: d=%lld must be in [1, %d]", (long long)d, ssa::kIvfMaxD);
  SSA_REQUIRE(m >= 0 && m < (int64_t(1) << 31) && group > 0 && row_stride >= d, SSA_ERR_INVALID,
              "ccc_stage: need 0 <= m < 2^31, group > 0, row_stride >= d");
  SSA_REQUIRE(quota >= 0 && quota <= ssa::kIvfCap, SSA_ERR_UNSUPPORTED,
              "ccc_stage: quota=%lld must be in [0, %d]", (long long)quota, ssa::kIvfCap);
  if (m == 0) return SSA_OK;
  if (quota > 0) {
    SSA_REQUIRE(m % group == 0, SSA_ERR_INVALID,
                "ccc_stage: m=%lld rows are not whole groups of %lld", (long long)m,
                (long long)group);
    SSA_REQUIRE(out_vec != nullptr && out_parent != nullptr && out_pos != nullptr && block > 0,
                SSA_ERR_INVALID, "ccc_stage: outlier outputs are NULL or block <= 0");
    const int64_t K = quota < m ? quota : m;
    SSA_TRY(check_ccc_buffer("ccc_stage", ws, ws_bytes,
                             size_t(m) * 8 + size_t(K) * 8 * ((m + ssa::kIvfCap - 1) / ssa::kIvfCap)));
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  unsigned long long* keys = static_cast<unsigned long long*>(ws);
  switch (dtype) {
    case SSA_F32:
      return ccc_stage_impl<SSA_F32>(x, m, d, row_stride, group, means, quota, base_tok, block,
                                     out_vec, out_parent, out_pos, keys, s);
    case SSA_F16:
      return ccc_stage_impl<SSA_F16>(x, m, d, row_stride, group, means, quota, base_tok, block,
                                     out_vec, out_parent, out_pos, keys, s);
    default:
      return ccc_stage_impl<SSA_BF16>(x, m, d, row_stride, group, means, quota, base_tok, block,
                                      out_vec, out_parent, out_pos, keys, s);
  }
}

extern "C" int ssa_ccc_assign(const float* x, int64_t n, int64_t d, const float* cent,
                              int64_t nlist, int32_t* assign, void* ws, size_t ws_bytes,
                              ssa_stream_t stream) {
  SSA_TRY(check_ccc_rows("ccc_assign", x, n, d, nlist));
  SSA_REQUIRE(cent != nullptr && assign != nullptr, SSA_ERR_INVALID,
              "ccc_assign: cent / assign is NULL");
  SSA_TRY(check_ccc_cap("ccc_assign", n, nlist));
  const CccLayout L = ssa::ccc_layout(n, nlist, d);
  SSA_TRY(check_ccc_buffer("ccc_assign", ws, ws_bytes, L.total));
  char* base = static_cast<char*>(ws);
  return ssa::ccc_assign_rows(x, n, 0, d, cent, nlist,
                              reinterpret_cast<unsigned long long*>(base + L.pbest), L.pcap,
                              assign, nullptr, static_cast<hipStream_t>(stream));
}

extern "C" int ssa_ccc_kmeans(const float* x, int64_t n, int64_t d, int64_t nlist, int64_t iters,
                              int warm, float* cent, void* ws, size_t ws_bytes,
                              ssa_stream_t stream) {
  SSA_TRY(check_ccc_rows("ccc_kmeans", x, n, d, nlist));
  SSA_REQUIRE(cent != nullptr && iters >= 0, SSA_ERR_INVALID,
              "ccc_kmeans: cent is NULL or iters < 0");
  SSA_TRY(check_ccc_cap("ccc_kmeans", n, nlist));
  const CccLayout L = ssa::ccc_layout(n, nlist, d);
  SSA_TRY(check_ccc_buffer("ccc_kmeans", ws, ws_bytes, L.total));
  char* base = static_cast<char*>(ws);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!warm) {
    ssa::ccc_init_kernel<<<(unsigned)nlist, 64, 0, s>>>(x, n, d, nlist, cent);
    SSA_TRY(ssa::launch_status("ccc_init_kernel"));
  }
  const dim3 gc((unsigned)nlist, 1);
  for (int64_t it = 0; it < iters; ++it) {
    SSA_TRY(ssa::ccc_assign_rows(x, n, 0, d, cent, nlist,
                                 reinterpret_cast<unsigned long long*>(base + L.pbest), L.pcap,
                                 reinterpret_cast<int32_t*>(base + L.assign), nullptr, s));
    SSA_TRY(ssa::ccc_lists(x, n, d, nlist, L, base, false, nullptr, s));
    const int32_t* count = reinterpret_cast<const int32_t*>(base + L.count);
    const int32_t* off = reinterpret_cast<const int32_t*>(base + L.off);
    const int32_t* ids = reinterpret_cast<const int32_t*>(base + L.ids);
    switch ((d + 63) / 64) {
      case 1: ssa::ivf_update_kernel<1, false><<<gc, 64, 0, s>>>(x, count, off, ids, n, d, nlist, cent); break;
      case 2: ssa::ivf_update_kernel<2, false><<<gc, 64, 0, s>>>(x, count, off, ids, n, d, nlist, cent); break;
      case 3: ssa::ivf_update_kernel<3, false><<<gc, 64, 0, s>>>(x, count, off, ids, n, d, nlist, cent); break;
      default: ssa::ivf_update_kernel<4, false><<<gc, 64, 0, s>>>(x, count, off, ids, n, d, nlist, cent); break;
    }
    SSA_TRY(ssa::launch_status("ivf_update_kernel"));
  }
  return SSA_OK;
}

extern "C" int ssa_ccc_index_build(const float* x, int64_t n, int64_t d, int64_t nlist,
                                   const float* cent, void* index, int64_t n_cap,
                                   size_t index_bytes, ssa_stream_t stream) {
  SSA_TRY(check_ccc_rows("ccc_index_build", x, n, d, nlist));
  SSA_REQUIRE(cent != nullptr && n_cap >= n, SSA_ERR_INVALID,
              "ccc_index_build: cent is NULL or n_cap < n");
  SSA_TRY(check_ccc_cap("ccc_index_build", n_cap, nlist));
  const CccLayout L = ssa::ccc_layout(n_cap, nlist, d);
  SSA_TRY(check_ccc_buffer("ccc_index_build", index, index_bytes, L.total));
  char* base = static_cast<char*>(index);
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* ic = reinterpret_cast<float*>(base + L.cent);
  float* rc = reinterpret_cast<float*>(base + L.rc);
  if (cent != ic) {
    ssa::ccc_copy_kernel<<<(unsigned)((nlist * d + 63) / 64), 64, 0, s>>>(cent, ic, nlist * d);
    SSA_TRY(ssa::launch_status("ccc_copy_kernel"));
  }
  ssa::ccc_fill_kernel<<<(unsigned)((nlist + 255) / 256), 256, 0, s>>>(rc, nlist, 0.0f);
  SSA_TRY(ssa::launch_status("ccc_fill_kernel"));
  SSA_TRY(ssa::ccc_assign_rows(x, n, 0, d, ic, nlist,
                               reinterpret_cast<unsigned long long*>(base + L.pbest), L.pcap,
                               reinterpret_cast<int32_t*>(base + L.assign), rc, s));
  SSA_TRY(ssa::ccc_lists(x, n, d, nlist, L, base, true, nullptr, s));
  ssa::ivf_transpose_cent_kernel<<<dim3((unsigned)nlist, 1), 64, 0, s>>>(
      ic, d, nlist, reinterpret_cast<float*>(base + L.centT));
  return ssa::launch_status("ivf_transpose_cent_kernel");
}

extern "C" int ssa_ccc_index_add(const float* x, int64_t n_old, int64_t n, int64_t d,
                                 int64_t nlist, void* index, int64_t n_cap, size_t index_bytes,
                                 ssa_stream_t stream) {
  SSA_TRY(check_ccc_rows("ccc_index_add", x, n, d, nlist));
  SSA_REQUIRE(n_old >= 0 && n_old <= n && n <= n_cap, SSA_ERR_INVALID,
              "ccc_index_add: need 0 <= n_old <= n <= n_cap");
  SSA_TRY(check_ccc_cap("ccc_index_add", n_cap, nlist));
  const CccLayout L = ssa::ccc_layout(n_cap, nlist, d);
  SSA_TRY(check_ccc_buffer("ccc_index_add", index, index_bytes, L.total));
  if (n_old == n) return SSA_OK;
  char* base = static_cast<char*>(index);
  hipStream_t s = static_cast<hipStream_t>(stream);
  SSA_TRY(ssa::ccc_assign_rows(x + n_old * d, n - n_old, n_old, d,
                               reinterpret_cast<const float*>(base + L.cent), nlist,
                               reinterpret_cast<unsigned long long*>(base + L.pbest), L.pcap,
                               reinterpret_cast<int32_t*>(base + L.assign),
                               reinterpret_cast<float*>(base + L.rc), s));
  return ssa::ccc_lists_add(x, n_old, n, d, nlist, L, base, s);
}

extern "C" int ssa_ccc_route(const float* qr, int64_t nbq, int64_t qb_start, int64_t d,
                             const float* means, int64_t committed, int64_t n_sub, int64_t spb,
                             const void* index, int64_t n_cap, int64_t nlist,
                             const float* out_vec, const int64_t* out_parent, int64_t n_out,
                             int64_t top_c, int64_t local, int64_t outlier_cap,
                             int64_t search_k_staged, int64_t search_k, int64_t nprobe,
                             int64_t escalate_factor, int64_t max_escalations, int certify,
                             float cert_margin, int32_t* kv_num, int32_t* kv_idx, int64_t W,
                             uint8_t* cert, int32_t* rounds, void* ws, size_t ws_bytes,
                             ssa_stream_t stream) {
  SSA_REQUIRE(nbq >= 0 && nbq <= 0x7fffffff && qb_start >= 0, SSA_ERR_INVALID,
              "ccc_route: bad nbq / qb_start");
  if (nbq == 0) return SSA_OK;
  SSA_REQUIRE(qr != nullptr && ssa::aligned16(qr), SSA_ERR_INVALID,
              "ccc_route: qr must be a 16-byte aligned device pointer");
  SSA_REQUIRE(d > 0 && d % 32 == 0 && d <= ssa::kIvfMaxD, SSA_ERR_UNSUPPORTED,
              "ccc_route: d=%lld must be a multiple of 32 and at most %d", (long long)d,
              ssa::kIvfMaxD);
  SSA_REQUIRE(committed >= 0 && committed <= n_sub && n_sub < (int64_t(1) << 31) && spb >= 1,
              SSA_ERR_INVALID, "ccc_route: need 0 <= committed <= n_sub < 2^31, spb >= 1");
  SSA_REQUIRE(n_sub == 0 || (means != nullptr && ssa::aligned16(means)), SSA_ERR_INVALID,
              "ccc_route: means must be a 16-byte aligned device pointer");
  SSA_REQUIRE(n_out >= 0 && (n_out == 0 || (out_vec != nullptr && out_parent != nullptr &&
                                            ssa::aligned16(out_vec))),
              SSA_ERR_INVALID, "ccc_route: outlier arrays are NULL or unaligned");
  SSA_REQUIRE(top_c >= 0 && local >= 0 && outlier_cap >= 0 && search_k_staged >= 1 &&
                  search_k >= 1 && nprobe >= 1 && escalate_factor >= 1 && max_escalations >= 0,
              SSA_ERR_INVALID, "ccc_route: negative or zero budget / search parameter");
  SSA_REQUIRE(kv_num != nullptr && kv_idx != nullptr && cert != nullptr && rounds != nullptr,
              SSA_ERR_INVALID, "ccc_route: an output is NULL");
  const int64_t ns = n_sub - committed;
  const int64_t ks = search_k_staged < ns ? search_k_staged : ns;
  int64_t skmax = search_k < committed ? search_k : committed;
  if (index != nullptr && certify) {
    int64_t sk = search_k;
    for (int64_t r = 0; r < max_escalations; ++r) sk = sk * 2 < committed ? sk * 2 : committed;
    skmax = sk > skmax ? sk : skmax;
  }
  SSA_REQUIRE(ks <= ssa::kIvfMaxSearch && skmax <= ssa::kIvfMaxSearch, SSA_ERR_UNSUPPORTED,
              "ccc_route: search_k (staged %lld, committed up to %lld) exceeds %d",
              (long long)ks, (long long)skmax, ssa::kIvfMaxSearch);
  const int64_t keep = top_c < ks + skmax ? top_c : ks + skmax;
  const int64_t ocap = outlier_cap < n_out ? outlier_cap : n_out;
  SSA_REQUIRE(ocap <= ssa::kIvfMaxSearch, SSA_ERR_UNSUPPORTED,
              "ccc_route: min(outlier_cap, n_out)=%lld exceeds %d", (long long)ocap,
              ssa::kIvfMaxSearch);
  const int64_t nb_global = qb_start + nbq;
  const int64_t win = (local < nb_global - 1 ? local : nb_global - 1) + 1;
  SSA_REQUIRE(keep + ocap + win <= ssa::kIvfCap, SSA_ERR_UNSUPPORTED,
              "ccc_route: top_c + outlier_cap + local + 1 = %lld exceeds %d",
              (long long)(keep + ocap + win), ssa::kIvfCap);
  const int64_t wfull = top_c + local + 1 + outlier_cap;
  const int64_t wneed = wfull < nb_global ? wfull : nb_global;
  SSA_REQUIRE(W >= wneed, SSA_ERR_INVALID,
              "ccc_route: W=%lld < min(top_c + local + 1 + outlier_cap, qb_start + nbq)=%lld",
              (long long)W, (long long)wneed);
  ssa::CccRouteArgs a = {};
  if (index != nullptr) {
    SSA_REQUIRE(nlist >= 1 && nlist <= ssa::kIvfCap && n_cap >= committed && committed > 0,
                SSA_ERR_INVALID, "ccc_route: bad index geometry (nlist, n_cap, committed)");
    SSA_REQUIRE((reinterpret_cast<uintptr_t>(index) & 255u) == 0, SSA_ERR_INVALID,
                "ccc_route: index must be a 256-byte aligned device pointer");
    SSA_TRY(check_ccc_cap("ccc_route", n_cap, nlist));
    const CccLayout L = ssa::ccc_layout(n_cap, nlist, d);
    const char* base = static_cast<const char*>(index);
    a.has_index = 1;
    a.centT = reinterpret_cast<const float*>(base + L.centT);
    a.muL = reinterpret_cast<const float*>(base + L.muL);
    a.count = reinterpret_cast<const int32_t*>(base + L.count);
    a.off = reinterpret_cast<const int32_t*>(base + L.off);
    a.ids = reinterpret_cast<const int32_t*>(base + L.ids);
    a.rc = reinterpret_cast<const float*>(base + L.rc);
    a.nlist = nlist;
  }
  a.qr = qr;
  a.nbq = nbq;
  a.qb_start = qb_start;
  a.d = d;
  a.means = means;
  a.committed = committed;
  a.n_sub = n_sub;
  a.spb = spb;
  a.ovec = out_vec;
  a.opar = out_parent;
  a.n_out = n_out;
  a.top_c = top_c;
  a.local = local;
  a.ocap = outlier_cap;
  a.ks = search_k_staged;
  a.sk0 = search_k;
  a.nprobe0 = index != nullptr ? (nprobe < nlist ? nprobe : nlist) : nprobe;
  a.esc = escalate_factor;
  a.max_esc = max_escalations;
  a.certify = certify ? 1 : 0;
  a.margin = cert_margin;
  a.kv_num = kv_num;
  a.kv_idx = kv_idx;
  a.W = W;
  a.cert = cert;
  a.rounds = rounds;
  if (index != nullptr && certify && max_escalations > 0) {
    // the escalation carry: nbq rows of skmax keys (skmax >= every round's search_k)
    const size_t need = size_t(nbq) * size_t(skmax) * 8;
    SSA_REQUIRE(ws != nullptr && (reinterpret_cast<uintptr_t>(ws) & 7u) == 0, SSA_ERR_INVALID,
                "ccc_route: escalation needs an 8-byte aligned workspace");
    SSA_REQUIRE(ws_bytes >= need, SSA_ERR_WORKSPACE,
                "ccc_route: workspace holds %zu bytes, escalation needs %zu", ws_bytes, need);
    a.carry = static_cast<unsigned long long*>(ws);
    a.kkeep = skmax;
  }
  ssa::ccc_route_kernel<<<(unsigned)nbq, 256, 0, static_cast<hipStream_t>(stream)>>>(a);
  return ssa::launch_status("ccc_route_kernel");
}
