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
#include "ivf_parts.h"

namespace ssa {
namespace {

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
    ssa::ivf_score_kernel<<<gs, ssa::kScoreTile, ssa::kAssignC * d * sizeof(double), s>>>(
        mu, cent, nb, d, nlist, L.per_group, pbest);
    SSA_TRY(ssa::launch_status("ivf_score_kernel"));
    ssa::ivf_rank_kernel<<<gt, ssa::kTile, 0, s>>>(pbest, nb, nlist, L.ntiles, L.groups, assign,
                                                    rank, tcount);
    SSA_TRY(ssa::launch_status("ivf_rank_kernel"));
    SSA_TRY(ssa::ivf_lists(assign, rank, tcount, BH, nb, nlist, L.ntiles, count, off, ids, mu, d,
                           last ? muL : nullptr, s));
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
