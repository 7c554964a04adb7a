// Bounded-candidate treecode router: an F-ary tree over the key blocks of each head, each node
// carrying a mean, a diagonal variance, a recursive radius R (every key below the node lies
// within R of its mean) and the first token it covers; a query descends it with a fixed-width
// beam, scoring the W·F children of the frontier by the admissible bound <q, mu> + |q| R (plus
// the cumulant term beta/2 <q*q, var>), and returns the top_c leaf blocks of the last frontier.
// Reference: ssa/treecode.py:34-86 (build_tree), :89-137 (descend_beam).
//
// Layout (tree_layout): levels from the leaves (level 0, nb nodes) up to the first level of at
// most top_cap nodes; per level mu (BH, n, d) fp32, var (BH, n, d) fp32, R (BH, n) fp32 and lo (n)
// int64, each region 256-byte aligned. Node p of level l + 1 has children p F .. p F + F - 1 of
// level l (those below that level's count).
//
// Numerics: sums in fp64 from the stored fp32 values, each stored value rounded once. Scores are
// fp64, rounded to fp32 and ranked by (score desc, node asc): the frontier is kept in ascending
// node order, so its children enter the wave's selection in ascending node order and ties at the
// cut go to the lower node.
#include <math.h>

#include "common.h"
#include "select.h"

namespace ssa {
namespace {

constexpr int kTreeMaxD = 512;
constexpr int kTreeMaxLevels = 24;
constexpr int kTreeMaxF = 16;
constexpr int kTreeMaxW = 64;
constexpr int kTreeMaxTop = 64;

struct TreeLayout {
  int nlev;
  int64_t n[kTreeMaxLevels];
  int64_t mu[kTreeMaxLevels], var[kTreeMaxLevels], R[kTreeMaxLevels], lo[kTreeMaxLevels];
  int64_t total;
};

// Levels while the last one holds more than top_cap nodes (ssa/treecode.py:55): n_{l+1} =
// ceil(n_l / F). Returns false when more than kTreeMaxLevels levels would be needed.
bool tree_layout(int64_t BH, int64_t nb, int64_t d, int64_t F, int64_t top_cap, TreeLayout* L) {
  const auto r256 = [](int64_t x) { return (x + 255) / 256 * 256; };
  int64_t off = 0, n = nb;
  int l = 0;
  while (true) {
    if (l == kTreeMaxLevels) return false;
    L->n[l] = n;
    L->mu[l] = off;
    off += r256(BH * n * d * 4);
    L->var[l] = off;
    off += r256(BH * n * d * 4);
    L->R[l] = off;
    off += r256(BH * n * 4);
    L->lo[l] = off;
    off += r256(n * 8);
    ++l;
    if (n <= top_cap) break;
    n = (n + F - 1) / F;
  }
  L->nlev = l;
  L->total = off;
  return true;
}

template <int DT>
__device__ inline float tree_load(const char* base, int64_t idx) {
  if constexpr (DT == SSA_F32) return reinterpret_cast<const float*>(base)[idx];
  else {
    const unsigned short u = reinterpret_cast<const unsigned short*>(base)[idx];
    if constexpr (DT == SSA_BF16) return __uint_as_float((unsigned int)u << 16);
    else return (float)__builtin_bit_cast(_Float16, u);
  }
}

__device__ inline double wave_sum_d(double x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += lane_xor(x, off);
  return x;
}
__device__ inline double wave_max_d(double x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = fmax(x, lane_xor(x, off));
  return x;
}

// Leaves (ssa/treecode.py:40-52): block c of head bh, a workgroup of 256 threads that loads the
// block once. A key row is read by LPR = d / DPL threads (DPL = 4 or 8 consecutive dims each, LPR
// a power of two), RPI = 256 / LPR rows per pass, U passes (U RPI >= block), every value held in
// registers. Mean and population variance E[k^2] - mean^2 from fp64 sums (reduced over the
// threads sharing a dim slice, then over the 4 waves), then each row's |k - fl32(mean)|^2 from the
// registers, R = the largest, square-rooted. grid (nb, BH).
template <int DT, int DPL, int U>
__global__ __launch_bounds__(256) void tree_leaf_kernel(const char* __restrict__ k, int64_t H,
                                                        int64_t sb, int64_t sh, int64_t sn, int d,
                                                        int64_t block, int64_t nb, float* mu,
                                                        float* var, float* R, int64_t* lo) {
  extern __shared__ double tree_dyn[];  // [2][4][d] cross-wave partial sums
  __shared__ float smu[kTreeMaxD];
  __shared__ double rmax[4];
  auto red = [&](int which, int w, int e) -> double& { return tree_dyn[(which * 4 + w) * d + e]; };
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t c = blockIdx.x, bh = blockIdx.y;
  const int64_t head = (bh / H) * sb + (bh % H) * sh;
  const int64_t row0 = c * block;
  const int lpr = d / DPL, rpi = 256 / lpr;
  const int sub = tid / lpr, e0 = (tid % lpr) * DPL;  // this thread's first row and first dim
  float x[U][DPL];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t j = sub + (int64_t)rpi * u;
#pragma unroll
    for (int t = 0; t < DPL; ++t) x[u][t] = 0.0f;
    if (j < block) {
      const int64_t rb = head + (row0 + j) * sn + e0;
      if constexpr (DT == SSA_F32) {
#pragma unroll
        for (int t = 0; t < DPL; t += 4) {
          const f32x4 v =
              *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(k) + rb + t);
#pragma unroll
          for (int w = 0; w < 4; ++w) x[u][t + w] = v[w];
        }
      } else {
#pragma unroll
        for (int t = 0; t < DPL; t += 4) {
          const uint2 w2 =
              *reinterpret_cast<const uint2*>(reinterpret_cast<const unsigned short*>(k) + rb + t);
          const unsigned int ww[2] = {w2.x, w2.y};
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const unsigned short h = (unsigned short)(ww[w >> 1] >> (16 * (w & 1)));
            if constexpr (DT == SSA_BF16) x[u][t + w] = __uint_as_float((unsigned int)h << 16);
            else x[u][t + w] = (float)__builtin_bit_cast(_Float16, h);
          }
        }
      }
    }
  }
  // per-dim sums over the thread's rows, then over the wave's row groups, then over the waves
  double s1[DPL], s2[DPL];
#pragma unroll
  for (int t = 0; t < DPL; ++t) {
    s1[t] = s2[t] = 0.0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      s1[t] += (double)x[u][t];
      s2[t] = fma((double)x[u][t], (double)x[u][t], s2[t]);
    }
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1)  // (unrolled: lane_xor needs a constant distance)
    if (off >= lpr)
#pragma unroll
      for (int t = 0; t < DPL; ++t) {
        s1[t] += lane_xor(s1[t], off);
        s2[t] += lane_xor(s2[t], off);
      }
  if (lane < lpr)
#pragma unroll
    for (int t = 0; t < DPL; ++t) {
      red(0, wv, e0 + t) = s1[t];
      red(1, wv, e0 + t) = s2[t];
    }
  __syncthreads();
  if (tid < lpr) {
    float* m_out = mu + (bh * nb + c) * d + e0;
    float* v_out = var + (bh * nb + c) * d + e0;
#pragma unroll
    for (int t = 0; t < DPL; ++t) {
      const double a1 = red(0, 0, e0 + t) + red(0, 1, e0 + t) + red(0, 2, e0 + t) + red(0, 3, e0 + t);
      const double a2 = red(1, 0, e0 + t) + red(1, 1, e0 + t) + red(1, 2, e0 + t) + red(1, 3, e0 + t);
      const double m = a1 / (double)block;
      const float mf = (float)m;
      m_out[t] = mf;
      v_out[t] = (float)(a2 / (double)block - m * m);
      smu[e0 + t] = mf;
    }
  }
  __syncthreads();
  float mf[DPL];
#pragma unroll
  for (int t = 0; t < DPL; ++t) mf[t] = smu[e0 + t];
  double mx = 0.0;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    double acc = 0.0;
#pragma unroll
    for (int t = 0; t < DPL; ++t) {
      const double y = (double)x[u][t] - (double)mf[t];
      acc = fma(y, y, acc);
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1)
      if (off < lpr) acc += lane_xor(acc, off);
    if (sub + (int64_t)rpi * u < block) mx = fmax(mx, acc);
  }
  mx = wave_max_d(mx);
  if (lane == 0) rmax[wv] = mx;
  __syncthreads();
  if (tid == 0) {
    R[bh * nb + c] = (float)sqrt(fmax(fmax(rmax[0], rmax[1]), fmax(rmax[2], rmax[3])));
    if (bh == 0) lo[c] = row0;
  }
}

// Leaves for head dims whose row does not split into a power-of-two number of 4- / 8-dim lane
// slices: pass 1 lane e over dims e, e + 64, ...; pass 2 lane j over keys j, j + 64, ... (the same
// statistics as tree_leaf_kernel).
template <int DT>
__global__ __launch_bounds__(64) void tree_leaf_any_kernel(const char* __restrict__ k, int64_t H,
                                                           int64_t sb, int64_t sh, int64_t sn,
                                                           int d, int64_t block, int64_t nb,
                                                           float* mu, float* var, float* R,
                                                           int64_t* lo) {
  __shared__ float smu[kTreeMaxD];
  constexpr int NE = kTreeMaxD / 64;
  const int lane = threadIdx.x;
  const int64_t c = blockIdx.x, bh = blockIdx.y;
  const int64_t head = (bh / H) * sb + (bh % H) * sh;
  const int64_t row0 = c * block;
  double s1[NE], s2[NE];
#pragma unroll
  for (int t = 0; t < NE; ++t) s1[t] = s2[t] = 0.0;
  for (int64_t j = 0; j < block; ++j) {
    const int64_t rb = head + (row0 + j) * sn;
#pragma unroll
    for (int t = 0; t < NE; ++t) {
      const int e = lane + 64 * t;
      if (e < d) {
        const double x = (double)tree_load<DT>(k, rb + e);
        s1[t] += x;
        s2[t] = fma(x, x, s2[t]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < NE; ++t) {
    const int e = lane + 64 * t;
    if (e < d) {
      const double m = s1[t] / (double)block;
      const float mf = (float)m;
      mu[(bh * nb + c) * d + e] = mf;
      var[(bh * nb + c) * d + e] = (float)(s2[t] / (double)block - m * m);
      smu[e] = mf;
    }
  }
  wave_lds_sync();
  double mx = 0.0;
  for (int64_t j = lane; j < block; j += 64) {
    const int64_t rb = head + (row0 + j) * sn;
    double acc = 0.0;
    for (int e = 0; e < d; ++e) {
      const double x = (double)tree_load<DT>(k, rb + e) - (double)smu[e];
      acc = fma(x, x, acc);
    }
    mx = fmax(mx, acc);
  }
  mx = wave_max_d(mx);
  if (lane == 0) {
    R[bh * nb + c] = (float)sqrt(mx);
    if (bh == 0) lo[c] = row0;
  }
}

// One level up (ssa/treecode.py:55-76): parent p of head bh over its real children c = p F + f
// (c < nc): mean of the children's means, variance mean(var_c + mu_c^2) - mean^2, R = max_c
// (|mu_c - fl32(mean)| + R_c), lo = min_c lo_c. grid (np, BH), one wave.
__global__ __launch_bounds__(64) void tree_level_kernel(const float* __restrict__ cmu,
                                                        const float* __restrict__ cvar,
                                                        const float* __restrict__ cR,
                                                        const int64_t* __restrict__ clo, int64_t nc,
                                                        float* pmu, float* pvar, float* pR,
                                                        int64_t* plo, int64_t np, int d, int F) {
  __shared__ float sp[kTreeMaxD];
  const int lane = threadIdx.x;
  const int64_t p = blockIdx.x, bh = blockIdx.y;
  const int64_t c0 = p * F;
  const int cnt = (int)(nc - c0 < F ? nc - c0 : F);
  const float* m_in = cmu + (bh * nc + c0) * d;
  const float* v_in = cvar + (bh * nc + c0) * d;
  for (int e = lane; e < d; e += 64) {
    double s1 = 0.0, s2 = 0.0;
    for (int f = 0; f < cnt; ++f) {
      const double m = (double)m_in[f * d + e];
      s1 += m;
      s2 += (double)v_in[f * d + e] + m * m;
    }
    const double m = s1 / (double)cnt;
    const float mf = (float)m;
    pmu[(bh * np + p) * d + e] = mf;
    pvar[(bh * np + p) * d + e] = (float)(s2 / (double)cnt - m * m);
    sp[e] = mf;
  }
  wave_lds_sync();
  double r = -INFINITY;
  for (int f = 0; f < cnt; ++f) {
    double acc = 0.0;
    for (int e = lane; e < d; e += 64) {
      const double x = (double)m_in[f * d + e] - (double)sp[e];
      acc = fma(x, x, acc);
    }
    acc = wave_sum_d(acc);
    r = fmax(r, sqrt(acc) + (double)cR[bh * nc + c0 + f]);
  }
  if (lane == 0) {
    pR[bh * np + p] = (float)r;
    if (bh == 0) {
      int64_t l = clo[c0];
      for (int f = 1; f < cnt; ++f) l = clo[c0 + f] < l ? clo[c0 + f] : l;
      plo[p] = l;
    }
  }
}

struct TreeArgs {
  const char* tree;
  TreeLayout L;
  const float* q;        // (BH, Q, d)
  const int64_t* q_pos;  // (BH, Q) or NULL (no causal mask)
  int64_t BH, Q;
  int d, F, W, tc;
  double half_beta;
  int32_t* sel;  // (BH, Q, tc)
};

// The admissible bound of node `node` of level l for the wave's query (q in LDS, |q| = qn):
// <q, mu> + qn R (+ beta/2 <q*q, var>), fp64, rounded to fp32.
__device__ inline float tree_score(const TreeArgs& a, int l, int64_t bh, int64_t node,
                                   const float* sq, double qn) {
  const int64_t n = a.L.n[l];
  const float* m = reinterpret_cast<const float*>(a.tree + a.L.mu[l]) + (bh * n + node) * a.d;
  double e1 = 0.0, e2 = 0.0;
  for (int e = 0; e < a.d; e += 4) {
    const f32x4 mm = *reinterpret_cast<const f32x4*>(m + e);
#pragma unroll
    for (int t = 0; t < 4; ++t) e1 = fma((double)sq[e + t], (double)mm[t], e1);
  }
  if (a.half_beta != 0.0) {
    const float* v = reinterpret_cast<const float*>(a.tree + a.L.var[l]) + (bh * n + node) * a.d;
    for (int e = 0; e < a.d; e += 4) {
      const f32x4 vv = *reinterpret_cast<const f32x4*>(v + e);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const double x = (double)sq[e + t];
        e2 = fma(x * x, (double)vv[t], e2);
      }
    }
  }
  const double Rn = (double)reinterpret_cast<const float*>(a.tree + a.L.R[l])[bh * n + node];
  return (float)((e1 + qn * Rn) + a.half_beta * e2);
}

// One wave per query (grid (Q, BH)): the top level scanned whole, then per level the W F
// children of the frontier scored and the best W kept (J = candidate slots per lane), then the
// best tc leaves of the last frontier in (score desc, node asc) order, -1 past the valid ones.
template <int J>
__global__ __launch_bounds__(64) void tree_descend_kernel(TreeArgs a) {
  __shared__ float sq[kTreeMaxD];
  __shared__ int64_t fr[kTreeMaxW];
  __shared__ unsigned int fk[kTreeMaxW];
  const int lane = threadIdx.x;
  const int64_t qi = blockIdx.x, bh = blockIdx.y;
  const unsigned long long lt = (1ull << lane) - 1ull;
  const float* qrow = a.q + (bh * a.Q + qi) * a.d;
  double qn2 = 0.0;
  for (int e = lane; e < a.d; e += 64) {
    const float x = qrow[e];
    sq[e] = x;
    qn2 = fma((double)x, (double)x, qn2);
  }
  const double qn = sqrt(wave_sum_d(qn2));
  const int64_t qpos = a.q_pos ? a.q_pos[bh * a.Q + qi] : INT64_MAX;
  wave_lds_sync();

  // top level: every node (at most 64, one per lane)
  const int top = a.L.nlev - 1;
  int nf = 0;
  {
    const int64_t n = a.L.n[top];
    const int64_t* lo = reinterpret_cast<const int64_t*>(a.tree + a.L.lo[top]);
    const bool valid = lane < n && lo[lane] <= qpos;
    unsigned int key[1] = {valid ? score_key(tree_score(a, top, bh, lane, sq, qn)) : 0u};
    const unsigned long long vb = __ballot(valid);
    const int nvalid = (int)__popcll(vb);
    const unsigned int take = wave_select_top<1>(key, valid ? 1u : 0u, a.W, nvalid);
    const unsigned long long tb = __ballot(take & 1u);
    if (take & 1u) {
      const int slot = (int)__popcll(tb & lt);
      fr[slot] = lane;
      fk[slot] = key[0];
    }
    nf = (int)__popcll(tb);
    wave_lds_sync();
  }
  // levels below: children of the frontier, ascending (the frontier is ascending)
  for (int l = top - 1; l >= 0; --l) {
    const int64_t n = a.L.n[l];
    const int64_t* lo = reinterpret_cast<const int64_t*>(a.tree + a.L.lo[l]);
    const int ncand = nf * a.F;
    unsigned int key[J];
    int64_t node[J];
    unsigned int cm = 0u;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int s = lane + 64 * j;
      key[j] = 0u;
      node[j] = -1;
      if (s < ncand) {
        const int64_t c = fr[s / a.F] * a.F + (s % a.F);
        if (c < n && lo[c] <= qpos) {
          node[j] = c;
          key[j] = score_key(tree_score(a, l, bh, c, sq, qn));
          cm |= 1u << j;
        }
      }
    }
    int nvalid = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) nvalid += (int)__popcll(__ballot((cm >> j) & 1u));
    const unsigned int take = wave_select_top<J>(key, cm, a.W, nvalid);
    wave_lds_sync();  // every lane has read the old frontier
    int at = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const bool t = (take >> j) & 1u;
      const unsigned long long tb = __ballot(t);
      if (t) {
        const int slot = at + (int)__popcll(tb & lt);
        fr[slot] = node[j];
        fk[slot] = key[j];
      }
      at += (int)__popcll(tb);
    }
    nf = at;
    wave_lds_sync();
  }
  // the best tc leaves, (score desc, node asc)
  unsigned int k = lane < nf ? fk[lane] : 0u;
  unsigned int c = lane < nf ? (unsigned int)fr[lane] : 0xffffffffu;
  wave_sort_desc(k, c);
  if (lane < a.tc)
    a.sel[(bh * a.Q + qi) * a.tc + lane] = lane < nf ? (int32_t)c : -1;
}


constexpr int kTreePackMax = 256;  // candidates of a packed row: leaves + local window

// One wave per row r of (b, h, i) rows, i = r % nb: the descent's leaves of the row (sel[r, 0..tc),
// -1 = none) OR blocks i - local .. i, distinct and ascending in kv_idx[r] (pad 0), counted in
// kv_num[r]. A value is kept at its first occurrence; its slot is the number of kept values
// below it.
__global__ __launch_bounds__(64) void tree_pack_kernel(const int32_t* __restrict__ sel, int64_t nb,
                                                        int tc, int64_t local,
                                                        int32_t* __restrict__ kv_num,
                                                        int32_t* __restrict__ kv_idx, int64_t W) {
  __shared__ int c[kTreePackMax];
  __shared__ int first[kTreePackMax];
  const int64_t r = blockIdx.x;
  const int lane = threadIdx.x;
  const int64_t i = r % nb;
  const int nloc = (int)((local < i ? local : i) + 1);
  const int n = tc + nloc;
  for (int e = lane; e < n; e += 64) {
    int v = e < tc ? sel[r * tc + e] : (int)(i - (e - tc));
    c[e] = v < 0 ? 0x7fffffff : v;
  }
  __syncthreads();
  for (int e = lane; e < n; e += 64) {
    const int v = c[e];
    bool f = v != 0x7fffffff;
    for (int g = 0; g < e && f; ++g) f = c[g] != v;
    first[e] = f ? 1 : 0;
  }
  __syncthreads();
  int mine = 0;
  for (int e = lane; e < n; e += 64) mine += first[e];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mine += __shfl_xor(mine, o);
  int32_t* out = kv_idx + r * W;
  for (int e = lane; e < n; e += 64) {
    if (!first[e]) continue;
    const int v = c[e];
    int rank = 0;
    for (int g = 0; g < n; ++g) rank += (first[g] && c[g] < v) ? 1 : 0;
    out[rank] = v;
  }
  for (int64_t s = mine + lane; s < W; s += 64) out[s] = 0;
  if (lane == 0) kv_num[r] = mine;
}

}  // namespace
}  // namespace ssa

extern "C" size_t ssa_tree_size(int64_t BH, int64_t nb, int64_t d, int64_t F, int64_t top_cap) {
  ssa::TreeLayout L;
  if (BH <= 0 || nb <= 0 || d <= 0 || F < 2 || top_cap < 1) return 0;
  if (!ssa::tree_layout(BH, nb, d, F, top_cap, &L)) return 0;
  return (size_t)L.total;
}

extern "C" int ssa_tree_build(const void* k, int dtype, int64_t B, int64_t H, int64_t n, int64_t d,
                              int64_t block, const int64_t* strides, int64_t F, int64_t top_cap,
                              void* tree, size_t tree_bytes, ssa_stream_t stream) {
  using namespace ssa;
  SSA_REQUIRE(k && strides && tree, SSA_ERR_INVALID, "tree_build: NULL pointer argument");
  SSA_REQUIRE(dtype == SSA_F32 || dtype == SSA_F16 || dtype == SSA_BF16, SSA_ERR_UNSUPPORTED,
              "tree_build: unknown dtype %d", dtype);
  SSA_REQUIRE(B > 0 && H > 0 && block > 0 && n >= block, SSA_ERR_INVALID,
              "tree_build: need B, H > 0 and at least one whole block (n=%lld, block=%lld)",
              (long long)n, (long long)block);
  SSA_REQUIRE(d > 0 && d <= kTreeMaxD && d % 4 == 0, SSA_ERR_UNSUPPORTED,
              "tree_build: head_dim must be a multiple of 4 up to %d", kTreeMaxD);
  SSA_REQUIRE(F >= 2 && F <= kTreeMaxF && top_cap >= 1 && top_cap <= kTreeMaxTop,
              SSA_ERR_UNSUPPORTED, "tree_build: need 2 <= F <= %d and 1 <= top_cap <= %d",
              kTreeMaxF, kTreeMaxTop);
  const int64_t nb = n / block, BH = B * H;
  SSA_REQUIRE(BH < 65536 && nb < (1ll << 31), SSA_ERR_UNSUPPORTED, "tree_build: grid too large");
  TreeLayout L;
  SSA_REQUIRE(tree_layout(BH, nb, d, F, top_cap, &L), SSA_ERR_UNSUPPORTED,
              "tree_build: more than %d levels", kTreeMaxLevels);
  SSA_REQUIRE(tree_bytes >= (size_t)L.total && aligned16(tree), SSA_ERR_WORKSPACE,
              "tree_build: the tree needs %lld bytes (16-byte aligned)", (long long)L.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* t = static_cast<char*>(tree);
  const auto f = [&](int64_t off) { return reinterpret_cast<float*>(t + off); };
  const auto i64 = [&](int64_t off) { return reinterpret_cast<int64_t*>(t + off); };
  const char* kc = static_cast<const char*>(k);
  const dim3 g0((unsigned)nb, (unsigned)BH);
  // DPL dims per thread: 4 up to d = 256, 8 at d = 512; the block-resident kernel needs a
  // power-of-two number of threads per row, 4-element-aligned rows and U = ceil(block * LPR /
  // 256) <= 16 passes; else the scalar kernel runs
  const int dpl = d <= 256 ? 4 : 8;
  const int64_t lpr = d / dpl;
  const int64_t passes = (block * lpr + 255) / 256;
  const bool vec = (lpr & (lpr - 1)) == 0 && d % dpl == 0 && lpr <= 64 && passes * dpl <= 64 &&
                   strides[0] % 4 == 0 && strides[1] % 4 == 0 && strides[2] % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(k) % (4 * (size_t)dtype_size(dtype))) == 0;
  const int up = passes <= 1 ? 1 : passes <= 2 ? 2 : passes <= 4 ? 4 : passes <= 8 ? 8 : 16;
#define SSA_TREE_LEAF_U(DT, P, UU)                                                                \
  tree_leaf_kernel<DT, P, UU><<<g0, 256, 64 * d, st>>>(kc, H, strides[0], strides[1], strides[2],      \
                                                  (int)d, block, nb, f(L.mu[0]), f(L.var[0]),     \
                                                  f(L.R[0]), i64(L.lo[0]))
#define SSA_TREE_LEAF(DT, P)                                                                      \
  do {                                                                                            \
    if (up == 1) SSA_TREE_LEAF_U(DT, P, 1);                                                       \
    else if (up == 2) SSA_TREE_LEAF_U(DT, P, 2);                                                  \
    else if (up == 4) SSA_TREE_LEAF_U(DT, P, 4);                                                  \
    else if (up == 8) SSA_TREE_LEAF_U(DT, P, 8);                                                  \
    else SSA_TREE_LEAF_U(DT, P, 16);                                                              \
  } while (0)
  if (!vec) {
    if (dtype == SSA_F32)
      tree_leaf_any_kernel<SSA_F32><<<g0, 64, 0, st>>>(kc, H, strides[0], strides[1], strides[2],
                                                       (int)d, block, nb, f(L.mu[0]), f(L.var[0]),
                                                       f(L.R[0]), i64(L.lo[0]));
    else if (dtype == SSA_F16)
      tree_leaf_any_kernel<SSA_F16><<<g0, 64, 0, st>>>(kc, H, strides[0], strides[1], strides[2],
                                                       (int)d, block, nb, f(L.mu[0]), f(L.var[0]),
                                                       f(L.R[0]), i64(L.lo[0]));
    else
      tree_leaf_any_kernel<SSA_BF16><<<g0, 64, 0, st>>>(kc, H, strides[0], strides[1], strides[2],
                                                        (int)d, block, nb, f(L.mu[0]), f(L.var[0]),
                                                        f(L.R[0]), i64(L.lo[0]));
  } else if (dtype == SSA_F32) {
    if (dpl == 4) SSA_TREE_LEAF(SSA_F32, 4);
    else SSA_TREE_LEAF(SSA_F32, 8);
  } else if (dtype == SSA_F16) {
    if (dpl == 4) SSA_TREE_LEAF(SSA_F16, 4);
    else SSA_TREE_LEAF(SSA_F16, 8);
  } else {
    if (dpl == 4) SSA_TREE_LEAF(SSA_BF16, 4);
    else SSA_TREE_LEAF(SSA_BF16, 8);
  }
#undef SSA_TREE_LEAF
#undef SSA_TREE_LEAF_U
  SSA_TRY(launch_status("tree_leaf_kernel"));
  for (int l = 1; l < L.nlev; ++l) {
    const dim3 g((unsigned)L.n[l], (unsigned)BH);
    tree_level_kernel<<<g, 64, 0, st>>>(f(L.mu[l - 1]), f(L.var[l - 1]), f(L.R[l - 1]),
                                        i64(L.lo[l - 1]), L.n[l - 1], f(L.mu[l]), f(L.var[l]),
                                        f(L.R[l]), i64(L.lo[l]), L.n[l], (int)d, (int)F);
    SSA_TRY(launch_status("tree_level_kernel"));
  }
  return SSA_OK;
}

extern "C" int ssa_tree_descend(const void* tree, const float* q, const int64_t* q_pos, int64_t BH,
                                int64_t Q, int64_t nb, int64_t d, int64_t F, int64_t top_cap,
                                int64_t W, int64_t top_c, float beta, int32_t* sel,
                                ssa_stream_t stream) {
  using namespace ssa;
  SSA_REQUIRE(tree && q && sel, SSA_ERR_INVALID, "tree_descend: NULL pointer argument");
  SSA_REQUIRE(BH > 0 && Q > 0 && nb > 0, SSA_ERR_INVALID, "tree_descend: sizes must be positive");
  SSA_REQUIRE(BH < 65536 && Q < (1ll << 31), SSA_ERR_UNSUPPORTED, "tree_descend: grid too large");
  SSA_REQUIRE(d > 0 && d <= kTreeMaxD && d % 4 == 0, SSA_ERR_UNSUPPORTED,
              "tree_descend: head_dim must be a multiple of 4 up to %d", kTreeMaxD);
  SSA_REQUIRE(F >= 2 && F <= kTreeMaxF && top_cap >= 1 && top_cap <= kTreeMaxTop,
              SSA_ERR_UNSUPPORTED, "tree_descend: need 2 <= F <= %d and 1 <= top_cap <= %d",
              kTreeMaxF, kTreeMaxTop);
  SSA_REQUIRE(W >= 1 && W <= kTreeMaxW && W * F <= 1024 && top_c >= 1, SSA_ERR_UNSUPPORTED,
              "tree_descend: need 1 <= W <= %d, W*F <= 1024 and top_c >= 1", kTreeMaxW);
  SSA_REQUIRE(aligned16(tree) && aligned16(q), SSA_ERR_INVALID,
              "tree_descend: tree and q must be 16-byte aligned");
  TreeArgs a;
  SSA_REQUIRE(tree_layout(BH, nb, d, F, top_cap, &a.L), SSA_ERR_UNSUPPORTED,
              "tree_descend: more than %d levels", kTreeMaxLevels);
  a.tree = static_cast<const char*>(tree);
  a.q = q;
  a.q_pos = q_pos;
  a.BH = BH;
  a.Q = Q;
  a.d = (int)d;
  a.F = (int)F;
  a.W = (int)W;
  a.tc = (int)(top_c < W ? top_c : W);
  a.half_beta = 0.5 * (double)beta;
  a.sel = sel;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 g((unsigned)Q, (unsigned)BH);
  const int64_t c = W * F;
  if (c <= 64) tree_descend_kernel<1><<<g, 64, 0, st>>>(a);
  else if (c <= 128) tree_descend_kernel<2><<<g, 64, 0, st>>>(a);
  else if (c <= 256) tree_descend_kernel<4><<<g, 64, 0, st>>>(a);
  else if (c <= 512) tree_descend_kernel<8><<<g, 64, 0, st>>>(a);
  else tree_descend_kernel<16><<<g, 64, 0, st>>>(a);
  return launch_status("tree_descend_kernel");
}

extern "C" int ssa_tree_pack(const int32_t* sel, int64_t rows, int64_t nb, int64_t tc,
                             int64_t local, int32_t* kv_num, int32_t* kv_idx, int64_t W,
                             ssa_stream_t stream) {
  using namespace ssa;
  SSA_REQUIRE(rows >= 0 && rows <= 0x7fffffff && nb >= 1 && rows % nb == 0, SSA_ERR_INVALID,
              "tree_pack: rows=%lld must be a multiple of nb=%lld", (long long)rows, (long long)nb);
  SSA_REQUIRE(tc >= 0 && local >= 0, SSA_ERR_INVALID, "tree_pack: tc and local must be >= 0");
  const int64_t win = (local < nb - 1 ? local : nb - 1) + 1;
  SSA_REQUIRE(tc + win <= kTreePackMax, SSA_ERR_UNSUPPORTED,
              "tree_pack: tc + min(local, nb - 1) + 1 = %lld exceeds %d", (long long)(tc + win),
              kTreePackMax);
  SSA_REQUIRE(W >= tc + win, SSA_ERR_INVALID, "tree_pack: W=%lld < tc + min(local, nb - 1) + 1",
              (long long)W);
  if (rows == 0) return SSA_OK;
  SSA_REQUIRE(kv_num != nullptr && kv_idx != nullptr && (tc == 0 || sel != nullptr),
              SSA_ERR_INVALID, "tree_pack: NULL pointer argument");
  tree_pack_kernel<<<(unsigned)rows, 64, 0, static_cast<hipStream_t>(stream)>>>(
      sel, nb, (int)tc, local, kv_num, kv_idx, W);
  return launch_status("tree_pack_kernel");
}
