// Cumulant router: scores every (row, candidate key block) pair, then selects the top-keep
// candidates per row, merges the local window and emits compact ascending block lists.
//
// Stage 1 (route_score_kernel): a 64-row x 64-candidate tile per workgroup. Rows of one key head
//   (its Hq/Hkv query heads x the query blocks of the current chunk) share the candidates'
//   mu / var / m3, which are staged once per tile in LDS. Inner products accumulate in fp64 from
//   the fp32 operands (so each score is the correctly rounded value of the reference's formula up
//   to fp64 noise) and the fp32 score is assembled in the reference's evaluation order. Scores
//   are stored as order-preserving uint32 keys in the workspace.
// Stage 2 (route_select_kernel): one 256-thread workgroup per row. An 8-bit-digit radix select
//   finds the keep-th largest key T; keys > T are taken, and keys == T in increasing block order
//   until keep is reached (ties -> lowest block index). The selection, the own block and its
//   `local` predecessors are OR-ed into an LDS bitmap that is compacted in ascending order.
//   With at most 1024 key blocks, route_select_small_kernel does the same with one wave per row;
//   with at most 64 (no pooling, no m3) route_rows_small_kernel scores and selects in one pass.
//
// Reference: ssa/ssa_kernel.py:45-57 (block_route), :92-118 (block_route_budget),
// ssa/gemma_ssa.py:99-131 (_selection_mask).
#include <math.h>

#include <type_traits>

#include "common.h"
#include "select.h"

namespace ssa {
namespace {

constexpr int kTile = 64;       // rows and candidates per score tile
constexpr int kDK = 32;         // head-dim chunk staged in LDS
constexpr int kSelThreads = 256;
constexpr int kMaxNbk = 65536;  // bitmap capacity of the select kernel
constexpr int kCacheKeys = 8192;
constexpr int kCand = 2048;        // candidate capacity of the filtered select
constexpr int kFilterMin = 2048;   // rows with more candidates than this are filtered first

struct RouteGeom {
  int mode;
  int64_t Hq, Hkv, G;
  int64_t nbq;       // query rows per head (whole problem)
  int64_t nbk;       // key blocks
  int64_t i0, ni;    // current chunk of query rows [i0, i0+ni)
  int64_t query_pos;
  int64_t block;
  int64_t top_c;
  float budget_frac;
  int64_t local;
  int64_t pool;  // scored candidates per key block (sub-blocks max-pooled to the block; 1 = none)
  int rows_dt;   // element type of the query rows: SSA_F32, SSA_F16 or SSA_BF16 (exact in fp32)
};

// Element idx of the query rows as fp32 (16-bit types convert exactly).
__device__ inline float load_row(const void* rows, int64_t idx, int dt) {
  if (dt == SSA_F32) return static_cast<const float*>(rows)[idx];
  const unsigned short u = static_cast<const unsigned short*>(rows)[idx];
  if (dt == SSA_BF16) return __uint_as_float((unsigned int)u << 16);
  return (float)__builtin_bit_cast(_Float16, u);
}

// Number of candidates of query row i: budget -> c < i, flat -> c <= i, query -> complete blocks.
__host__ __device__ inline int64_t row_cmax(const RouteGeom& g, int64_t i) {
  int64_t c;
  if (g.mode == SSA_ROUTE_BUDGET) c = i;
  else if (g.mode == SSA_ROUTE_FLAT) c = i + 1;
  else if (g.mode == SSA_ROUTE_STARTED) c = (g.query_pos + i) / g.block + 1;
  else c = (g.query_pos + i + 1) / g.block;
  if (c > g.nbk) c = g.nbk;
  return c < 0 ? 0 : c;
}

// scored candidates of row i (sub-block units)
__host__ __device__ inline int64_t row_cmax_s(const RouteGeom& g, int64_t i) {
  return row_cmax(g, i) * g.pool;
}

__host__ __device__ inline int64_t row_own(const RouteGeom& g, int64_t i) {
  return g.mode == SSA_ROUTE_QUERY || g.mode == SSA_ROUTE_STARTED ? (g.query_pos + i) / g.block
                                                                  : i;
}

// keep count before clipping to the candidate count. Budget: ceil(fp32(frac) * nvis) in fp32,
// clamped to >= 1 (ssa/ssa_kernel.py:105-106, ssa/gemma_ssa.py:115-118).
__host__ __device__ inline int64_t row_keep(const RouteGeom& g, int64_t cmax) {
  if (g.mode == SSA_ROUTE_FLAT || g.top_c >= 0) return g.top_c;
  float prod = g.budget_frac * (float)cmax;
  int64_t k = (int64_t)ceilf(prod);
  return k < 1 ? 1 : k;
}

template <bool EDGE, int RT>
__global__ __launch_bounds__(256) void route_score_kernel(
    const void* __restrict__ rows, const float* __restrict__ mu, const float* __restrict__ var,
    const float* __restrict__ m3, RouteGeom g, int d, float coef2, float coef3,
    unsigned int* __restrict__ keys, int64_t row_tiles, int64_t cand_tiles) {
  // operands staged as fp64 (converted once per element, not once per use)
  // RT rows x kTile candidates per workgroup; a thread owns RA = RT/16 rows x 4 candidates
  constexpr int DK = 16;
  constexpr int RA = RT / 16;
  __shared__ double Qs[DK][RT + 1];
  __shared__ double Q2s[DK][RT + 1];
  __shared__ double Ms[DK][kTile + 1];
  __shared__ double Vs[DK][kTile + 1];
  __shared__ double Q3s[EDGE ? DK : 1][RT + 1];
  __shared__ double M3s[EDGE ? DK : 1][kTile + 1];

  const int64_t bk = blockIdx.y;  // b * Hkv + kvh
  const int64_t b = bk / g.Hkv, kvh = bk % g.Hkv;
  const int64_t rt = blockIdx.x / cand_tiles, ct = blockIdx.x % cand_tiles;
  const int64_t R = g.G * g.ni;  // rows of this key head in the chunk
  const int64_t r0 = rt * RT;
  const int64_t c0 = ct * kTile;
  if (r0 >= R) return;
  int64_t r_last = r0 + RT - 1 < R ? r0 + RT - 1 : R - 1;
  const int64_t imax = (r0 / g.ni != r_last / g.ni) ? g.i0 + g.ni - 1 : g.i0 + r_last % g.ni;
  if (c0 >= row_cmax_s(g, imax)) return;  // uniform: no row of the tile has these candidates
  const int64_t nbs = g.nbk * g.pool;     // scored candidates per key row

  const int tid = threadIdx.x;
  const int tr = tid / 16, tc = tid % 16;
  double e1[RA][4], e2[RA][4], e3[EDGE ? RA : 1][EDGE ? 4 : 1];
#pragma unroll
  for (int a = 0; a < RA; ++a)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      e1[a][c] = 0.0;
      e2[a][c] = 0.0;
      if constexpr (EDGE) e3[a][c] = 0.0;
    }

  const float* kv_mu = mu + (bk * nbs) * d;
  const float* kv_var = var ? var + (bk * nbs) * d : nullptr;
  const float* kv_m3 = EDGE ? m3 + (bk * nbs) * d : nullptr;
  // element offset of each tile row in `rows` (-1: past the chunk), computed once
  __shared__ int64_t row_off[RT];
  if (tid < RT) {
    const int64_t r = r0 + tid;
    int64_t off = -1;
    if (r < R) {
      const int64_t h = kvh * g.G + r / g.ni;
      const int64_t i = g.i0 + r % g.ni;
      off = ((b * g.Hq + h) * g.nbq + i) * d;
    }
    row_off[tid] = off;
  }

  for (int k0 = 0; k0 < d; k0 += DK) {
    __syncthreads();
    for (int idx = tid; idx < RT * DK; idx += 256) {
      const int rr = idx / DK, kk = idx % DK;
      const bool kin = k0 + kk < d;
      float q = 0.0f;
      const int64_t roff = row_off[rr];
      if (roff >= 0 && kin) q = load_row(rows, roff + k0 + kk, g.rows_dt);
      const float q2 = q * q;  // rounded to fp32 like the reference's elementwise products
      Qs[kk][rr] = (double)q;
      Q2s[kk][rr] = (double)q2;
      if constexpr (EDGE) Q3s[kk][rr] = (double)(q2 * q);
    }
    for (int idx = tid; idx < kTile * DK; idx += 256) {
      const int rr = idx / DK, kk = idx % DK;
      const bool kin = k0 + kk < d;
      const int64_t c = c0 + rr;
      float m = 0.0f, v = 0.0f, t = 0.0f;
      if (c < nbs && kin) {
        m = kv_mu[c * d + k0 + kk];
        if (kv_var) v = kv_var[c * d + k0 + kk];
        if constexpr (EDGE) t = kv_m3[c * d + k0 + kk];
      }
      Ms[kk][rr] = (double)m;
      Vs[kk][rr] = (double)v;
      if constexpr (EDGE) M3s[kk][rr] = (double)t;
    }
    __syncthreads();
    const int kend = d - k0 < DK ? d - k0 : DK;
    for (int kk = 0; kk < kend; ++kk) {
      double qd[RA], q2d[RA], md[4], vd[4];
#pragma unroll
      for (int a = 0; a < RA; ++a) {
        qd[a] = Qs[kk][tr + 16 * a];
        q2d[a] = Q2s[kk][tr + 16 * a];
      }
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        md[a] = Ms[kk][tc + 16 * a];
        vd[a] = Vs[kk][tc + 16 * a];
      }
#pragma unroll
      for (int a = 0; a < RA; ++a)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          e1[a][c] = fma(qd[a], md[c], e1[a][c]);
          e2[a][c] = fma(q2d[a], vd[c], e2[a][c]);
        }
      if constexpr (EDGE) {
        double q3d[RA], td[4];
#pragma unroll
        for (int a = 0; a < RA; ++a) q3d[a] = Q3s[kk][tr + 16 * a];
#pragma unroll
        for (int a = 0; a < 4; ++a) td[a] = M3s[kk][tc + 16 * a];
#pragma unroll
        for (int a = 0; a < RA; ++a)
#pragma unroll
          for (int c = 0; c < 4; ++c) e3[a][c] = fma(q3d[a], td[c], e3[a][c]);
      }
    }
  }

#pragma unroll
  for (int a = 0; a < RA; ++a) {
    const int64_t r = r0 + tr + 16 * a;
    if (r >= R) continue;
    const int64_t h = kvh * g.G + r / g.ni;
    const int64_t il = r % g.ni;
    const int64_t cmax = row_cmax_s(g, g.i0 + il);
    unsigned int* krow = keys + ((b * g.Hq + h) * g.ni + il) * nbs;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int64_t cand = c0 + tc + 16 * c;
      if (cand >= cmax) continue;
      // r = E1 + coef2*E2 (+ coef3*E3), each product term rounded to fp32 as torch does
      // explicit _rn ops: no FMA contraction, so the rounding matches torch's mul then add
      float s = __fadd_rn((float)e1[a][c], __fmul_rn(coef2, (float)e2[a][c]));
      if constexpr (EDGE) s = __fadd_rn(s, __fmul_rn(coef3, (float)e3[a][c]));
      krow[cand] = score_key(s);
    }
  }
}

// Few-row variant (R <= 16 rows per key head, e.g. a decode step): thread t scores candidate
// c0 + t / RP for row t % RP (RP = R rounded up to a power of two), so no work is spent on the
// empty rows of a 64-row tile. Same fp64 accumulation order over the head dim and the same
// fp32 assembly as route_score_kernel.
template <bool EDGE>
__global__ __launch_bounds__(256) void route_score_rows_kernel(
    const void* __restrict__ rows, const float* __restrict__ mu, const float* __restrict__ var,
    const float* __restrict__ m3, RouteGeom g, int d, float coef2, float coef3,
    unsigned int* __restrict__ keys, int rp_log2) {
  constexpr int kMaxR = 16;
  const int RP = 1 << rp_log2;
  const int CPB = 256 >> rp_log2;  // candidates per workgroup
  __shared__ float Qs[kMaxR][kDK + 1];
  __shared__ float Q2s[kMaxR][kDK + 1];
  __shared__ float Q3s[EDGE ? kMaxR : 1][kDK + 1];
  __shared__ float Ms[256][kDK + 1];
  __shared__ float Vs[256][kDK + 1];
  __shared__ float M3s[EDGE ? 256 : 1][kDK + 1];

  const int64_t bk = blockIdx.y;  // b * Hkv + kvh
  const int64_t b = bk / g.Hkv, kvh = bk % g.Hkv;
  const int64_t R = g.G * g.ni;
  const int64_t c0 = (int64_t)blockIdx.x * CPB;
  if (c0 >= row_cmax_s(g, g.i0 + g.ni - 1)) return;  // uniform: beyond every row's candidates
  const int64_t nbs = g.nbk * g.pool;
  const int tid = threadIdx.x;
  const int r = tid & (RP - 1);
  const int cl = tid >> rp_log2;
  const int64_t c = c0 + cl;

  const float* kv_mu = mu + (bk * nbs) * d;
  const float* kv_var = var ? var + (bk * nbs) * d : nullptr;
  const float* kv_m3 = EDGE ? m3 + (bk * nbs) * d : nullptr;
  // per row of the tile (once, not per element: 64-bit divisions are long instruction sequences)
  // the element offset of its query vector (-1: past the chunk), its key buffer and candidates
  __shared__ int64_t row_off[kMaxR], row_key[kMaxR], row_cm[kMaxR];
  if (tid < kMaxR) {
    int64_t off = -1, kofs = 0, cm = 0;
    if (tid < R) {
      const int64_t h = kvh * g.G + tid / g.ni;
      const int64_t il = tid % g.ni;
      off = ((b * g.Hq + h) * g.nbq + g.i0 + il) * d;
      kofs = ((b * g.Hq + h) * g.ni + il) * nbs;
      cm = row_cmax_s(g, g.i0 + il);
    }
    row_off[tid] = off;
    row_key[tid] = kofs;
    row_cm[tid] = cm;
  }
  double e1 = 0.0, e2 = 0.0, e3 = 0.0;
  for (int k0 = 0; k0 < d; k0 += kDK) {
    __syncthreads();
    for (int idx = tid; idx < kMaxR * kDK; idx += 256) {
      const int rr = idx / kDK, kk = idx % kDK;
      float q = 0.0f;
      const int64_t roff = row_off[rr];
      if (roff >= 0 && k0 + kk < d) q = load_row(rows, roff + k0 + kk, g.rows_dt);
      const float q2 = q * q;
      Qs[rr][kk] = q;
      Q2s[rr][kk] = q2;
      if constexpr (EDGE) Q3s[rr][kk] = q2 * q;
    }
    for (int idx = tid; idx < CPB * kDK; idx += 256) {
      const int cc = idx / kDK, kk = idx % kDK;
      const int64_t cand = c0 + cc;
      float m = 0.0f, v = 0.0f, t = 0.0f;
      if (cand < nbs && k0 + kk < d) {
        m = kv_mu[cand * d + k0 + kk];
        if (kv_var) v = kv_var[cand * d + k0 + kk];
        if constexpr (EDGE) t = kv_m3[cand * d + k0 + kk];
      }
      Ms[cc][kk] = m;
      Vs[cc][kk] = v;
      if constexpr (EDGE) M3s[cc][kk] = t;
    }
    __syncthreads();
    const int kend = d - k0 < kDK ? d - k0 : kDK;
    for (int kk = 0; kk < kend; ++kk) {
      e1 = fma((double)Qs[r][kk], (double)Ms[cl][kk], e1);
      e2 = fma((double)Q2s[r][kk], (double)Vs[cl][kk], e2);
      if constexpr (EDGE) e3 = fma((double)Q3s[r][kk], (double)M3s[cl][kk], e3);
    }
  }
  if (r >= R) return;
  if (c >= row_cm[r]) return;
  float s = __fadd_rn((float)e1, __fmul_rn(coef2, (float)e2));
  if constexpr (EDGE) s = __fadd_rn(s, __fmul_rn(coef3, (float)e3));
  keys[row_key[r] + c] = score_key(s);
}

// ---- certified scoring -------------------------------------------------------------------------
// With approximate (MFMA) keys, a select kernel certifies its selection: with e a bound on
// |approximate - exact| for every score of the row, and T~ the keep-th largest approximate score,
// the exact keep-th largest lies within e of T~, so a candidate scoring above T~ + 2e is in the
// exact top-keep and one below T~ - 2e is out; the candidates in between (the band) are rescored
// with the exact formula (fp64 sums, fp32 assembly as route_score_kernel) and the remaining
// places go to the best of them by (exact key, lowest block index) -- the exact router's
// selection. When the band holds exactly the remaining places (the usual case: the keep-th
// candidate alone), they are taken without rescoring.
// The approximation is one MFMA contraction of the rows' A = [q | c2 fl32(q*q) | c3 fl32(q*q*q)]
// against the candidates' B = [mu | var | m3] (route_score_mfma_kernel, n products per score).
// For a row and a 64-candidate tile the score kernel stores
//   emag = sum_t |A_t| max_c |B_t,c| + 2^-56 sum_t (|A_t| + max|B_t|)
// (norms from fp32 squares; their relative error, below d 2^-24, is covered by the margin below);
// the select takes M = the largest emag over the row's tiles and
//   e = ecoef (1 + 2^-10) M + 2^-100,  ecoef = 1.03 (3n + 16) 2^-23 + 2^-14:
// the 3n bf16 products are exact and their fp32 sum, in any order with each addition rounded or
// truncated (2^-23 per operation), is within 3n 2^-23 of the sum of their magnitudes (at most
// 1.02 sum|a_k b_k|); the bf16 split and the dropped lo.lo products add under 3.1 2^-16
// sum|a_k b_k|; the pre-multiplied c2 q^2, c3 q^3 and the exact score's own fp32 roundings a few
// 2^-24 sum|a_k b_k|, inside the 16; Cauchy-Schwarz bounds sum|a_k b_k| by sum_t |A_t||B_t|.
// Inputs or products flushed below 2^-126 move the sum by less than n 2^-126 (max|A| + max|B|)
// + n 2^-126, covered by the 2^-56 term and 2^-100. A non-finite bound or threshold makes every
// candidate uncertain.
struct CertArgs {
  int on;                      // the keys are MFMA approximations to certify
  const void* rows;            // (B, Hq, nbq, d) query rows of type g.rows_dt
  const float* mu;
  const float* var;            // may be NULL (coef2 = 0)
  const float* m3;             // may be NULL
  const float* emag;           // (chunk rows, ntile) error magnitude per row and candidate tile
  const unsigned int* tmax;    // (chunk rows, ntile) largest key per row and tile, or NULL
  int64_t ntile;
  int d;
  double ecoef;                // e = ecoef (1 + 2^-10) M + 2^-100 (M: the row's largest emag)
  float coef2, coef3;
};

constexpr int kNormTile = 64;  // candidates (sub-block units) per score tile of emag / tmax
constexpr int kBand = 512;     // capacity of a row's certificate band (larger: rescore the row)
constexpr int kMaxQReg = 8;    // head dims per lane in the exact rescoring (d <= 512)
// The select kernels are instantiated for QR = ceil(d / 64) head dims per lane (1, 2, 4, 8).
constexpr int kMaxTiles = kMaxNbk / kNormTile;  // tile maxima of a row staged by the select

// Bytes per routed row of the certified router's workspace: the keys, then emag and tmax.
inline size_t route_row_bytes(int64_t nbs) {
  return (size_t)nbs * 4u + (size_t)((nbs + kNormTile - 1) / kNormTile) * 8u;
}
// The wave select's bookkeeping at the end of the workspace: its deferred-row list (4 bytes per
// routed row of a chunk) below kRouteTail bytes that hold one counter per chunk (the first
// kRouteCounters chunks; alignment slack included).
constexpr size_t kRouteTail = 512;
constexpr int kRouteCounters = 64;

// Approximate scores for the certified router: one MFMA contraction of the query rows
// A = [q | c2 fl32(q*q) | c3 fl32(q*q*q)] against the candidates' B = [mu | var | m3] (n = 2d, 3d
// with m3, d without var), each fp32 operand split into bf16 hi + lo parts (hi = bf16(x),
// lo = bf16(x - hi), |x - hi - lo| <= 2^-16 |x|) and a.b taken as hi.hi + hi.lo + lo.hi on
// v_mfma_f32_32x32x16_bf16 (the products are exact in fp32; dropping lo.lo and the split errors
// leave under 3.1 2^-16 |a||b|). A workgroup scores 64 rows x 64 candidates, each of its 4 waves a
// 32 x 32 block (lane l supplies A[l%32][8(l/32) .. +8] and B[8(l/32) .. +8][l%32] per 16 head
// dims; accumulator j of lane l is C[(j/4)*8 + (l/32)*4 + j%4][l%32]). Operands are staged in LDS
// 32 head dims at a time as bf16 rows of 40 (80 bytes: the 16 lanes of a ds_read_b128 phase, 16
// consecutive rows, cover the 64 banks once), a thread loading 8 consecutive head dims of one row
// and of one candidate (16-byte loads: d % 8 == 0, aligned operands). Same tile geometry and
// causal tile skip as route_score_kernel; the keys are stored in the same layout. Per row and
// tile it also stores emag (the certificate's error magnitude) and, with TMAX, the largest key
// over the row's candidates in the tile.
constexpr int kStageLd = 40;  // bf16 per staged row (32 head dims + 8 pad)

// hi / lo bf16 parts of 8 fp32 values, packed in pairs (element 2e in the low half of word e).
__device__ inline void split_bf16x8(const float (&x)[8], u32x4& hi, u32x4& lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const __bf16 h0 = (__bf16)x[2 * e], h1 = (__bf16)x[2 * e + 1];
    const __bf16 l0 = (__bf16)(x[2 * e] - (float)h0), l1 = (__bf16)(x[2 * e + 1] - (float)h1);
    hi[e] = (unsigned int)__builtin_bit_cast(unsigned short, h0) |
            ((unsigned int)__builtin_bit_cast(unsigned short, h1) << 16);
    lo[e] = (unsigned int)__builtin_bit_cast(unsigned short, l0) |
            ((unsigned int)__builtin_bit_cast(unsigned short, l1) << 16);
  }
}

template <bool EDGE, bool TMAX>
__global__ __launch_bounds__(256) void route_score_mfma_kernel(
    const void* __restrict__ rows, const float* __restrict__ mu, const float* __restrict__ var,
    const float* __restrict__ m3, RouteGeom g, int d, float coef2, float coef3,
    unsigned int* __restrict__ keys, float* __restrict__ emag, unsigned int* __restrict__ tmax,
    int64_t ntile, int64_t row_tiles, int64_t cand_tiles) {
  constexpr int KC = 32;
  // staging: A hi, A lo, B hi, B lo, [kTile][kStageLd] bf16 each; after the last contraction,
  // TMAX reuses it as a [kTile][kTile + 1] array of keys
  static_assert(4 * kTile * kStageLd * 2 >= kTile * (kTile + 1) * 4, "stage too small");
  __shared__ __attribute__((aligned(16))) unsigned short stage[4][kTile][kStageLd];
  __shared__ int64_t row_off[kTile];  // element offset of the tile's rows in `rows` (-1: none)
  __shared__ int64_t row_key[kTile];  // chunk row index (b*Hq + h)*ni + il of the tile's rows
  __shared__ int64_t row_cm[kTile];   // scored candidates of the tile's rows (0: none)
  __shared__ float sqa[3][kTile], sqb[3][kTile];  // squared norms per term: rows, candidates
  __shared__ unsigned int smax[kTile];

  const int64_t bk = blockIdx.y;  // b * Hkv + kvh
  const int64_t b = bk / g.Hkv, kvh = bk % g.Hkv;
  const int64_t rt = blockIdx.x / cand_tiles, ct = blockIdx.x % cand_tiles;
  const int64_t R = g.G * g.ni;
  const int64_t r0 = rt * kTile;
  const int64_t c0 = ct * kTile;
  if (r0 >= R) return;
  const int64_t r_last = r0 + kTile - 1 < R ? r0 + kTile - 1 : R - 1;
  const int64_t imax = (r0 / g.ni != r_last / g.ni) ? g.i0 + g.ni - 1 : g.i0 + r_last % g.ni;
  if (c0 >= row_cmax_s(g, imax)) return;  // uniform: no row of the tile has these candidates
  const int64_t nbs = g.nbk * g.pool;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wr = w & 1, wc = w >> 1;
  if (tid < kTile) {  // per-row geometry, once per tile (64-bit divisions)
    const int64_t r = r0 + tid;
    int64_t off = -1, lr = 0, cm = 0;
    if (r < R) {
      const int64_t h = kvh * g.G + r / g.ni;
      const int64_t il = r % g.ni;
      off = ((b * g.Hq + h) * g.nbq + g.i0 + il) * d;
      lr = (b * g.Hq + h) * g.ni + il;
      cm = row_cmax_s(g, g.i0 + il);
    }
    row_off[tid] = off;
    row_key[tid] = lr;
    row_cm[tid] = cm;
  }
  if (tid < 3 * kTile) {
    sqa[tid / kTile][tid % kTile] = 0.0f;
    sqb[tid / kTile][tid % kTile] = 0.0f;
  }
  f32x16 acc;
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
  const int rr = tid >> 2, k8 = (tid & 3) * 8;  // staging: row / candidate rr, dims k8..k8+7
  for (int term = 0; term < (EDGE ? 3 : 2); ++term) {
    if (term == 1 && var == nullptr) continue;  // centroid routing: no variance term
    const float* src = (term == 0 ? mu : term == 1 ? var : m3) + (bk * nbs) * d;
    const float cf = term == 0 ? 1.0f : term == 1 ? coef2 : coef3;
    float sa = 0.0f, sb = 0.0f;
    for (int k0 = 0; k0 < d; k0 += KC) {
      __syncthreads();
      const int64_t roff = row_off[rr];
      float q[8], bv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) q[e] = bv[e] = 0.0f;
      if (roff >= 0 && k0 + k8 < d) {
        if (g.rows_dt == SSA_F32) {
          const f32x4* pq =
              reinterpret_cast<const f32x4*>(static_cast<const float*>(rows) + roff + k0 + k8);
          const f32x4 x0 = pq[0], x1 = pq[1];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            q[e] = x0[e];
            q[4 + e] = x1[e];
          }
        } else {
          const u32x4 wq = *reinterpret_cast<const u32x4*>(
              static_cast<const unsigned short*>(rows) + roff + k0 + k8);
          unpack8(wq, q, g.rows_dt == SSA_BF16);
        }
      }
      const int64_t cand = c0 + rr;
      if (cand < nbs && k0 + k8 < d) {
        const f32x4* pb = reinterpret_cast<const f32x4*>(src + cand * d + k0 + k8);
        const f32x4 y0 = pb[0], y1 = pb[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          bv[e] = y0[e];
          bv[4 + e] = y1[e];
        }
      }
      float a[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        a[e] = q[e];
        if (term == 1) a[e] = cf * (q[e] * q[e]);
        else if (term == 2) a[e] = cf * ((q[e] * q[e]) * q[e]);
        sa = fmaf(a[e], a[e], sa);
        sb = fmaf(bv[e], bv[e], sb);
      }
      u32x4 ahi, alo, bhi, blo;
      split_bf16x8(a, ahi, alo);
      split_bf16x8(bv, bhi, blo);
      *reinterpret_cast<u32x4*>(&stage[0][rr][k8]) = ahi;
      *reinterpret_cast<u32x4*>(&stage[1][rr][k8]) = alo;
      *reinterpret_cast<u32x4*>(&stage[2][rr][k8]) = bhi;
      *reinterpret_cast<u32x4*>(&stage[3][rr][k8]) = blo;
      __syncthreads();
#pragma unroll
      for (int s = 0; s < KC / 16; ++s) {
        const int kk = s * 16 + (lane >> 5) * 8;
        const int ra = wr * 32 + (lane & 31), rb = wc * 32 + (lane & 31);
        const bf16x8 xah = *reinterpret_cast<const bf16x8*>(&stage[0][ra][kk]);
        const bf16x8 xal = *reinterpret_cast<const bf16x8*>(&stage[1][ra][kk]);
        const bf16x8 xbh = *reinterpret_cast<const bf16x8*>(&stage[2][rb][kk]);
        const bf16x8 xbl = *reinterpret_cast<const bf16x8*>(&stage[3][rb][kk]);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xah, xbh, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xah, xbl, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xal, xbh, acc, 0, 0, 0);
      }
    }
    // the 4 staging threads of row / candidate rr are adjacent lanes
    sa += __shfl_xor(sa, 1, 64);
    sa += __shfl_xor(sa, 2, 64);
    sb += __shfl_xor(sb, 1, 64);
    sb += __shfl_xor(sb, 2, 64);
    if ((tid & 3) == 0) {
      sqa[term][rr] = sa;
      sqb[term][rr] = sb;
    }
  }
  const int64_t cand = c0 + wc * 32 + (lane & 31);
  unsigned int mk[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int rl = wr * 32 + (j >> 2) * 8 + (lane >> 5) * 4 + (j & 3);
    mk[j] = 0u;
    if (cand >= row_cm[rl]) continue;  // past the row's candidates (or no row: 0)
    const unsigned int k = score_key(acc[j]);
    keys[row_key[rl] * nbs + cand] = k;
    mk[j] = k;
  }
  if constexpr (TMAX) {
    // row maxima: the tile's keys go to LDS as [row][candidate], 4 threads reduce each row
    unsigned int* red = reinterpret_cast<unsigned int*>(&stage[0][0][0]);
    __syncthreads();  // every wave is past its last contraction
#pragma unroll
    for (int j = 0; j < 16; ++j)
      red[(wr * 32 + (j >> 2) * 8 + (lane >> 5) * 4 + (j & 3)) * (kTile + 1) + wc * 32 +
          (lane & 31)] = mk[j];
    __syncthreads();
    const unsigned int* pr = red + (tid >> 2) * (kTile + 1) + (tid & 3) * 16;
    unsigned int mx = 0u;
#pragma unroll
    for (int e = 0; e < 16; ++e) mx = pr[e] > mx ? pr[e] : mx;
    unsigned int o = __shfl_xor(mx, 1, 64);
    mx = o > mx ? o : mx;
    o = __shfl_xor(mx, 2, 64);
    mx = o > mx ? o : mx;
    if ((tid & 3) == 0) smax[tid >> 2] = mx;
  }
  __syncthreads();
  if (w == 0) {
    float M[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      M[t] = sqb[t][lane];  // zero for candidates past nbs (staged as zeros)
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) M[t] = fmaxf(M[t], __shfl_xor(M[t], off, 64));
    }
    if (c0 < row_cm[lane]) {
      double mag = 0.0, nsum = 0.0;
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        const double a = sqrt((double)sqa[t][lane]), bb = sqrt((double)M[t]);
        mag += a * bb;
        nsum += a + bb;
      }
      mag += 0x1p-56 * nsum;
      float f = (float)mag;
      if ((double)f < mag) f = __uint_as_float(__float_as_uint(f) + 1u);  // round up (f >= 0)
      const int64_t lrow = row_key[lane];
      emag[lrow * ntile + ct] = f;
      if constexpr (TMAX) tmax[lrow * ntile + ct] = smax[lane];
    }
  }
}


// ---- operands split once per call ---------------------------------------------------------
// route_score_split_kernel reads the certified scoring's operands already split: for each query
// row of the chunk A = [q | c2 fl32(q*q) | c3 fl32(q*q*q)] and for each candidate of a key head
// B = [mu | var | m3] (the present terms, nt of them, concatenated: nk = nt*d values), as bf16 hi
// and lo parts (split_bf16x8, the same values route_score_mfma_kernel forms in every tile), with
// the fp32 squared norm of every term. route_split_kernel writes them, one wave per item, lane l
// taking 8 consecutive values at a time.
struct SplitOut {
  unsigned short* hi;  // (items, nk)
  unsigned short* lo;  // (items, nk)
  float* sq;           // (items, 3): squared norm of term slot t (absent slots 0)
};

// QROWS: items are the chunk's query rows (item lr = (b*Hq + h)*ni + il, read from `src` of type
// g.rows_dt and transformed per term); else the candidates of every key head (item bk*nbs + c,
// term t read from terms[t] as is).
template <bool QROWS>
__global__ __launch_bounds__(256) void route_split_kernel(const void* __restrict__ src,
                                                          const float* __restrict__ t0,
                                                          const float* __restrict__ t1,
                                                          const float* __restrict__ t2, RouteGeom g,
                                                          int d, int nt, float coef2, float coef3,
                                                          int64_t items, SplitOut o) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= items) return;
  const int nk = nt * d;
  int64_t off;  // element offset of the item's values
  if constexpr (QROWS) {
    const int64_t bh = item / g.ni, il = item % g.ni;  // bh = b*Hq + h
    off = (bh * g.nbq + g.i0 + il) * d;
  } else {
    off = item * d;
  }
  // term slot s -> operand: slot 0 q / mu, then var (if present), then m3 (if present)
  const float* terms[3] = {t0, t1, t2};
  float sq[3] = {0.0f, 0.0f, 0.0f};
  for (int j = lane * 8; j < nk; j += 64 * 8) {
    const int s = j / d, e0 = j % d;
    float x[8];
    if constexpr (QROWS) {
      float q[8];
      if (g.rows_dt == SSA_F32) {
        const f32x4* pq = reinterpret_cast<const f32x4*>(static_cast<const float*>(src) + off + e0);
        const f32x4 a0 = pq[0], a1 = pq[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          q[e] = a0[e];
          q[4 + e] = a1[e];
        }
      } else {
        const u32x4 wq =
            *reinterpret_cast<const u32x4*>(static_cast<const unsigned short*>(src) + off + e0);
        unpack8(wq, q, g.rows_dt == SSA_BF16);
      }
      const int term = s == 0 ? 0 : (t1 != nullptr && s == 1 ? 1 : 2);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[e] = q[e];
        if (term == 1) x[e] = coef2 * (q[e] * q[e]);
        else if (term == 2) x[e] = coef3 * ((q[e] * q[e]) * q[e]);
      }
    } else {
      const f32x4* pb = reinterpret_cast<const f32x4*>(terms[s] + off + e0);
      const f32x4 b0 = pb[0], b1 = pb[1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[e] = b0[e];
        x[4 + e] = b1[e];
      }
    }
    float a2 = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) a2 = fmaf(x[e], x[e], a2);
    sq[s] += a2;
    u32x4 hi, lo;
    split_bf16x8(x, hi, lo);
    *reinterpret_cast<u32x4*>(o.hi + item * nk + j) = hi;
    *reinterpret_cast<u32x4*>(o.lo + item * nk + j) = lo;
  }
#pragma unroll
  for (int t = 0; t < 3; ++t)
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) sq[t] += __shfl_xor(sq[t], m, 64);
  if (lane < 3) o.sq[item * 3 + lane] = lane == 0 ? sq[0] : lane == 1 ? sq[1] : sq[2];
}

// route_score_mfma_kernel on pre-split operands (route_split_kernel): the same tiles, products,
// keys, emag and tile maxima; the staging copies 16-byte runs of the bf16 parts (the
// concatenated terms as one contraction of nk values) instead of forming and splitting them.
template <bool TMAX>
__global__ __launch_bounds__(256) void route_score_split_kernel(
    SplitOut A, SplitOut Bs, RouteGeom g, int nk, unsigned int* __restrict__ keys,
    float* __restrict__ emag, unsigned int* __restrict__ tmax, int64_t ntile, int64_t row_tiles,
    int64_t cand_tiles) {
  constexpr int KC = 32;
  static_assert(4 * kTile * kStageLd * 2 >= kTile * (kTile + 1) * 4, "stage too small");
  __shared__ __attribute__((aligned(16))) unsigned short stage[4][kTile][kStageLd];
  __shared__ int64_t row_key[kTile];  // chunk row index (b*Hq + h)*ni + il of the tile's rows (-1: none)
  __shared__ int64_t row_cm[kTile];   // scored candidates of the tile's rows (0: none)
  __shared__ float sqa[3][kTile], sqb[3][kTile];  // squared norms per term: rows, candidates
  __shared__ unsigned int smax[kTile];

  const int64_t bk = blockIdx.y;  // b * Hkv + kvh
  const int64_t b = bk / g.Hkv, kvh = bk % g.Hkv;
  const int64_t rt = blockIdx.x / cand_tiles, ct = blockIdx.x % cand_tiles;
  const int64_t R = g.G * g.ni;
  const int64_t r0 = rt * kTile;
  const int64_t c0 = ct * kTile;
  if (r0 >= R) return;
  const int64_t r_last = r0 + kTile - 1 < R ? r0 + kTile - 1 : R - 1;
  const int64_t imax = (r0 / g.ni != r_last / g.ni) ? g.i0 + g.ni - 1 : g.i0 + r_last % g.ni;
  if (c0 >= row_cmax_s(g, imax)) return;  // uniform: no row of the tile has these candidates
  const int64_t nbs = g.nbk * g.pool;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wr = w & 1, wc = w >> 1;
  if (tid < kTile) {  // per-row geometry, once per tile (64-bit divisions)
    const int64_t r = r0 + tid;
    int64_t lr = -1, cm = 0;
    if (r < R) {
      const int64_t h = kvh * g.G + r / g.ni;
      const int64_t il = r % g.ni;
      lr = (b * g.Hq + h) * g.ni + il;
      cm = row_cmax_s(g, g.i0 + il);
    }
    row_key[tid] = lr;
    row_cm[tid] = cm;
  } else if (tid < 2 * kTile) {  // the norms, from the split pass
    const int t = tid - kTile;
    const int64_t r = r0 + t;
    int64_t lr = -1;
    if (r < R) lr = (b * g.Hq + kvh * g.G + r / g.ni) * g.ni + r % g.ni;
    const int64_t c = c0 + t;
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      sqa[s][t] = lr >= 0 ? A.sq[lr * 3 + s] : 0.0f;
      sqb[s][t] = c < nbs ? Bs.sq[(bk * nbs + c) * 3 + s] : 0.0f;
    }
  }
  f32x16 acc;
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
  const int rr = tid >> 2, k8 = (tid & 3) * 8;  // staging: row / candidate rr, values k8..k8+7
  const int64_t cand_s = c0 + rr;
  for (int k0 = 0; k0 < nk; k0 += KC) {
    __syncthreads();
    const int64_t lr = row_key[rr];
    u32x4 ah = {0u, 0u, 0u, 0u}, al = ah, bh = ah, bl = ah;
    if (k0 + k8 < nk) {
      if (lr >= 0) {
        ah = *reinterpret_cast<const u32x4*>(A.hi + lr * nk + k0 + k8);
        al = *reinterpret_cast<const u32x4*>(A.lo + lr * nk + k0 + k8);
      }
      if (cand_s < nbs) {
        bh = *reinterpret_cast<const u32x4*>(Bs.hi + (bk * nbs + cand_s) * nk + k0 + k8);
        bl = *reinterpret_cast<const u32x4*>(Bs.lo + (bk * nbs + cand_s) * nk + k0 + k8);
      }
    }
    *reinterpret_cast<u32x4*>(&stage[0][rr][k8]) = ah;
    *reinterpret_cast<u32x4*>(&stage[1][rr][k8]) = al;
    *reinterpret_cast<u32x4*>(&stage[2][rr][k8]) = bh;
    *reinterpret_cast<u32x4*>(&stage[3][rr][k8]) = bl;
    __syncthreads();
#pragma unroll
    for (int s = 0; s < KC / 16; ++s) {
      const int kk = s * 16 + (lane >> 5) * 8;
      const int ra = wr * 32 + (lane & 31), rb = wc * 32 + (lane & 31);
      const bf16x8 xah = *reinterpret_cast<const bf16x8*>(&stage[0][ra][kk]);
      const bf16x8 xal = *reinterpret_cast<const bf16x8*>(&stage[1][ra][kk]);
      const bf16x8 xbh = *reinterpret_cast<const bf16x8*>(&stage[2][rb][kk]);
      const bf16x8 xbl = *reinterpret_cast<const bf16x8*>(&stage[3][rb][kk]);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xah, xbh, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xah, xbl, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xal, xbh, acc, 0, 0, 0);
    }
  }
  const int64_t cand = c0 + wc * 32 + (lane & 31);
  unsigned int mk[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int rl = wr * 32 + (j >> 2) * 8 + (lane >> 5) * 4 + (j & 3);
    mk[j] = 0u;
    if (cand >= row_cm[rl]) continue;  // past the row's candidates (or no row: 0)
    const unsigned int k = score_key(acc[j]);
    keys[row_key[rl] * nbs + cand] = k;
    mk[j] = k;
  }
  if constexpr (TMAX) {
    // row maxima: the tile's keys go to LDS as [row][candidate], 4 threads reduce each row
    unsigned int* red = reinterpret_cast<unsigned int*>(&stage[0][0][0]);
    __syncthreads();  // every wave is past its last contraction
#pragma unroll
    for (int j = 0; j < 16; ++j)
      red[(wr * 32 + (j >> 2) * 8 + (lane >> 5) * 4 + (j & 3)) * (kTile + 1) + wc * 32 +
          (lane & 31)] = mk[j];
    __syncthreads();
    const unsigned int* pr = red + (tid >> 2) * (kTile + 1) + (tid & 3) * 16;
    unsigned int mx = 0u;
#pragma unroll
    for (int e = 0; e < 16; ++e) mx = pr[e] > mx ? pr[e] : mx;
    unsigned int o = __shfl_xor(mx, 1, 64);
    mx = o > mx ? o : mx;
    o = __shfl_xor(mx, 2, 64);
    mx = o > mx ? o : mx;
    if ((tid & 3) == 0) smax[tid >> 2] = mx;
  }
  __syncthreads();
  if (w == 0) {
    float M[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      M[t] = sqb[t][lane];  // zero for candidates past nbs
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) M[t] = fmaxf(M[t], __shfl_xor(M[t], off, 64));
    }
    if (c0 < row_cm[lane]) {
      double mag = 0.0, nsum = 0.0;
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        const double a = sqrt((double)sqa[t][lane]), bb = sqrt((double)M[t]);
        mag += a * bb;
        nsum += a + bb;
      }
      mag += 0x1p-56 * nsum;
      float f = (float)mag;
      if ((double)f < mag) f = __uint_as_float(__float_as_uint(f) + 1u);  // round up (f >= 0)
      const int64_t lrow = row_key[lane];
      emag[lrow * ntile + ct] = f;
      if constexpr (TMAX) tmax[lrow * ntile + ct] = smax[lane];
    }
  }
}

// route_score_split_kernel's products for long rows with the row operands held in registers: a
// workgroup takes a strip of kStripRows chunk rows (wave w: rows 32w .. 32w+31, lane l holding
// A[row 32w + l%32][16 ks + 8 (l/32) .. +8] for every 16-value step ks of the contraction, hi and
// lo parts) and walks a segment of kStripSeg candidate tiles, staging each tile's 64 candidates
// (hi and lo rows of NK values, padded to NK + 8: a ds_read_b128 phase of 16 lanes covers the 64
// banks once) in LDS, the next tile's loads in flight in registers meanwhile; per tile every
// wave forms its 32 x 64 block as two 32 x 32 MFMA blocks with the same operands and the same
// product order as route_score_split_kernel, so the keys, emag and tile maxima are the same bits.
// The key operands are then read once per 128-row strip instead of once per 64-row tile (C5: 1.2
// instead of 8.9 GB per route). Contractions of 64 or 128 values (NKS 4, 8: the row fragments
// and two waves per SIMD fit the registers). Grid: segment-major (block x = segment * nstrips +
// strip): the strips running together share the segment's candidate tiles in L2.
constexpr int kStripRows = 128;
constexpr int kStripSeg = 16;

template <int NKS, bool TMAX>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void route_score_strip_kernel(
    SplitOut A, SplitOut Bs, RouteGeom g, unsigned int* __restrict__ keys,
    float* __restrict__ emag, unsigned int* __restrict__ tmax, int64_t ntile, int64_t nstrips) {
  constexpr int NK = NKS * 16;
  constexpr int LD = NK + 8;
  constexpr int kPieces = kTile * NK / 8;  // 16-byte pieces per part of a staged tile
  __shared__ __attribute__((aligned(16))) unsigned short sb[2][kTile][LD];
  __shared__ int64_t row_key[kStripRows];  // chunk row index of the strip's rows (-1: none)
  __shared__ int64_t row_cm[kStripRows];   // scored candidates of the strip's rows (0: none)
  __shared__ double sroot[3];              // the tile's sqrt(largest candidate norm) per term

  const int64_t bk = blockIdx.y;  // b * Hkv + kvh
  const int64_t b = bk / g.Hkv, kvh = bk % g.Hkv;
  const int64_t seg = blockIdx.x / nstrips, st = blockIdx.x % nstrips;
  const int64_t R = g.G * g.ni;
  const int64_t r0 = st * kStripRows;
  if (r0 >= R) return;
  const int64_t r_last = r0 + kStripRows - 1 < R ? r0 + kStripRows - 1 : R - 1;
  const int64_t imax = (r0 / g.ni != r_last / g.ni) ? g.i0 + g.ni - 1 : g.i0 + r_last % g.ni;
  const int64_t cmax = row_cmax_s(g, imax);
  const int64_t ct0 = seg * kStripSeg;
  if (ct0 * kTile >= cmax) return;  // uniform: no row of the strip has these candidates
  const int64_t ct_end = (cmax + kTile - 1) / kTile;
  const int64_t ct1 = ct0 + kStripSeg < ct_end ? ct0 + kStripSeg : ct_end;
  const int64_t nbs = g.nbk * g.pool;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (tid < kStripRows) {
    const int64_t r = r0 + tid;
    int64_t lr = -1, cm = 0;
    if (r < R) {
      const int64_t h = kvh * g.G + r / g.ni;
      const int64_t il = r % g.ni;
      lr = (b * g.Hq + h) * g.ni + il;
      cm = row_cmax_s(g, g.i0 + il);
    }
    row_key[tid] = lr;
    row_cm[tid] = cm;
  }
  __syncthreads();
  const int ra = w * 32 + (lane & 31);
  const int64_t lra = row_key[ra];
  const int64_t cma = row_cm[ra];
  bf16x8 ah[NKS], al[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    u32x4 h = {0u, 0u, 0u, 0u}, l = h;
    if (lra >= 0) {
      const int64_t off = lra * NK + ks * 16 + (lane >> 5) * 8;
      h = *reinterpret_cast<const u32x4*>(A.hi + off);
      l = *reinterpret_cast<const u32x4*>(A.lo + off);
    }
    ah[ks] = __builtin_bit_cast(bf16x8, h);
    al[ks] = __builtin_bit_cast(bf16x8, l);
  }
  double sa[3];  // square roots of the row's term norms (emag)
#pragma unroll
  for (int t = 0; t < 3; ++t) sa[t] = sqrt((double)(lra >= 0 ? A.sq[lra * 3 + t] : 0.0f));
  // rows of this lane's accumulator entries j: 32w + (j/4)*8 + (l/32)*4 + j%4
  const int rbase = w * 32 + (lane >> 5) * 4;
  // Full tiles: a whole strip of one head has consecutive chunk rows lr0 + rl, and a tile whose
  // candidates all lie below the strip's first row's candidate count (the counts grow along the
  // rows) holds every candidate for every row: its key rows are addressed from lr0 alone and
  // need no bounds checks.
  const bool contig = r0 + kStripRows <= R && r0 / g.ni == (r0 + kStripRows - 1) / g.ni;
  const int64_t lr0 = (b * g.Hq + kvh * g.G + r0 / g.ni) * g.ni + r0 % g.ni;
  const int64_t cm_first = contig ? row_cmax_s(g, g.i0 + r0 % g.ni) : 0;

  // the next tile's pieces and candidate norms (lane = candidate) are loaded into registers
  // while the current tile is multiplied
  constexpr int kPer = 2 * kPieces / 256;
  u32x4 pf[kPer];
  float pn[3];
  const auto fetch = [&](int64_t c0) {
    if (c0 + kTile <= nbs) {  // the tile's hi and lo rows: two contiguous 64 x NK blocks
      const unsigned short* ph = Bs.hi + (bk * nbs + c0) * NK;
      const unsigned short* pl = Bs.lo + (bk * nbs + c0) * NK;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int p = tid + 256 * i;
        pf[i] = *reinterpret_cast<const u32x4*>((p < kPieces ? ph : pl) + (p % kPieces) * 8);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int p = tid + 256 * i;
        const int part = p / kPieces, rem = p % kPieces;
        const int64_t c = c0 + rem / (NK / 8);
        pf[i] = u32x4{0u, 0u, 0u, 0u};
        if (c < nbs)
          pf[i] = *reinterpret_cast<const u32x4*>((part ? Bs.lo : Bs.hi) + (bk * nbs + c) * NK +
                                                  (rem % (NK / 8)) * 8);
      }
    }
    const int64_t cl = c0 + lane;
#pragma unroll
    for (int t = 0; t < 3; ++t) pn[t] = cl < nbs ? Bs.sq[(bk * nbs + cl) * 3 + t] : 0.0f;
  };
  fetch(ct0 * kTile);
  for (int64_t ct = ct0; ct < ct1; ++ct) {
    const int64_t c0 = ct * kTile;
    __syncthreads();  // every wave is done with the previous tile
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int p = tid + 256 * i;
      const int part = p / kPieces, rem = p % kPieces;
      *reinterpret_cast<u32x4*>(&sb[part][rem / (NK / 8)][(rem % (NK / 8)) * 8]) = pf[i];
    }
    // sqrt of the tile's largest candidate norm per term, for emag: wave t (< 3) reduces term t
    if (w < 3) {
      float mt = w == 0 ? pn[0] : w == 1 ? pn[1] : pn[2];
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) mt = fmaxf(mt, __shfl_xor(mt, off, 64));
      if (lane == 0) sroot[w] = sqrt((double)mt);
    }
    __syncthreads();  // the tile and its roots are staged
    if (ct + 1 < ct1) fetch(c0 + kTile);
    f32x16 acc0, acc1;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      acc0[j] = 0.0f;
      acc1[j] = 0.0f;
    }
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int kk = ks * 16 + (lane >> 5) * 8;
      const bf16x8 bh0 = *reinterpret_cast<const bf16x8*>(&sb[0][lane & 31][kk]);
      const bf16x8 bl0 = *reinterpret_cast<const bf16x8*>(&sb[1][lane & 31][kk]);
      const bf16x8 bh1 = *reinterpret_cast<const bf16x8*>(&sb[0][32 + (lane & 31)][kk]);
      const bf16x8 bl1 = *reinterpret_cast<const bf16x8*>(&sb[1][32 + (lane & 31)][kk]);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[ks], bh0, acc0, 0, 0, 0);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[ks], bl0, acc0, 0, 0, 0);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[ks], bh0, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[ks], bh1, acc1, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[ks], bl1, acc1, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[ks], bh1, acc1, 0, 0, 0);
    }
    const int64_t cA = c0 + (lane & 31), cB = cA + 32;
    const bool full = contig && c0 + kTile <= cm_first;  // wave-uniform
    unsigned int m[16];
    if (full) {
      // key row of entry j: lr0 + rbase + (j/4)*8 + j%4, a wave-uniform base plus a 32-bit
      // per-lane offset
      const unsigned int vb = (unsigned int)(rbase * nbs + cA) * 4u;  // byte offset
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        char* kj = reinterpret_cast<char*>(keys + (lr0 + (j >> 2) * 8 + (j & 3)) * nbs);
        const unsigned int k0 = score_key(acc0[j]), k1 = score_key(acc1[j]);
        *reinterpret_cast<unsigned int*>(kj + vb) = k0;
        *reinterpret_cast<unsigned int*>(kj + vb + 128u) = k1;
        m[j] = k0 > k1 ? k0 : k1;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int rl = rbase + (j >> 2) * 8 + (j & 3);
        const int64_t cm = row_cm[rl];
        unsigned int* kr = keys + row_key[rl] * nbs;
        unsigned int k0 = 0u, k1 = 0u;
        if (cA < cm) {
          k0 = score_key(acc0[j]);
          kr[cA] = k0;
        }
        if (cB < cm) {
          k1 = score_key(acc1[j]);
          kr[cB] = k1;
        }
        m[j] = k0 > k1 ? k0 : k1;
      }
    }
    if constexpr (TMAX) {
      // row maxima over the 32 lanes of each half-wave: a transposing butterfly (at the step of
      // xor mask s a lane keeps the half of its values that its bit s selects and takes the other
      // half's maxima from its partner), 8 + 4 + 2 + 1 + 1 shuffles for 16 rows
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const bool up = lane & 16;
        const unsigned int keep = up ? m[i + 8] : m[i], send = up ? m[i] : m[i + 8];
        const unsigned int o = __shfl_xor(send, 16, 64);
        m[i] = keep > o ? keep : o;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool up = lane & 8;
        const unsigned int keep = up ? m[i + 4] : m[i], send = up ? m[i] : m[i + 4];
        const unsigned int o = __shfl_xor(send, 8, 64);
        m[i] = keep > o ? keep : o;
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const bool up = lane & 4;
        const unsigned int keep = up ? m[i + 2] : m[i], send = up ? m[i] : m[i + 2];
        const unsigned int o = __shfl_xor(send, 4, 64);
        m[i] = keep > o ? keep : o;
      }
      {
        const bool up = lane & 2;
        const unsigned int keep = up ? m[1] : m[0], send = up ? m[0] : m[1];
        const unsigned int o = __shfl_xor(send, 2, 64);
        m[0] = keep > o ? keep : o;
      }
      const unsigned int o = __shfl_xor(m[0], 1, 64);
      const unsigned int mx = m[0] > o ? m[0] : o;
      // lane l now holds the maximum of entry j = (l % 32) / 2
      const int j = (lane & 31) >> 1;
      const int rl = rbase + (j >> 2) * 8 + (j & 3);
      if (full) {
        if ((lane & 1) == 0) tmax[(lr0 + rl) * ntile + ct] = mx;
      } else if ((lane & 1) == 0 && c0 < row_cm[rl]) {
        tmax[row_key[rl] * ntile + ct] = mx;
      }
    }
    // emag of the strip's rows
    if (lane < 32 && c0 < cma) {
      double mag = 0.0, nsum = 0.0;
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        const double a = sa[t], bb = sroot[t];
        mag += a * bb;
        nsum += a + bb;
      }
      mag += 0x1p-56 * nsum;
      float f = (float)mag;
      if ((double)f < mag) f = __uint_as_float(__float_as_uint(f) + 1u);  // round up (f >= 0)
      emag[lra * ntile + ct] = f;
    }
  }
}

// Inverse of score_key.
__device__ inline float key_value(unsigned int k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ inline double wave_sum_f64(double x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// The wave loads query row `roff` (element offset) into qreg (lane l: dims l + 64 t).
template <int QR>
__device__ inline void cert_load_q(const CertArgs& ca, int rows_dt, int64_t roff,
                                   float (&qreg)[QR]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int t = 0; t < QR; ++t) {
    const int k = lane + 64 * t;
    qreg[t] = k < ca.d ? load_row(ca.rows, roff + k, rows_dt) : 0.0f;
  }
}

// Largest emag over the score tiles of candidates [0, cmax_s) of chunk row lrow, over `nthreads`
// threads from `tid` (each thread's partial maximum; the caller reduces).
__device__ inline float cert_emag_max(const CertArgs& ca, int64_t lrow, int64_t cmax_s, int tid,
                                      int nthreads) {
  const int64_t nt = (cmax_s + kNormTile - 1) / kNormTile;
  const float* p = ca.emag + lrow * ca.ntile;
  float m = 0.0f;
  for (int64_t t = tid; t < nt; t += nthreads) m = fmaxf(m, p[t]);
  return m;
}

// (lo, hi) score keys of the certificate band around the approximate threshold key T, given M,
// the row's largest emag.
__device__ inline void cert_band(const CertArgs& ca, unsigned int T, float M, unsigned int* lo,
                                 unsigned int* hi) {
  const double e = ca.ecoef * (1.0 + 0x1p-10) * (double)M + 0x1p-100;
  const double tau = (double)key_value(T);
  if (!(e < 1e300) || !(fabs(tau) < 1e300)) {  // non-finite: certify nothing
    *lo = 0u;
    *hi = 0xffffffffu;
    return;
  }
  const double lod = tau - 2.0 * e, hid = tau + 2.0 * e;
  float lof = (float)lod, hif = (float)hid;
  // round outward: the adjacent float below / above (x finite)
  if ((double)lof > lod) {
    const unsigned int ub = __float_as_uint(lof);
    lof = lof > 0.0f ? __uint_as_float(ub - 1u) : lof < 0.0f ? __uint_as_float(ub + 1u)
                                                              : -__uint_as_float(1u);
  }
  if ((double)hif < hid) {
    const unsigned int ub = __float_as_uint(hif);
    hif = hif > 0.0f ? __uint_as_float(ub + 1u) : hif < 0.0f ? __uint_as_float(ub - 1u)
                                                              : __uint_as_float(1u);
  }
  *lo = score_key(lof);
  *hi = score_key(hif);
}

// Exact score key of candidate block c of the row held in qreg (its key head's summaries at
// element offset cbase of candidate 0): the fp64-accumulated formula of route_score_kernel, the
// max over the block's pool sub-blocks, computed by one wave.
template <int QR>
__device__ inline unsigned int cert_exact_key(const CertArgs& ca, const float (&qreg)[QR],
                                              int64_t cbase, int64_t c, int64_t pool) {
  const int lane = threadIdx.x & 63;
  unsigned int best = 0u;
  for (int64_t s = 0; s < pool; ++s) {
    const int64_t off = cbase + (c * pool + s) * ca.d;
    double e1 = 0.0, e2 = 0.0, e3 = 0.0;
#pragma unroll
    for (int t = 0; t < QR; ++t) {
      const int k = lane + 64 * t;
      if (k < ca.d) {
        const float q = qreg[t], q2 = q * q;
        e1 = fma((double)q, (double)ca.mu[off + k], e1);
        if (ca.var) e2 = fma((double)q2, (double)ca.var[off + k], e2);
        if (ca.m3) e3 = fma((double)(q2 * q), (double)ca.m3[off + k], e3);
      }
    }
    e1 = wave_sum_f64(e1);
    e2 = wave_sum_f64(e2);
    float sc = __fadd_rn((float)e1, __fmul_rn(ca.coef2, (float)e2));
    if (ca.m3) sc = __fadd_rn(sc, __fmul_rn(ca.coef3, (float)wave_sum_f64(e3)));
    const unsigned int k = score_key(sc);
    best = k > best ? k : best;
  }
  return best;
}

// Exact score key of candidate c (as cert_exact_key) computed by a group of 16 lanes: lane
// (lane & 15) sums head dims (lane & 15) + 16 t, the group reduces with lane exchanges; qg holds
// the query row at those dims. Every lane of the group returns the key.
template <int QR>
__device__ inline unsigned int group_exact_key(const CertArgs& ca, const float (&qg)[4 * QR],
                                               int64_t cbase, int64_t c, int64_t pool) {
  const int l16 = threadIdx.x & 15;
  unsigned int best = 0u;
  for (int64_t s = 0; s < pool; ++s) {
    const int64_t off = cbase + (c * pool + s) * ca.d;
    double e1 = 0.0, e2 = 0.0, e3 = 0.0;
#pragma unroll
    for (int t = 0; t < 4 * QR; ++t) {
      const int k = l16 + 16 * t;
      if (k < ca.d) {
        const float q = qg[t], q2 = q * q;
        e1 = fma((double)q, (double)ca.mu[off + k], e1);
        if (ca.var) e2 = fma((double)q2, (double)ca.var[off + k], e2);
        if (ca.m3) e3 = fma((double)(q2 * q), (double)ca.m3[off + k], e3);
      }
    }
#pragma unroll
    for (int w = 1; w < 16; w <<= 1) {
      e1 += lane_xor(e1, w);
      e2 += lane_xor(e2, w);
      if (ca.m3) e3 += lane_xor(e3, w);
    }
    float sc = __fadd_rn((float)e1, __fmul_rn(ca.coef2, (float)e2));
    if (ca.m3) sc = __fadd_rn(sc, __fmul_rn(ca.coef3, (float)e3));
    const unsigned int k = score_key(sc);
    best = k > best ? k : best;
  }
  return best;
}

constexpr int kSmallNbk = 1024;  // one wave, J = 16 entries per lane

// Top-K of one row of score keys (K = min(keep, cmax)), ties to the lowest block index, then the
// row's local window, compacted ascending into kv_idx (pad 0) with kv_num.
// Rows of at most kCacheKeys candidates are staged in LDS. Rows of more than kFilterMin are first
// filtered: the keys are split into P >= K disjoint groups, so the smallest group maximum T0 is
// <= the K-th largest key; the indices of the keys >= T0 (and, for rows not staged, the keys)
// go to LDS and the radix select runs on them (rows whose filter keeps more than kCand keys use
// the full row). Filtering also pays for staged rows: the digit histograms of a few hundred
// survivors see far fewer same-bin atomics than those of thousands of similar keys.
// Approximate keys (ca.on) are certified: the band candidates, collected in block order, are
// rescored exactly and the remaining places chosen among them by a second radix select; a band
// of more than kCand candidates falls back to rescoring the whole row into the workspace and
// selecting on the exact keys.
template <int NT, int QR>
__global__ __launch_bounds__(NT) void route_select_kernel(
    unsigned int* __restrict__ keys, RouteGeom g, int32_t* __restrict__ kv_num,
    int32_t* __restrict__ kv_idx, int64_t W, CertArgs ca,
    const unsigned int* __restrict__ rowlist, const unsigned int* __restrict__ nlist) {
  __shared__ unsigned int bits[kMaxNbk / 32];
  __shared__ unsigned int cache[kCacheKeys];  // the row's keys, or the filtered candidates
  __shared__ unsigned int cidx[kCand];        // candidate block indices (filtered rows)
  __shared__ unsigned int hist[256];
  __shared__ int wave_sums[NT / 64];
  __shared__ unsigned int bidx[kBand], bkey[kBand];  // the certificate band
  __shared__ unsigned int sh_digit, sh_above, sh_min, sh_ncand, sh_whole, sh_nin, sh_nunc, sh_nq;
  __shared__ float sh_norm[NT / 64];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  int64_t lrow = blockIdx.x;  // (b*Hq + h) * ni + il
  if (rowlist != nullptr) {  // the rows route_select_wave_kernel deferred (workgroup-uniform)
    if (blockIdx.x >= *nlist) return;
    lrow = rowlist[blockIdx.x];
  }
  const int64_t bh = lrow / g.ni, il = lrow % g.ni;
  const int64_t i = g.i0 + il;
  const int64_t cmax = row_cmax(g, i);
  int64_t keep = row_keep(g, cmax);
  const int64_t K = keep < cmax ? keep : cmax;
  unsigned int* kraw = keys + lrow * g.nbk * g.pool;
  // key of block c: the largest of its pool sub-block keys (keys order like the scores, so this is
  // the key of the max-pooled score)
  auto krow = [&](int64_t c) -> unsigned int {
    if (g.pool == 1) return kraw[c];
    unsigned int m = kraw[c * g.pool];
    for (int64_t t = 1; t < g.pool; ++t) {
      const unsigned int x = kraw[c * g.pool + t];
      m = x > m ? x : m;
    }
    return m;
  };
  const int nwords = (int)((g.nbk + 31) / 32);
  bool cert = ca.on && K > 0 && K < cmax;

  // radix select of the K-th largest of src(0..n): returns T, with *rank = the rank of T among
  // the keys equal to it that is still to take, *whole = every key equal to T is taken
  auto radix_kth = [&](auto src, int64_t n, unsigned int kk, unsigned int* rank,
                       bool* whole_out) -> unsigned int {
    unsigned int prefix = 0u, pmask = 0u;
    bool whole = false;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int t = tid; t < 256; t += NT) hist[t] = 0u;
      __syncthreads();
      for (int64_t c = tid; c < n; c += NT) {
        const unsigned int key = src(c);
        if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid < 64) {
        unsigned int v[4], t = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[j] = hist[4 * tid + j];
          t += v[j];
        }
        unsigned int suf = t;  // inclusive suffix over lanes >= tid
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          unsigned int o = __shfl_down(suf, off, 64);
          if (tid + off < 64) suf += o;
        }
        unsigned int above = suf - t;  // keys in bins of higher lanes
#pragma unroll
        for (int j = 3; j >= 0; --j) {
          if (above < kk && kk <= above + v[j]) {
            sh_digit = (unsigned int)(4 * tid + j);
            sh_above = above;
            sh_whole = kk == above + v[j];
          }
          above += v[j];
        }
      }
      __syncthreads();
      prefix |= sh_digit << shift;
      pmask |= 0xffu << shift;
      kk -= sh_above;
      whole = sh_whole != 0u;
      __syncthreads();
      // the digit's whole bin is taken: exactly K keys are >= prefix (lower bits zero), so no
      // tie straddles the cut and the remaining digits need not be resolved
      if (whole) break;
    }
    *rank = kk;
    *whole_out = whole;
    return prefix;
  };

  for (int w = tid; w < nwords; w += NT) bits[w] = 0u;
  const int64_t nt = (cmax * g.pool + kNormTile - 1) / kNormTile;  // score tiles of the row
  for (int pass = 0; pass < 2; ++pass) {
    // tile filter: certified keys with per-tile maxima, more tiles than places
    const bool tilef = cert && ca.tmax != nullptr && g.pool == 1 && K <= NT && nt > K &&
                       cmax > kFilterMin;
    const bool cached = cmax <= kCacheKeys && !tilef;  // whole row in LDS, index order
    if (cached && K > 0 && K < cmax)
      for (int64_t c = tid; c < cmax; c += NT) cache[c] = krow(c);
    if (tid == 0) {
      sh_min = 0xffffffffu;
      sh_ncand = 0u;
      sh_nq = 0u;
    }
    __syncthreads();
    auto rowkey = [&](int64_t c) -> unsigned int { return cached ? cache[c] : krow(c); };

    // keys the radix select runs over: src[0, nsel), block index of entry c: filt ? cidx[c] : c
    bool filt = false;
    int64_t nsel = cmax;
    if (tilef) {
      // T0 = the K-th largest tile maximum: K distinct tiles hold a key >= T0, so T0 <= the K-th
      // largest key, and only tiles whose maximum reaches T0 hold keys >= T0. Tile maxima and
      // the list of those tiles live in the part of `cache` past the kCand candidates.
      unsigned int* tk = cache + kCand;
      unsigned int* qt = cache + kCand + kMaxTiles;
      const unsigned int* tm = ca.tmax + lrow * ca.ntile;
      for (int64_t t = tid; t < nt; t += NT) tk[t] = tm[t];
      __syncthreads();
      unsigned int rk;
      bool wh;
      const unsigned int t0 = radix_kth([&](int64_t t) { return tk[t]; }, nt, (unsigned int)K,
                                        &rk, &wh);
      for (int64_t t = tid; t < nt; t += NT)
        if (tk[t] >= t0) qt[atomicAdd(&sh_nq, 1u)] = (unsigned int)t;
      if (tid == 0) sh_min = t0;
      __syncthreads();
      const unsigned int nq = sh_nq;
      const unsigned long long lt = (1ull << lane) - 1ull;
      // a wave per tile, a lane per candidate, 4 tiles in flight
      for (unsigned int q0 = 4u * wv; q0 < nq; q0 += 4u * (NT / 64)) {
        unsigned int kq[4];
        int64_t cq[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          cq[u] = q0 + u < nq ? (int64_t)qt[q0 + u] * kNormTile + lane : cmax;
          kq[u] = cq[u] < cmax ? kraw[cq[u]] : 0u;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const bool take = cq[u] < cmax && kq[u] >= t0;
          const unsigned long long bm = __ballot(take);
          unsigned int base = 0u;
          if (lane == 0 && bm) base = atomicAdd(&sh_ncand, (unsigned int)__popcll(bm));
          base = __shfl(base, 0, 64);
          const unsigned int slot = base + (unsigned int)__popcll(bm & lt);
          if (take && slot < (unsigned int)kCand) {
            cache[slot] = kq[u];
            cidx[slot] = (unsigned int)cq[u];
          }
        }
      }
      __syncthreads();
      if (sh_ncand <= (unsigned int)kCand) {
        filt = true;
        nsel = sh_ncand;
      }
    } else if (K > 0 && K < cmax && K <= NT && cmax > kFilterMin) {
      int pk = 1;
      while (pk < K) pk <<= 1;
      const int gs = NT / pk < 64 ? NT / pk : 64;  // threads per group (a power of two <= 64)
      unsigned int mx = 0u;
      for (int64_t c = tid; c < cmax; c += NT) {
        const unsigned int key = cached ? cache[c] : krow(c);
        mx = key > mx ? key : mx;
      }
      for (int off = 1; off < gs; off <<= 1) {
        const unsigned int o = __shfl_xor(mx, off, 64);
        mx = o > mx ? o : mx;
      }
      // every lane now holds its group's maximum: T0 = the minimum over all lanes
      for (int off = 1; off < 64; off <<= 1) {
        const unsigned int o = __shfl_xor(mx, off, 64);
        mx = o < mx ? o : mx;
      }
      if (lane == 0) atomicMin(&sh_min, mx);
      __syncthreads();
      const unsigned int t0 = sh_min;
      for (int64_t c = tid; c < cmax; c += NT) {
        const unsigned int key = cached ? cache[c] : krow(c);
        if (key >= t0) {
          const unsigned int slot = atomicAdd(&sh_ncand, 1u);
          if (slot < (unsigned int)kCand) {
            if (!cached) cache[slot] = key;  // a cached row keeps its keys in place
            cidx[slot] = (unsigned int)c;
          }
        }
      }
      __syncthreads();
      if (sh_ncand <= (unsigned int)kCand) {
        filt = true;
        nsel = sh_ncand;
      }
    }
    auto src = [&](int64_t c) -> unsigned int {
      if (filt) return cached ? cache[cidx[c]] : cache[c];
      return cached ? cache[c] : krow(c);
    };
    auto mark = [&](int64_t c) {
      const unsigned int blk = filt ? cidx[c] : (unsigned int)c;
      atomicOr(&bits[blk >> 5], 1u << (blk & 31));
    };

    if (K >= cmax) {
      for (int64_t c = tid; c < cmax; c += NT) atomicOr(&bits[c >> 5], 1u << (c & 31));
      break;
    }
    if (K <= 0) break;
    unsigned int need_eq;
    bool whole;
    const unsigned int T = radix_kth(src, nsel, (unsigned int)K, &need_eq, &whole);
    if (!cert) {
      const unsigned int n_eq = whole ? need_eq : hist[T & 255u];  // keys equal to T
      __syncthreads();
      if (need_eq == n_eq) {
        for (int64_t c = tid; c < nsel; c += NT)
          if (src(c) >= T) mark(c);
      } else {
        for (int64_t c = tid; c < nsel; c += NT)
          if (src(c) > T) mark(c);
        // ties at T: the lowest block indices first (scan in index order)
        unsigned int taken = 0;
        for (int64_t base = 0; base < cmax && taken < need_eq; base += NT) {
          const int64_t c = base + tid;
          const int flag = c < cmax && rowkey(c) == T;
          int tot;
          int pre = block_exclusive_scan<NT>(flag, wave_sums, &tot);
          if (flag && taken + (unsigned int)pre < need_eq)
            atomicOr(&bits[c >> 5], 1u << (c & 31));
          taken += (unsigned int)tot;
        }
      }
      break;
    }

    // ---- certify the approximate selection ----
    {
      float M = cert_emag_max(ca, lrow, cmax * g.pool, tid, NT);
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
      if (lane == 0) sh_norm[wv] = M;
      if (tid == 0) {
        sh_nin = 0u;
        sh_nunc = 0u;
      }
      __syncthreads();
    }
    float M = 0.0f;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) M = fmaxf(M, sh_norm[w]);
    // A filtered list holds exactly the keys >= T0 (sh_min). When the radix select stopped at a
    // digit prefix below T0, the list holds exactly K keys, so exactly K keys of the row are
    // >= T0: T0 is then the threshold (no key of the row lies in [T, T0) outside the list).
    const unsigned int Tc = filt && T < sh_min ? sh_min : T;
    unsigned int lo, hi;
    cert_band(ca, Tc, M, &lo, &hi);
    // Every candidate that can hold a key >= lo: the filtered list when the band lies above its
    // threshold, else the tiles whose maximum reaches lo (tile filter), else the whole row.
    const bool in_list = filt && lo >= sh_min;
    auto for_band_candidates = [&](auto fn) {
      if (in_list) {
        for (int64_t c = tid; c < nsel; c += NT) fn(src(c), cidx[c]);
      } else if (tilef) {
        const unsigned int* tk = cache + kCand;
        for (int64_t t = wv; t < nt; t += NT / 64) {
          if (tk[t] < lo) continue;  // wave-uniform
          const int64_t c = t * kNormTile + lane;
          if (c < cmax) fn(kraw[c], (unsigned int)c);
        }
      } else {
        for (int64_t c = tid; c < cmax; c += NT) fn(rowkey(c), (unsigned int)c);
      }
    };
    // classify: above the band -> taken; in the band -> listed for exact ranking
    for_band_candidates([&](unsigned int key, unsigned int blk) {
      if (key > hi) {
        atomicOr(&bits[blk >> 5], 1u << (blk & 31));
        atomicAdd(&sh_nin, 1u);
      } else if (key >= lo) {
        const unsigned int slot = atomicAdd(&sh_nunc, 1u);
        if (slot < (unsigned int)kBand) bidx[slot] = blk;
      }
    });
    __syncthreads();
    const unsigned int nin = sh_nin, nunc = sh_nunc;
    const unsigned int m = (unsigned int)K - nin;  // places left for the band
    if (nunc <= m) {  // the band fills them exactly
      if (nunc <= (unsigned int)kBand) {
        for (unsigned int u = tid; u < nunc; u += NT) atomicOr(&bits[bidx[u] >> 5], 1u << (bidx[u] & 31));
      } else {
        for_band_candidates([&](unsigned int key, unsigned int blk) {
          if (key >= lo && key <= hi) atomicOr(&bits[blk >> 5], 1u << (blk & 31));
        });
      }
      break;
    }
    const int64_t b = bh / g.Hq, h = bh % g.Hq;
    const int64_t bk = b * g.Hkv + h / g.G;
    const int64_t cbase = bk * g.nbk * g.pool * ca.d;
    float qreg[QR];
    cert_load_q(ca, g.rows_dt, ((b * g.Hq + h) * g.nbq + i) * ca.d, qreg);
    if (nunc <= (unsigned int)kBand) {
      // rescore the band exactly (a wave per candidate)
      for (unsigned int u = wv; u < nunc; u += NT / 64) {
        const unsigned int k = cert_exact_key(ca, qreg, cbase, bidx[u], g.pool);
        if (lane == 0) bkey[u] = k;
      }
      __syncthreads();
      // the band's best K - nin by (exact key, lowest block): taken when fewer rank above
      for (unsigned int u = tid; u < nunc; u += NT) {
        const unsigned int ku = bkey[u], cu = bidx[u];
        unsigned int above = 0;
        for (unsigned int v = 0; v < nunc; ++v)
          above += (bkey[v] > ku || (bkey[v] == ku && bidx[v] < cu)) ? 1u : 0u;
        if (above < m) atomicOr(&bits[cu >> 5], 1u << (cu & 31));
      }
      break;
    }
    // a wide band: rescore the whole row exactly into its keys and select again
    for (int64_t c = wv; c < cmax; c += NT / 64) {
      const unsigned int k = cert_exact_key(ca, qreg, cbase, c, g.pool);
      if (lane == 0)
        for (int64_t t = 0; t < g.pool; ++t) kraw[c * g.pool + t] = k;
    }
    __threadfence_block();
    for (int w = tid; w < nwords; w += NT) bits[w] = 0u;
    __syncthreads();
    cert = false;
  }
  __syncthreads();
  // own block and its `local` predecessors, clipped to [0, own] and to existing blocks
  const int64_t own = row_own(g, i);
  int64_t lo = own - g.local;
  if (lo < 0) lo = 0;
  int64_t hi = own < g.nbk - 1 ? own : g.nbk - 1;
  for (int64_t c = lo + tid; c <= hi; c += NT) atomicOr(&bits[c >> 5], 1u << (c & 31));
  __syncthreads();

  // ascending compaction of the bitmap
  const int wpt = (nwords + NT - 1) / NT;
  const int w0 = tid * wpt;
  int cnt = 0;
  for (int w = w0; w < w0 + wpt && w < nwords; ++w) cnt += __popc(bits[w]);
  int total;
  int pos = block_exclusive_scan<NT>(cnt, wave_sums, &total);
  int32_t* out = kv_idx + (bh * g.nbq + i) * W;
  for (int w = w0; w < w0 + wpt && w < nwords; ++w) {
    unsigned int m = bits[w];
    while (m) {
      int bit = __ffs(m) - 1;
      m &= m - 1;
      if (pos < W) out[pos] = (int32_t)(w * 32 + bit);
      ++pos;
    }
  }
  const int64_t num = total < W ? total : W;
  for (int64_t p = num + tid; p < W; p += NT) out[p] = 0;
  if (tid == 0) kv_num[bh * g.nbq + i] = (int32_t)num;
}

// Rows of at most 64 * J key blocks: one wave per row, lane l holds candidates l + 64 j
// (wave_select_top); the selection plus the local window is compacted in ascending order from
// the per-j ballots. Approximate keys (ca.on) are certified: candidates above the band are
// taken, those below are not; when the band holds more candidates than places remain, they are
// rescored exactly (a wave per candidate) and ranked by (exact key, lowest block).
// wave_kth_key / wave_select_top over the first J of kSmallJ slots per lane (the slots past them
// hold no candidate), J the smallest power of two >= jeff: a row with fewer candidates than the
// kernel's slots searches only the slots that hold them (wave-uniform dispatch).
template <int J, int kSmallJ>
__device__ inline unsigned int kth_first(const unsigned int (&key)[kSmallJ], int64_t K) {
  unsigned int k2[J];
#pragma unroll
  for (int j = 0; j < J; ++j) k2[j] = key[j];
  return wave_kth_key<J>(k2, K);
}
template <int kSmallJ>
__device__ inline unsigned int kth_slots(const unsigned int (&key)[kSmallJ], int64_t K, int jeff) {
  if (kSmallJ >= 2 && jeff <= 1) return kth_first<1>(key, K);
  if constexpr (kSmallJ >= 4)
    if (jeff <= 2) return kth_first<2>(key, K);
  if constexpr (kSmallJ >= 8)
    if (jeff <= 4) return kth_first<4>(key, K);
  if constexpr (kSmallJ >= 16)
    if (jeff <= 8) return kth_first<8>(key, K);
  return wave_kth_key<kSmallJ>(key, K);
}
template <int J, int kSmallJ>
__device__ inline unsigned int select_first(const unsigned int (&key)[kSmallJ], unsigned int cm,
                                            int64_t K, int64_t ncand) {
  unsigned int k2[J];
#pragma unroll
  for (int j = 0; j < J; ++j) k2[j] = key[j];
  return wave_select_top<J>(k2, cm, K, ncand);
}
// wave_kth_key over J slots, except that the search stops early (at a value with exactly K keys
// at or above it) only at trial values >= floor_: the slots hold only the keys >= floor_.
template <int J>
__device__ inline unsigned int wave_kth_key_above(const unsigned int (&key)[J], int64_t K,
                                                  unsigned int floor_) {
  unsigned int all = 0xffffffffu, any = 0u;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    all &= key[j] ? key[j] : 0xffffffffu;
    any |= key[j];
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    all &= lane_xor(all, off);
    any |= lane_xor(any, off);
  }
  const unsigned int diff = all ^ any;
  if (diff == 0u) return all;
  const int top = 31 - __clz(diff);
  unsigned int T = top == 31 ? 0u : all & ~((2u << top) - 1u);
  for (int bit = top; bit >= 0; --bit) {
    const unsigned int t = T | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) cnt += __popcll(__ballot(key[j] >= t));
    if (cnt >= K) {
      T = t;
      if (cnt == K && t >= floor_) break;  // wave-uniform
    }
  }
  return T;
}

// kth_slots on fewer slots: T0, the K-th largest of the lanes' maxima (K <= 64), is at most the
// K-th largest key (K lanes hold a key >= T0), so the search runs over the keys >= T0 alone,
// compacted through the wave's LDS buffer `buf` (64 kSmallJ entries) into 2, 4 or 8 slots. It
// returns the K-th largest key or a value with exactly K keys at or above it, as kth_slots does
// (not always the same value: the certified selection is the same for either).
template <int kSmallJ>
__device__ inline unsigned int kth_filtered(const unsigned int (&key)[kSmallJ], int64_t K,
                                            int jeff, unsigned int* buf) {
  if (jeff <= 2 || K <= 0 || K > 64) return kth_slots<kSmallJ>(key, K, jeff);
  const int lane = threadIdx.x & 63;
  const unsigned long long lt = (1ull << lane) - 1ull;
  unsigned int mx = 0u;
#pragma unroll
  for (int j = 0; j < kSmallJ; ++j) mx = key[j] > mx ? key[j] : mx;
  unsigned int t0;
  if (K == 64) {  // the smallest lane maximum (0 when a lane holds no candidate)
    t0 = mx;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const unsigned int o = lane_xor(t0, off);
      t0 = o < t0 ? o : t0;
    }
  } else {
    const unsigned int m1[1] = {mx};
    t0 = wave_kth_key<1>(m1, K);  // 0 when fewer than K lanes hold a candidate
  }
  if (t0 == 0u) return kth_slots<kSmallJ>(key, K, jeff);
  int n = 0;
#pragma unroll
  for (int j = 0; j < kSmallJ; ++j) {
    const bool take = key[j] >= t0;
    const unsigned long long bt = __ballot(take);
    if (take) buf[n + (int)__popcll(bt & lt)] = key[j];
    n += (int)__popcll(bt);
  }
  wave_lds_sync();
  const auto search = [&](auto jc) -> unsigned int {
    constexpr int J = decltype(jc)::value;
    unsigned int s[J];
#pragma unroll
    for (int j = 0; j < J; ++j) s[j] = lane + 64 * j < n ? buf[lane + 64 * j] : 0u;
    wave_lds_sync();  // the buffer is free for the wave's next use
    return wave_kth_key_above<J>(s, K, t0);
  };
  if (n <= 128) return search(std::integral_constant<int, 2>{});
  if (n <= 256) return search(std::integral_constant<int, 4>{});
  if constexpr (kSmallJ >= 8)
    if (n <= 512) return search(std::integral_constant<int, 8>{});
  return kth_slots<kSmallJ>(key, K, jeff);
}

template <int kSmallJ>
__device__ inline unsigned int select_slots(const unsigned int (&key)[kSmallJ], unsigned int cm,
                                            int64_t K, int64_t ncand, int jeff) {
  if (kSmallJ >= 2 && jeff <= 1) return select_first<1>(key, cm, K, ncand);
  if constexpr (kSmallJ >= 4)
    if (jeff <= 2) return select_first<2>(key, cm, K, ncand);
  if constexpr (kSmallJ >= 8)
    if (jeff <= 4) return select_first<4>(key, cm, K, ncand);
  if constexpr (kSmallJ >= 16)
    if (jeff <= 8) return select_first<8>(key, cm, K, ncand);
  return wave_select_top<kSmallJ>(key, cm, K, ncand);
}

template <int kSmallJ, int QR>
__global__ __launch_bounds__(256) void route_select_small_kernel(
    const unsigned int* __restrict__ keys, RouteGeom g, int32_t* __restrict__ kv_num,
    int32_t* __restrict__ kv_idx, int64_t W, int64_t nrows, CertArgs ca) {
  const int lane = threadIdx.x & 63;
  const int64_t lrow = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (lrow >= nrows) return;  // whole wave
  const int64_t bh = lrow / g.ni, il = lrow % g.ni;
  const int64_t i = g.i0 + il;
  const int64_t cmax = row_cmax(g, i);
  const int64_t keep = row_keep(g, cmax);
  const int64_t K = keep < cmax ? keep : cmax;
  const unsigned int* kraw = keys + lrow * g.nbk * g.pool;
  const unsigned long long lt = (1ull << lane) - 1ull;
  // entry lane + 64 j: block c; non-candidates hold key 0. Per-slot flags are kept as per-lane
  // bit masks (bit j), not as arrays of wave masks.
  unsigned int key[kSmallJ];
#pragma unroll
  for (int j = 0; j < kSmallJ; ++j) {
    const int64_t c = lane + 64 * j;
    unsigned int m = 0u;
    if (c < cmax) {
      m = kraw[c * g.pool];
      for (int64_t t = 1; t < g.pool; ++t) {
        const unsigned int x = kraw[c * g.pool + t];
        m = x > m ? x : m;
      }
    }
    key[j] = m;
  }
  unsigned int selm;
  const int jeff = (int)((cmax + 63) / 64);  // slots holding candidates (wave-uniform)
  if (ca.on && K > 0 && K < cmax) {
    float M = cert_emag_max(ca, lrow, cmax * g.pool, lane, 64);
    __shared__ unsigned int kbuf[4][64 * kSmallJ];
    const unsigned int T = kth_filtered<kSmallJ>(key, K, jeff, kbuf[threadIdx.x >> 6]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
    unsigned int lo, hi;
    cert_band(ca, T, M, &lo, &hi);
    // above the band: taken; in the band: to rank exactly; below: out
    unsigned int uncm = 0u;
    int nin = 0, nunc = 0;
    selm = 0u;
#pragma unroll
    for (int j = 0; j < kSmallJ; ++j) {
      const bool cd = lane + 64 * j < cmax;
      const bool s = cd && key[j] > hi;
      const bool u = cd && !s && key[j] >= lo;
      selm |= (s ? 1u : 0u) << j;
      uncm |= (u ? 1u : 0u) << j;
      nin += __popcll(__ballot(s));
      nunc += __popcll(__ballot(u));
    }
    const int m = (int)K - nin;
    if (nunc <= m) {  // the band fills the remaining places exactly
      selm |= uncm;
    } else if (nunc <= 64) {
      // the band (in block order) to LDS; its exact keys four at a time (a 16-lane group per
      // candidate); candidate i is taken when fewer than m band candidates rank above it
      // (larger exact key, or equal key and lower block)
      __shared__ int band_c[4][64];
      __shared__ unsigned int band_k[4][64];
      __shared__ int band_t[4][64];
      const int wv = threadIdx.x >> 6;
      int bpos[kSmallJ];
      int nb = 0;
#pragma unroll
      for (int j = 0; j < kSmallJ; ++j) {
        const bool u = (uncm >> j) & 1u;
        const unsigned long long bal = __ballot(u);
        bpos[j] = nb + (int)__popcll(bal & lt);
        if (u) band_c[wv][bpos[j]] = lane + 64 * j;
        nb += (int)__popcll(bal);
      }
      const int64_t b = bh / g.Hq, h = bh % g.Hq;
      const int64_t bk = b * g.Hkv + h / g.G;
      const int64_t cbase = bk * g.nbk * g.pool * ca.d;
      float qg[4 * QR];
      {
        const int64_t roff = ((b * g.Hq + h) * g.nbq + i) * ca.d;
#pragma unroll
        for (int t = 0; t < 4 * QR; ++t) {
          const int k = (lane & 15) + 16 * t;
          qg[t] = k < ca.d ? load_row(ca.rows, roff + k, g.rows_dt) : 0.0f;
        }
      }
      wave_lds_sync();
      for (int base = 0; base < nb; base += 4) {  // wave-uniform
        const int bi = base + (lane >> 4);
        const int cb = bi < nb ? band_c[wv][bi] : 0;
        const unsigned int kx = group_exact_key<QR>(ca, qg, cbase, cb, g.pool);
        if ((lane & 15) == 0 && bi < nb) band_k[wv][bi] = kx;
      }
      wave_lds_sync();
      if (lane < nb) {
        const unsigned int ki = band_k[wv][lane];
        const int ci = band_c[wv][lane];
        int above = 0;
        for (int jj = 0; jj < nb; ++jj) {
          const unsigned int kj = band_k[wv][jj];
          above += (kj > ki || (kj == ki && band_c[wv][jj] < ci)) ? 1 : 0;
        }
        band_t[wv][lane] = above < m ? 1 : 0;
      }
      wave_lds_sync();
#pragma unroll
      for (int j = 0; j < kSmallJ; ++j)
        if (((uncm >> j) & 1u) && band_t[wv][bpos[j]]) selm |= 1u << j;
    } else {
      // rescore the band exactly, one candidate at a time in block order (a wave-uniform loop),
      // then take its best m by (exact key, lowest block)
      const int64_t b = bh / g.Hq, h = bh % g.Hq;
      const int64_t bk = b * g.Hkv + h / g.G;
      float qreg[QR];
      cert_load_q(ca, g.rows_dt, ((b * g.Hq + h) * g.nbq + i) * ca.d, qreg);
      const int64_t cbase = bk * g.nbk * g.pool * ca.d;
#pragma unroll
      for (int j = 0; j < kSmallJ; ++j)
        if (!((uncm >> j) & 1u)) key[j] = 0u;
      unsigned int rem = uncm;
      while (true) {
        const int lj = rem ? __ffs(rem) - 1 : 32;  // the lane's first band slot
        int jmin = lj;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) jmin = min(jmin, __shfl_xor(jmin, off, 64));
        if (jmin == 32) break;
        const int src_lane = __ffsll((long long)__ballot(lj == jmin)) - 1;
        const int64_t c = src_lane + 64 * jmin;
        const unsigned int k = cert_exact_key(ca, qreg, cbase, c, g.pool);
        if (lane == src_lane) rem &= ~(1u << jmin);
#pragma unroll
        for (int j = 0; j < kSmallJ; ++j)
          if (lane + 64 * j == c) key[j] = k;
      }
      // rank: a band candidate is taken when fewer than m band candidates rank above it
      unsigned int rem2 = uncm;
      while (true) {
        const int lj = rem2 ? __ffs(rem2) - 1 : 32;
        int jmin = lj;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) jmin = min(jmin, __shfl_xor(jmin, off, 64));
        if (jmin == 32) break;
        const int src_lane = __ffsll((long long)__ballot(lj == jmin)) - 1;
        const int cc = src_lane + 64 * jmin;
        unsigned int kc = 0u;
#pragma unroll
        for (int j = 0; j < kSmallJ; ++j)
          if (j == jmin) kc = key[j];
        kc = __shfl(kc, src_lane, 64);
        int above = 0;
#pragma unroll
        for (int jj = 0; jj < kSmallJ; ++jj)
          above += __popcll(__ballot(((uncm >> jj) & 1u) &&
                                     (key[jj] > kc || (key[jj] == kc && lane + 64 * jj < cc))));
        if (lane == src_lane) {
          rem2 &= ~(1u << jmin);
          if (above < m) selm |= 1u << jmin;
        }
      }
    }
  } else {
    unsigned int cm = 0u;
#pragma unroll
    for (int j = 0; j < kSmallJ; ++j) cm |= (lane + 64 * j < cmax ? 1u : 0u) << j;
    selm = select_slots<kSmallJ>(key, cm, K, cmax, jeff);
  }
  const int64_t own = row_own(g, i);
  int64_t lo = own - g.local;
  if (lo < 0) lo = 0;
  const int64_t hi = own < g.nbk - 1 ? own : g.nbk - 1;
  int32_t* out = kv_idx + (bh * g.nbq + i) * W;
  int pos = 0;
#pragma unroll
  for (int j = 0; j < kSmallJ; ++j) {
    const int64_t c = lane + 64 * j;
    const bool take = ((selm >> j) & 1u) || (c >= lo && c <= hi);
    const unsigned long long b = __ballot(take);
    const int p = pos + __popcll(b & lt);
    if (take && p < W) out[p] = (int32_t)c;
    pos += __popcll(b);
  }
  const int64_t num = pos < W ? pos : W;
  for (int64_t p = num + lane; p < W; p += 64) out[p] = 0;
  if (lane == 0) kv_num[bh * g.nbq + i] = (int32_t)num;
}

// Long rows with certified keys and per-tile maxima (pool 1, keep <= kWaveK): one wave per row,
// no workgroup barriers, 4 rows per workgroup. T0, the K-th largest tile maximum (K distinct
// tiles hold a key >= T0), bounds the K-th largest key from below, so every key >= T0 lies in a
// tile whose maximum reaches T0: those tiles are read (8 in flight per lane) and their keys
// >= T0 kept in the wave's LDS list. T, the K-th largest of the list, is the row's K-th largest
// key (or a prefix with exactly K list keys >= it, in which case exactly K keys of the row are
// >= T0 and T0 serves as the threshold). The certificate band [lo, hi] around it is classified
// from the list when lo >= T0, else from the tiles whose maximum reaches lo; keys above hi are
// taken, and when the band holds more candidates than places remain they are rescored exactly
// (16 lanes per candidate) and ranked by (exact key, lowest block). The taken blocks and the
// local window are written in ascending order. A row this kernel does not take (keep > kWaveK,
// too few tiles, more than kWaveCap keys >= T0, a band of more than kWaveBand) is appended to
// `defer` for route_select_kernel; no output of that row is written here.
constexpr int kWaveK = 64;       // largest keep of the wave select
constexpr int kWaveCap = 512;    // keys >= T0 one wave holds
constexpr int kWaveBand = 128;   // band candidates one wave ranks exactly
constexpr int kWaveSel = 128;    // taken blocks + local window (W <= kWaveSel)
constexpr int kWaveSlots = kMaxTiles / 64;  // tile maxima per lane

template <int QR>
__global__ __launch_bounds__(256) void route_select_wave_kernel(
    const unsigned int* __restrict__ keys, RouteGeom g, int32_t* __restrict__ kv_num,
    int32_t* __restrict__ kv_idx, int64_t W, int64_t nrows, CertArgs ca,
    unsigned int* __restrict__ defer, unsigned int* __restrict__ ndefer) {
  __shared__ unsigned int skey[4][kWaveCap], sidx[4][kWaveCap];
  __shared__ unsigned int bkey[4][kWaveBand], bidx[4][kWaveBand];
  __shared__ unsigned int sel[4][kWaveSel];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t lrow = (int64_t)blockIdx.x * 4 + wv;
  if (lrow >= nrows) return;  // whole wave
  const unsigned long long lt = (1ull << lane) - 1ull;
  const int64_t bh = lrow / g.ni, il = lrow % g.ni;
  const int64_t i = g.i0 + il;
  const int64_t cmax = row_cmax(g, i);
  const int64_t keep = row_keep(g, cmax);
  const int64_t K = keep < cmax ? keep : cmax;
  const int64_t nt = (cmax + kNormTile - 1) / kNormTile;
  auto defer_row = [&]() {
    if (lane == 0) defer[atomicAdd(ndefer, 1u)] = (unsigned int)lrow;
  };
  if (!(K > 0 && K < cmax && K <= kWaveK && nt > K && nt <= kMaxTiles)) {
    defer_row();
    return;
  }
  const unsigned int* kraw = keys + lrow * g.nbk;
  const unsigned int* tm = ca.tmax + lrow * ca.ntile;
  unsigned int tk[kWaveSlots];
#pragma unroll
  for (int j = 0; j < kWaveSlots; ++j) {
    const int64_t t = lane + 64 * j;
    tk[j] = t < nt ? tm[t] : 0u;
  }
  const unsigned int T0 = wave_kth_key<kWaveSlots>(tk, K);
  if (T0 == 0u) {  // fewer than K nonzero tile maxima
    defer_row();
    return;
  }
  // each tile of the lanes' mask m of slot j whose maximum reaches `th`: fn(key, block, valid)
  // for its 64 candidates (lane l: candidate 64 t + l), 8 tiles in flight
  auto for_tiles = [&](unsigned int th, auto fn) {
#pragma unroll
    for (int j = 0; j < kWaveSlots; ++j) {
      unsigned long long m = __ballot(lane + 64 * j < nt && tk[j] >= th);
      while (m) {  // wave-uniform
        int64_t cq[8];
        unsigned int kq[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          int64_t c = cmax;
          if (m) {
            const int b = __ffsll((long long)m) - 1;
            m &= m - 1;
            c = (int64_t)(b + 64 * j) * kNormTile + lane;
          }
          cq[u] = c;
          kq[u] = c < cmax ? kraw[c] : 0u;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) fn(kq[u], (unsigned int)cq[u], cq[u] < cmax);
      }
    }
  };
  // the keys >= T0 (and their blocks) to the wave's list
  int ns = 0;
  for_tiles(T0, [&](unsigned int key, unsigned int blk, bool valid) {
    const bool take = valid && key >= T0;
    const unsigned long long bm = __ballot(take);
    const int slot = ns + (int)__popcll(bm & lt);
    if (take && slot < kWaveCap) {
      skey[wv][slot] = key;
      sidx[wv][slot] = blk;
    }
    ns += (int)__popcll(bm);
  });
  if (ns > kWaveCap) {
    defer_row();
    return;
  }
  wave_lds_sync();
  constexpr int SJ = kWaveCap / 64;
  unsigned int sk[SJ];
#pragma unroll
  for (int j = 0; j < SJ; ++j) sk[j] = lane + 64 * j < ns ? skey[wv][lane + 64 * j] : 0u;
  const unsigned int T = wave_kth_key<SJ>(sk, K);
  float M = cert_emag_max(ca, lrow, cmax, lane, 64);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
  const unsigned int Tc = T < T0 ? T0 : T;
  unsigned int lo, hi;
  cert_band(ca, Tc, M, &lo, &hi);
  // classify: above the band -> taken (to sel); in the band -> listed for exact ranking
  int nin = 0, nunc = 0;
  auto classify = [&](unsigned int key, unsigned int blk, bool valid) {
    const bool s = valid && key > hi;
    const bool u = valid && !s && key >= lo;
    const unsigned long long bs = __ballot(s), bu = __ballot(u);
    const int ps = nin + (int)__popcll(bs & lt), pu = nunc + (int)__popcll(bu & lt);
    if (s && ps < kWaveSel) sel[wv][ps] = blk;
    if (u && pu < kWaveBand) {
      bidx[wv][pu] = blk;
      bkey[wv][pu] = key;
    }
    nin += (int)__popcll(bs);
    nunc += (int)__popcll(bu);
  };
  if (lo >= T0) {
#pragma unroll
    for (int j = 0; j < SJ; ++j) {
      const int e = lane + 64 * j;
      classify(sk[j], e < ns ? sidx[wv][e] : 0u, e < ns);
    }
  } else {
    for_tiles(lo, classify);
  }
  const int m = (int)K - nin;  // places left for the band
  if (nin > (int)K || nunc > kWaveBand) {
    defer_row();
    return;
  }
  wave_lds_sync();
  int n = nin;
  if (nunc <= m) {  // the band fills them exactly
    for (int e = lane; e < nunc; e += 64) sel[wv][nin + e] = bidx[wv][e];
    n = nin + nunc;
  } else {
    // exact keys of the band, four candidates at a time (a 16-lane group each)
    const int64_t b = bh / g.Hq, h = bh % g.Hq;
    const int64_t bk = b * g.Hkv + h / g.G;
    const int64_t cbase = bk * g.nbk * ca.d;
    float qg[4 * QR];
    {
      const int64_t roff = ((b * g.Hq + h) * g.nbq + i) * ca.d;
#pragma unroll
      for (int t = 0; t < 4 * QR; ++t) {
        const int k = (lane & 15) + 16 * t;
        qg[t] = k < ca.d ? load_row(ca.rows, roff + k, g.rows_dt) : 0.0f;
      }
    }
    for (int base = 0; base < nunc; base += 4) {  // wave-uniform
      const int bi = base + (lane >> 4);
      const unsigned int cb = bi < nunc ? bidx[wv][bi] : 0u;
      const unsigned int kx = group_exact_key<QR>(ca, qg, cbase, (int64_t)cb, 1);
      if ((lane & 15) == 0 && bi < nunc) bkey[wv][bi] = kx;
    }
    wave_lds_sync();
    // band candidate e is taken when fewer than m rank above it (larger exact key, or equal key
    // and lower block); exactly m are taken
    int took = 0;
    for (int e0 = 0; e0 < nunc; e0 += 64) {  // wave-uniform
      const int e = e0 + lane;
      bool take = false;
      unsigned int ce = 0u;
      if (e < nunc) {
        const unsigned int ke = bkey[wv][e];
        ce = bidx[wv][e];
        int above = 0;
        for (int f = 0; f < nunc; ++f) {
          const unsigned int kf = bkey[wv][f];
          above += (kf > ke || (kf == ke && bidx[wv][f] < ce)) ? 1 : 0;
        }
        take = above < m;
      }
      const unsigned long long bt = __ballot(take);
      if (take) sel[wv][nin + took + (int)__popcll(bt & lt)] = ce;
      took += (int)__popcll(bt);
    }
    n = nin + took;
  }
  wave_lds_sync();
  // the own block and its `local` predecessors, clipped to [0, own] and to existing blocks,
  // unless taken already
  const int64_t own = row_own(g, i);
  int64_t llo = own - g.local;
  if (llo < 0) llo = 0;
  const int64_t lhi = own < g.nbk - 1 ? own : g.nbk - 1;
  for (int64_t c = llo; c <= lhi; ++c) {  // wave-uniform
    bool hit = false;
    for (int e = lane; e < n; e += 64) hit = hit || sel[wv][e] == (unsigned int)c;
    if (!__any(hit)) {
      if (lane == 0 && n < kWaveSel) sel[wv][n] = (unsigned int)c;
      ++n;
    }
    wave_lds_sync();
  }
  // ascending order: entry e goes to its rank among the (distinct) entries
  int32_t* out = kv_idx + (bh * g.nbq + i) * W;
  const int nw = n < (int)W ? n : (int)W;
  for (int e = lane; e < n; e += 64) {
    const unsigned int ce = sel[wv][e];
    int r = 0;
    for (int f = 0; f < n; ++f) r += sel[wv][f] < ce ? 1 : 0;
    if (r < (int)W) out[r] = (int32_t)ce;
  }
  for (int64_t p = nw + lane; p < W; p += 64) out[p] = 0;
  if (lane == 0) kv_num[bh * g.nbq + i] = (int32_t)nw;
}

__global__ void route_clear_kernel(unsigned int* __restrict__ p, int n) {
  for (int t = threadIdx.x; t < n; t += blockDim.x) p[t] = 0u;
}

// Rows of at most 64 key blocks without pooling or m3: a workgroup of kFusedRows waves takes
// rows of one query head and stages the key head's mu / var rows in LDS as fp64 (row stride
// d + 1 doubles); each wave scores and selects 2^r_log2 rows at once, 64 >> r_log2 lanes per row, no
// score workspace. Within a row, S = 2^s_log2 lanes per candidate each sum a contiguous
// ceil(d / S) slice of the head dims in fp64, combined by shuffles (the host uses S = 1 and the
// most rows per wave that still give every candidate a lane); the fp32 score is assembled as in
// route_score_kernel. A candidate is kept when fewer than keep candidates rank above it (larger
// key, or equal key and lower block index); the kept blocks and the local window are compacted
// in ascending order by ballot.
constexpr int kFusedRows = 8;       // waves per workgroup
constexpr int kFusedLds = 64 * 68;  // staged elements per array: nbk * (d + 4) must fit

__global__ __launch_bounds__(64 * kFusedRows) void route_rows_small_kernel(
    const void* __restrict__ rows, const float* __restrict__ mu, const float* __restrict__ var,
    RouteGeom g, int d, float coef2, int r_log2, int s_log2, bool vec4,
    int32_t* __restrict__ kv_num, int32_t* __restrict__ kv_idx, int64_t W) {
  // the key head's mu / var, converted to fp64 once per workgroup (not once per row): row
  // stride d + 1 doubles, so the 16-byte-apart candidates of a read fall in distinct banks
  extern __shared__ __attribute__((aligned(16))) double fused_lds_d[];  // 2 * nbk * (d + 1)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t bh = blockIdx.y;  // b * Hq + h
  const int64_t b = bh / g.Hq, h = bh % g.Hq, kvh = h / g.G;
  const int ds = d + 1, nk = (int)g.nbk;
  double* ms = fused_lds_d;
  double* vs = fused_lds_d + nk * ds;
  const float* kmu = mu + (b * g.Hkv + kvh) * g.nbk * d;
  const float* kvar = var ? var + (b * g.Hkv + kvh) * g.nbk * d : nullptr;
  for (int idx = tid; idx < nk * d; idx += 64 * kFusedRows) {
    const int c = idx / d, t = idx - c * d;
    ms[c * ds + t] = (double)kmu[idx];
    vs[c * ds + t] = kvar ? (double)kvar[idx] : 0.0;
  }
  __syncthreads();
  // the wave holds 2^r_log2 rows, Lr lanes each: lane = (row rr, candidate c, head-dim part)
  const int lr_log2 = 6 - r_log2, Lr = 1 << lr_log2;
  const int rr = lane >> lr_log2, ll = lane & (Lr - 1);
  const int S = 1 << s_log2;
  const int P = Lr >> s_log2;  // candidate capacity of a row (>= nbk)
  const int c = ll >> s_log2, part = ll & (S - 1);
  const int dl = (d + S - 1) >> s_log2;
  const int k0 = part * dl, k1 = k0 + dl < d ? k0 + dl : d;
  const unsigned long long gmask = Lr == 64 ? ~0ull : ((1ull << Lr) - 1ull);
  const unsigned long long lt = (1ull << ll) - 1ull;
  const int64_t i = ((int64_t)blockIdx.x * kFusedRows + wave) * (1 << r_log2) + rr;
  const bool row_ok = i < g.nbq;
  const int64_t lrow = bh * g.nbq + (row_ok ? i : 0);
  const int64_t cmax = row_ok ? row_cmax(g, i) : 0;
  const bool cand = c < cmax;
  double e1 = 0.0, e2 = 0.0;
  if (cand) {
    const float* q = static_cast<const float*>(rows) + lrow * d;
    const double* mrow = ms + c * ds;
    const double* vrow = vs + c * ds;
    if (vec4 && g.rows_dt != SSA_F32) {  // 16-bit rows, d a multiple of 8 * S: 16-byte loads
      const unsigned short* q16 = static_cast<const unsigned short*>(rows) + lrow * d;
      for (int t = k0; t < k1; t += 8) {
        float qa[8];
        unpack8(*reinterpret_cast<const u32x4*>(q16 + t), qa, g.rows_dt == SSA_BF16);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float q2 = qa[j] * qa[j];
          e1 = fma((double)qa[j], mrow[t + j], e1);
          e2 = fma((double)q2, vrow[t + j], e2);
        }
      }
    } else if (vec4) {  // d a multiple of 4 * S: 16-byte loads
#pragma unroll 4
      for (int t = k0; t < k1; t += 4) {
        const f32x4 qa = *reinterpret_cast<const f32x4*>(q + t);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float q2 = qa[j] * qa[j];  // rounded to fp32 like the reference's product
          e1 = fma((double)qa[j], mrow[t + j], e1);
          e2 = fma((double)q2, vrow[t + j], e2);
        }
      }
    } else {
      for (int t = k0; t < k1; ++t) {
        const float qf = load_row(rows, lrow * d + t, g.rows_dt);
        const float q2 = qf * qf;
        e1 = fma((double)qf, mrow[t], e1);
        e2 = fma((double)q2, vrow[t], e2);
      }
    }
  }
  for (int off = 1; off < S; off <<= 1) {
    e1 += __shfl_xor(e1, off, 64);
    e2 += __shfl_xor(e2, off, 64);
  }
  const bool lead = part == 0;
  const bool live = lead && cand;
  const unsigned int key = live ? score_key(__fadd_rn((float)e1, __fmul_rn(coef2, (float)e2))) : 0u;
  const int64_t keep = row_keep(g, cmax);
  const int64_t K = keep < cmax ? keep : cmax;
  // rank = candidates of the row with a larger key, or an equal key and a lower block index
  // (uniform loop over the row capacity; non-candidates hold key 0 and are not counted)
  int rank = 0;
  const int base = rr << lr_log2;
  for (int j = 0; j < P; ++j) {
    const unsigned int kj = __shfl(key, base + (j << s_log2), 64);
    rank += (j < cmax) && ((kj > key) || (kj == key && j < c));
  }
  const bool sel = K >= cmax ? live : (K > 0 && live && rank < K);
  const int64_t own = row_own(g, i);
  int64_t lo = own - g.local;
  if (lo < 0) lo = 0;
  const int64_t hi = own < g.nbk - 1 ? own : g.nbk - 1;
  const bool take = row_ok && lead && (sel || (c >= lo && c <= hi));
  const unsigned long long bt = (__ballot(take) >> base) & gmask;
  if (!row_ok) return;
  int32_t* out = kv_idx + lrow * W;
  const int p = __popcll(bt & lt);
  if (take && p < W) out[p] = c;
  const int tot = __popcll(bt);
  const int64_t num = tot < W ? tot : W;
  for (int64_t x = num + ll; x < W; x += Lr) out[x] = 0;
  if (ll == 0) kv_num[lrow] = (int32_t)num;
}

__global__ __launch_bounds__(kSelThreads) void expand_selection_kernel(
    const int32_t* __restrict__ kv_num, const int32_t* __restrict__ kv_idx, int64_t W,
    int64_t nbk, uint8_t* __restrict__ sel, int32_t* __restrict__ kv_full) {
  __shared__ unsigned int bits[kMaxNbk / 32];
  __shared__ unsigned int wpre[kMaxNbk / 32];
  __shared__ int wave_sums[kSelThreads / 64];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int nwords = (int)((nbk + 31) / 32);
  for (int w = tid; w < nwords; w += kSelThreads) bits[w] = 0u;
  __syncthreads();
  int num = kv_num[row];
  if (num > W) num = (int)W;
  if (num < 0) num = 0;
  for (int j = tid; j < num; j += kSelThreads) {
    int c = kv_idx[row * W + j];
    if (c >= 0 && c < nbk) atomicOr(&bits[c >> 5], 1u << (c & 31));
  }
  __syncthreads();
  const int wpt = (nwords + kSelThreads - 1) / kSelThreads;
  const int w0 = tid * wpt;
  int cnt = 0;
  for (int w = w0; w < w0 + wpt && w < nwords; ++w) cnt += __popc(bits[w]);
  int total;
  int pre = block_exclusive_scan<kSelThreads>(cnt, wave_sums, &total);
  for (int w = w0; w < w0 + wpt && w < nwords; ++w) {
    wpre[w] = (unsigned int)pre;
    pre += __popc(bits[w]);
  }
  __syncthreads();
  for (int64_t c = tid; c < nbk; c += kSelThreads) {
    const unsigned int word = bits[c >> 5];
    const bool s = (word >> (c & 31)) & 1u;
    const int64_t below = wpre[c >> 5] + __popc(word & ((1u << (c & 31)) - 1u));
    if (sel) sel[row * nbk + c] = s ? 1 : 0;
    if (kv_full) {
      const int64_t p = s ? below : total + (c - below);
      kv_full[row * nbk + p] = (int32_t)c;
    }
  }
}

// out[r][j] = fl32(sum_k x[r][k] * w[k][j]), accumulated in fp64 over k ascending (one rounding):
// the projection of query-block means and key-block means for low-dimensional routing.
__global__ __launch_bounds__(256) void project_rows_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ w,
                                                           int64_t rows, int64_t din,
                                                           int64_t dout, float* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * dout) return;
  const int64_t r = idx / dout, j = idx % dout;
  double acc = 0.0;
  for (int64_t k = 0; k < din; ++k) acc = fma((double)x[r * din + k], (double)w[k * dout + j], acc);
  out[idx] = (float)acc;
}

}  // namespace

// Routes every row; exposed to the decode step, which calls it with a single query row.
int route_impl(const void* rows, int rows_dt, const float* mu, const float* var, const float* m3,
               int64_t B,
               int64_t Hq, int64_t Hkv, int64_t nbq, int64_t nbk, int64_t d, int mode,
               int64_t top_c, float budget_frac, int64_t local, float coef2, float coef3,
               int64_t query_pos, int64_t block, int64_t pool, int32_t* kv_num, int32_t* kv_idx,
               int64_t W, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  SSA_REQUIRE(rows && mu && kv_num && kv_idx, SSA_ERR_INVALID, "route: NULL pointer argument");
  SSA_REQUIRE(rows_dt == SSA_F32 || rows_dt == SSA_F16 || rows_dt == SSA_BF16, SSA_ERR_UNSUPPORTED,
              "route: unknown rows dtype %d", rows_dt);
  SSA_REQUIRE(pool >= 1 && pool <= 64, SSA_ERR_INVALID, "route: pool must be in [1, 64]");
  SSA_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && nbq > 0 && nbk > 0 && d > 0, SSA_ERR_INVALID,
              "route: sizes must be positive");
  SSA_REQUIRE(Hq % Hkv == 0, SSA_ERR_INVALID, "route: Hq=%lld not a multiple of Hkv=%lld",
              (long long)Hq, (long long)Hkv);
  SSA_REQUIRE(mode == SSA_ROUTE_BUDGET || mode == SSA_ROUTE_FLAT || mode == SSA_ROUTE_QUERY ||
                  mode == SSA_ROUTE_STARTED,
              SSA_ERR_INVALID, "route: unknown mode %d", mode);
  SSA_REQUIRE(local >= 0, SSA_ERR_INVALID, "route: local must be >= 0");
  SSA_REQUIRE(mode != SSA_ROUTE_FLAT || top_c >= 0, SSA_ERR_INVALID, "route: flat mode needs top_c");
  SSA_REQUIRE(top_c >= 0 || budget_frac >= 0.0f, SSA_ERR_INVALID, "route: budget_frac < 0");
  SSA_REQUIRE((mode != SSA_ROUTE_QUERY && mode != SSA_ROUTE_STARTED) || (query_pos >= 0 && block > 0),
              SSA_ERR_INVALID,
              "route: query mode needs query_pos >= 0 and block > 0");
  SSA_REQUIRE(var != nullptr || coef2 == 0.0f, SSA_ERR_INVALID, "route: var is NULL, coef2 != 0");
  SSA_REQUIRE(nbk <= kMaxNbk, SSA_ERR_UNSUPPORTED, "route: %lld key blocks exceed %d",
              (long long)nbk, kMaxNbk);
  SSA_REQUIRE(W >= 1, SSA_ERR_INVALID, "route: W must be >= 1");
  const int64_t needW = ssa_route_width(mode, nbq, nbk, top_c, budget_frac, local, query_pos, block);
  SSA_REQUIRE(W >= needW, SSA_ERR_INVALID, "route: W=%lld below the required width %lld",
              (long long)W, (long long)needW);
  const size_t row_bytes = (size_t)nbk * (size_t)pool * 4;
  const size_t rows_per_i = (size_t)(B * Hq);
  SSA_REQUIRE(workspace != nullptr && workspace_bytes >= row_bytes * rows_per_i,
              SSA_ERR_WORKSPACE, "route: workspace of %zu bytes below the minimum %zu",
              workspace_bytes, row_bytes * rows_per_i);
  // The certified MFMA scoring stores per-tile error magnitudes and key maxima after the keys
  // (route_row_bytes per row); with a workspace sized for the keys alone, or operands that the
  // 16-byte staging cannot load, the fp64 scoring runs instead.
  const int64_t nbs = nbk * pool;
  const int64_t ntile = (nbs + kNormTile - 1) / kNormTile;
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  const bool vec = d % 8 == 0 && a16(rows) && a16(mu) && (var == nullptr || a16(var)) &&
                   (m3 == nullptr || a16(m3));
  const bool mfma_ok = vec && d <= 64 * kMaxQReg &&
                       workspace_bytes >= route_row_bytes(nbs) * rows_per_i;
  // rows of more than kSmallNbk candidates take the wave select (route_select_wave_kernel) when
  // the workspace also holds its deferred-row list and counters
  const bool wave_sel = mfma_ok && nbk > kSmallNbk && pool == 1 && W <= kWaveSel &&
                        workspace_bytes >= (route_row_bytes(nbs) + 4) * rows_per_i + kRouteTail;
  const size_t ws_eff = wave_sel ? workspace_bytes - kRouteTail : workspace_bytes;
  const size_t per_row = mfma_ok ? route_row_bytes(nbs) + (wave_sel ? 4 : 0) : row_bytes;
  int64_t chunk = (int64_t)(ws_eff / (per_row * rows_per_i));
  // Operands split once (route_split_kernel) when the workspace holds them beside the keys: the
  // candidates of every key head, then per chunk its query rows (bf16 hi + lo, 4 bytes per
  // value, and 3 norms per item), after the chunk's keys, emag and tile maxima.
  const auto r256 = [](size_t x) { return (x + 255) / 256 * 256; };
  const int nt = 1 + (var ? 1 : 0) + (m3 ? 1 : 0);
  const int64_t nk = nt * d;
  const size_t ncand_all = (size_t)(B * Hkv) * (size_t)nbs;
  const size_t cand_split = 2 * r256(ncand_all * nk * 2) + r256(ncand_all * 12);
  // (it pays only for long rows: at 1,024 candidates the two split launches cost what the
  // score kernel saves)
  bool presplit = false;
  if (mfma_ok && nbk > kSmallNbk && ws_eff > cand_split + 8 * 256) {
    const size_t per_split_row = route_row_bytes(nbs) + (size_t)nk * 4 + 12 + (wave_sel ? 4 : 0);
    const int64_t ch =
        (int64_t)((ws_eff - cand_split - 8 * 256) / (per_split_row * rows_per_i));
    if (ch >= 1) {
      presplit = true;
      chunk = ch;
    }
  }
  if (chunk > nbq) chunk = nbq;
  unsigned int* keys = static_cast<unsigned int*>(workspace);
  float* emag = reinterpret_cast<float*>(keys + (size_t)chunk * rows_per_i * (size_t)nbs);
  unsigned int* tmaxp =
      reinterpret_cast<unsigned int*>(emag + (size_t)chunk * rows_per_i * (size_t)ntile);
  SplitOut As{}, Bs{};
  // end of the keys, tile bounds / maxima (and split operands) of a chunk
  char* used_end = static_cast<char*>(workspace) + (size_t)chunk * rows_per_i * route_row_bytes(nbs);
  if (presplit) {
    const size_t nrow = (size_t)chunk * rows_per_i;
    char* sp = static_cast<char*>(workspace) +
               r256(nrow * ((size_t)nbs * 4 + (size_t)ntile * 8));
    As.hi = reinterpret_cast<unsigned short*>(sp);
    sp += r256(nrow * nk * 2);
    As.lo = reinterpret_cast<unsigned short*>(sp);
    sp += r256(nrow * nk * 2);
    As.sq = reinterpret_cast<float*>(sp);
    sp += r256(nrow * 12);
    Bs.hi = reinterpret_cast<unsigned short*>(sp);
    sp += r256(ncand_all * nk * 2);
    Bs.lo = reinterpret_cast<unsigned short*>(sp);
    sp += r256(ncand_all * nk * 2);
    Bs.sq = reinterpret_cast<float*>(sp);
    sp += r256(ncand_all * 12);
    SSA_REQUIRE(sp <= static_cast<char*>(workspace) + ws_eff, SSA_ERR_WORKSPACE,
                "route: split operands overflow the workspace");
    used_end = sp;
  }
  bool cands_split = false;
  // the wave select's deferred-row list (chunk rows) and per-chunk counters, cleared once here
  unsigned int* defer = nullptr;
  unsigned int* ndef = nullptr;
  if (wave_sel) {
    const uintptr_t end = reinterpret_cast<uintptr_t>(workspace) + workspace_bytes;
    ndef = reinterpret_cast<unsigned int*>((end - 256) & ~(uintptr_t)15);
    defer = reinterpret_cast<unsigned int*>(
        (end - kRouteTail - (uintptr_t)chunk * rows_per_i * 4 + 15) & ~(uintptr_t)15);
    SSA_REQUIRE(used_end <= reinterpret_cast<char*>(defer), SSA_ERR_WORKSPACE,
                "route: the deferred-row list overlaps the score workspace");
    const int64_t nchunks = (nbq + chunk - 1) / chunk;
    route_clear_kernel<<<1, 64, 0, stream>>>(
        ndef, nchunks < kRouteCounters ? (int)nchunks : kRouteCounters);
    SSA_TRY(launch_status("route_clear_kernel"));
  }

  RouteGeom g;
  g.mode = mode;
  g.Hq = Hq;
  g.Hkv = Hkv;
  g.G = Hq / Hkv;
  g.nbq = nbq;
  g.nbk = nbk;
  g.query_pos = query_pos;
  g.block = block;
  g.top_c = top_c;
  g.budget_frac = budget_frac;
  g.local = local;
  g.pool = pool;
  g.rows_dt = rows_dt;
  if (nbk <= 64 && nbk * (d + 4) <= kFusedLds && pool == 1 && m3 == nullptr &&
      B * Hq < 65536) {  // score + select fused, a wave per row
    g.i0 = 0;
    g.ni = nbq;
    // rows per wave 2^r_log2 with one lane per candidate (capacity P = 64 >> r_log2 >= nbk)
    int p_log2 = 0;
    while ((1ll << p_log2) < nbk) ++p_log2;
    const int r_log2 = 6 - p_log2, s_log2 = 0;
    const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    const bool vec4 = d % (rows_dt == SSA_F32 ? 4 : 8) == 0 && a16(rows);
    const int64_t rows_per_wg = (int64_t)kFusedRows << r_log2;
    const int64_t chunks = (nbq + rows_per_wg - 1) / rows_per_wg;
    SSA_REQUIRE(chunks < (1ll << 31), SSA_ERR_UNSUPPORTED, "route: too many rows");
    const size_t lds = (size_t)2 * nbk * (d + 1) * sizeof(double);
    route_rows_small_kernel<<<dim3((unsigned)chunks, (unsigned)(B * Hq)), 64 * kFusedRows, lds,
                              stream>>>(rows, mu, var, g, (int)d, coef2, r_log2, s_log2, vec4,
                                        kv_num, kv_idx, W);
    return launch_status("route_rows_small_kernel");
  }
  CertArgs ca{};
  ca.on = 0;
  for (int64_t i0 = 0; i0 < nbq; i0 += chunk) {
    g.i0 = i0;
    g.ni = nbq - i0 < chunk ? nbq - i0 : chunk;
    const int64_t R = g.G * g.ni;
    const int64_t row_tiles = (R + kTile - 1) / kTile;
    const int64_t imax = i0 + g.ni - 1;
    const int64_t cmax_all = row_cmax_s(g, imax);  // scored candidates (sub-block units)
    const int64_t cand_tiles = cmax_all > 0 ? (cmax_all + kTile - 1) / kTile : 0;
    if (cand_tiles > 0 && R <= 16) {
      ca.on = 0;
      int rp_log2 = 0;
      while ((1 << rp_log2) < R) ++rp_log2;
      const int64_t cpb = 256 >> rp_log2;
      const int64_t nblk = (cmax_all + cpb - 1) / cpb;
      SSA_REQUIRE(nblk < (1ll << 31) && B * Hkv < 65536, SSA_ERR_UNSUPPORTED,
                  "route: score grid too large");
      dim3 grid((unsigned)nblk, (unsigned)(B * Hkv));
      if (m3 != nullptr)
        route_score_rows_kernel<true><<<grid, 256, 0, stream>>>(rows, mu, var, m3, g, (int)d,
                                                                coef2, coef3, keys, rp_log2);
      else
        route_score_rows_kernel<false><<<grid, 256, 0, stream>>>(rows, mu, var, m3, g, (int)d,
                                                                 coef2, coef3, keys, rp_log2);
      SSA_TRY(launch_status("route_score_rows_kernel"));
    } else if (cand_tiles > 0 && mfma_ok) {
      SSA_REQUIRE(row_tiles * cand_tiles < (1ll << 31) && B * Hkv < 65536, SSA_ERR_UNSUPPORTED,
                  "route: score grid too large");
      // tile maxima feed the tile filter of route_select_kernel (pool 1, rows of > kSmallNbk)
      const bool tm = nbk > kSmallNbk && pool == 1;
      ca.on = 1;
      ca.rows = rows;
      ca.mu = mu;
      ca.var = var;
      ca.m3 = m3;
      ca.emag = emag;
      ca.tmax = tm ? tmaxp : nullptr;
      ca.ntile = ntile;
      ca.d = (int)d;
      {  // 3n exact bf16 products summed in fp32 (1.02: their magnitudes over |a||b|), the split
         // and dropped lo.lo terms (3.1 2^-16), the exact score's own roundings (the 16)
        const double n = (double)((1 + (var ? 1 : 0) + (m3 ? 1 : 0)) * d);
        ca.ecoef = 1.03 * (3.0 * n + 16.0) * 0x1p-23 + 0x1p-14;
      }
      ca.coef2 = coef2;
      ca.coef3 = coef3;
      dim3 grid((unsigned)(row_tiles * cand_tiles), (unsigned)(B * Hkv));
      if (presplit) {
        if (!cands_split) {
          SSA_REQUIRE(ncand_all < (1ull << 33), SSA_ERR_UNSUPPORTED, "route: too many candidates");
          // candidates: the present terms in slot order (mu, then var, then m3)
          const float* ct1 = var ? var : m3;
          const float* ct2 = var ? m3 : nullptr;
          route_split_kernel<false><<<(unsigned)((ncand_all + 3) / 4), 256, 0, stream>>>(
              nullptr, mu, ct1, ct2, g, (int)d, nt, coef2, coef3, (int64_t)ncand_all, Bs);
          SSA_TRY(launch_status("route_split_kernel"));
          cands_split = true;
        }
        const int64_t nrow = (int64_t)rows_per_i * g.ni;
        route_split_kernel<true><<<(unsigned)((nrow + 3) / 4), 256, 0, stream>>>(
            rows, nullptr, var, m3, g, (int)d, nt, coef2, coef3, nrow, As);
        SSA_TRY(launch_status("route_split_kernel"));
        if ((nk == 64 || nk == 128) && nbs < (1ll << 24)) {
          // the row operands in registers, a strip of rows per workgroup
          const int64_t nstrips = (R + kStripRows - 1) / kStripRows;
          const int64_t nseg = (cand_tiles + kStripSeg - 1) / kStripSeg;
          SSA_REQUIRE(nstrips * nseg < (1ll << 31), SSA_ERR_UNSUPPORTED,
                      "route: score grid too large");
          const dim3 sgrid((unsigned)(nstrips * nseg), (unsigned)(B * Hkv));
          const auto strip = [&](auto nks) {
            constexpr int N = decltype(nks)::value;
            if (tm)
              route_score_strip_kernel<N, true><<<sgrid, 256, 0, stream>>>(
                  As, Bs, g, keys, emag, tmaxp, ntile, nstrips);
            else
              route_score_strip_kernel<N, false><<<sgrid, 256, 0, stream>>>(
                  As, Bs, g, keys, emag, tmaxp, ntile, nstrips);
          };
          if (nk == 64) strip(std::integral_constant<int, 4>{});
          else strip(std::integral_constant<int, 8>{});
          SSA_TRY(launch_status("route_score_strip_kernel"));
        } else {
          if (tm)
            route_score_split_kernel<true><<<grid, 256, 0, stream>>>(
                As, Bs, g, (int)nk, keys, emag, tmaxp, ntile, row_tiles, cand_tiles);
          else
            route_score_split_kernel<false><<<grid, 256, 0, stream>>>(
                As, Bs, g, (int)nk, keys, emag, tmaxp, ntile, row_tiles, cand_tiles);
          SSA_TRY(launch_status("route_score_split_kernel"));
        }
      } else {
#define SSA_SCORE_MFMA(E, T)                                                                       \
  route_score_mfma_kernel<E, T><<<grid, 256, 0, stream>>>(rows, mu, var, m3, g, (int)d, coef2,    \
                                                          coef3, keys, emag, tmaxp, ntile,         \
                                                          row_tiles, cand_tiles)
      if (m3 != nullptr) {
        if (tm) SSA_SCORE_MFMA(true, true);
        else SSA_SCORE_MFMA(true, false);
      } else {
        if (tm) SSA_SCORE_MFMA(false, true);
        else SSA_SCORE_MFMA(false, false);
      }
#undef SSA_SCORE_MFMA
      SSA_TRY(launch_status("route_score_mfma_kernel"));
      }
    } else if (cand_tiles > 0) {
      SSA_REQUIRE(row_tiles * cand_tiles < (1ll << 31) && B * Hkv < 65536, SSA_ERR_UNSUPPORTED,
                  "route: score grid too large");
      ca.on = 0;
      if (m3 != nullptr) {
        dim3 grid((unsigned)(row_tiles * cand_tiles), (unsigned)(B * Hkv));
        route_score_kernel<true, kTile><<<grid, 256, 0, stream>>>(
            rows, mu, var, m3, g, (int)d, coef2, coef3, keys, row_tiles, cand_tiles);
      } else {
        dim3 grid((unsigned)(row_tiles * cand_tiles), (unsigned)(B * Hkv));
        route_score_kernel<false, kTile><<<grid, 256, 0, stream>>>(
            rows, mu, var, m3, g, (int)d, coef2, coef3, keys, row_tiles, cand_tiles);
      }
      SSA_TRY(launch_status("route_score_kernel"));
    }
    const int64_t nrows = B * Hq * g.ni;
    SSA_REQUIRE(nrows < (1ll << 31), SSA_ERR_UNSUPPORTED, "route: too many rows");
    const int qr = d <= 64 ? 1 : d <= 128 ? 2 : d <= 256 ? 4 : 8;  // (cert rows: d <= 512)
    const int64_t ci = i0 / chunk;  // chunk index: its wave-select counter
    const bool wave = wave_sel && ca.on && ca.tmax != nullptr && ci < kRouteCounters;
#define SSA_SELECT(QR)                                                                             \
  do {                                                                                             \
    if (nbk <= 256) /* few candidates: a wave per row */                                           \
      route_select_small_kernel<4, QR><<<(unsigned)((nrows + 3) / 4), 256, 0, stream>>>(          \
          keys, g, kv_num, kv_idx, W, nrows, ca);                                                  \
    else if (nbk <= kSmallNbk)                                                                     \
      route_select_small_kernel<16, QR><<<(unsigned)((nrows + 3) / 4), 256, 0, stream>>>(         \
          keys, g, kv_num, kv_idx, W, nrows, ca);                                                  \
    else if (wave) { /* long certified rows: a wave per row, the rows it defers next */          \
      route_select_wave_kernel<QR><<<(unsigned)((nrows + 3) / 4), 256, 0, stream>>>(             \
          keys, g, kv_num, kv_idx, W, nrows, ca, defer, ndef + ci);                                \
      SSA_TRY(launch_status("route_select_wave_kernel"));                                          \
      route_select_kernel<kSelThreads, QR><<<(unsigned)nrows, kSelThreads, 0, stream>>>(          \
          keys, g, kv_num, kv_idx, W, ca, defer, ndef + ci);                                       \
    } else if (nrows < 1024) /* few rows (e.g. a decode step): more threads per row */             \
      route_select_kernel<1024, QR><<<(unsigned)nrows, 1024, 0, stream>>>(keys, g, kv_num, kv_idx, \
                                                                           W, ca, nullptr, nullptr); \
    else                                                                                           \
      route_select_kernel<kSelThreads, QR><<<(unsigned)nrows, kSelThreads, 0, stream>>>(          \
          keys, g, kv_num, kv_idx, W, ca, nullptr, nullptr);                                       \
  } while (0)
    if (!ca.on || qr == 1) SSA_SELECT(1);
    else if (qr == 2) SSA_SELECT(2);
    else if (qr == 4) SSA_SELECT(4);
    else SSA_SELECT(8);
#undef SSA_SELECT
    SSA_TRY(launch_status("route_select_kernel"));
  }
  return SSA_OK;
}

}  // namespace ssa

extern "C" int64_t ssa_route_width(int mode, int64_t nbq, int64_t nbk, int64_t top_c,
                                   float budget_frac, int64_t local, int64_t query_pos,
                                   int64_t block) {
  ssa::RouteGeom g;
  g.mode = mode;
  g.nbq = nbq;
  g.nbk = nbk;
  g.top_c = top_c;
  g.budget_frac = budget_frac;
  g.local = local < 0 ? 0 : local;
  g.query_pos = query_pos;
  g.block = block > 0 ? block : 1;
  g.pool = 1;
  int64_t w = 1;
  // keep is monotone in cmax, and cmax is monotone in the row index: the last row is the widest
  // unless clipping by nbk makes several rows equal (still bounded by the last row).
  for (int64_t i = nbq - 1; i >= 0 && i >= nbq - 2; --i) {
    const int64_t cmax = ssa::row_cmax(g, i);
    const int64_t keep = ssa::row_keep(g, cmax);
    int64_t k = keep < cmax ? keep : cmax;
    int64_t cnt = k + g.local + 1;
    if (cnt > w) w = cnt;
  }
  return w < nbk ? w : nbk;
}

extern "C" size_t ssa_route_workspace_size_split(int64_t B, int64_t Hq, int64_t Hkv, int64_t nbq,
                                                 int64_t nbk, int64_t d, int64_t nterms) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || nbq <= 0 || nbk <= 0 || d <= 0 || nterms < 1 ||
      nterms > 3)
    return 0;
  const auto r256 = [](size_t x) { return (x + 255) / 256 * 256; };
  const size_t nk = (size_t)(nterms * d), rows = (size_t)(B * Hq * nbq);
  const size_t cands = (size_t)(B * Hkv) * (size_t)nbk;
  const size_t cand_split = 2 * r256(cands * nk * 2) + r256(cands * 12);
  return rows * (ssa::route_row_bytes(nbk) + 4 + nk * 4 + 12) + cand_split + 8 * 256 +
         ssa::kRouteTail;
}

extern "C" size_t ssa_route_workspace_size(int64_t B, int64_t Hq, int64_t nbq, int64_t nbk) {
  // keys, tile bounds and maxima, and the wave select's deferred-row slot per row; its counters
  return (size_t)B * (size_t)Hq * (size_t)nbq * (ssa::route_row_bytes(nbk) + 4) +
         ssa::kRouteTail;
}

extern "C" int ssa_route(const void* rows, int rows_dtype, const float* mu, const float* var,
                         const float* m3, int64_t B, int64_t Hq, int64_t Hkv, int64_t nbq, int64_t nbk, int64_t d,
                         int mode, int64_t top_c, float budget_frac, int64_t local, float coef2,
                         float coef3, int64_t query_pos, int64_t block, int32_t* kv_num,
                         int32_t* kv_idx, int64_t W, void* workspace, size_t workspace_bytes,
                         ssa_stream_t stream) {
  return ssa::route_impl(rows, rows_dtype, mu, var, m3, B, Hq, Hkv, nbq, nbk, d, mode, top_c,
                         budget_frac, local, coef2, coef3, query_pos, block, 1, kv_num, kv_idx, W,
                         workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int ssa_route_pooled(const void* rows, int rows_dtype, const float* mu,
                                const float* var, const float* m3, int64_t B, int64_t Hq, int64_t Hkv, int64_t nbq,
                                int64_t nbk, int64_t pool, int64_t d, int mode, int64_t top_c,
                                float budget_frac, int64_t local, float coef2, float coef3,
                                int64_t query_pos, int64_t block, int32_t* kv_num, int32_t* kv_idx,
                                int64_t W, void* workspace, size_t workspace_bytes,
                                ssa_stream_t stream) {
  return ssa::route_impl(rows, rows_dtype, mu, var, m3, B, Hq, Hkv, nbq, nbk, d, mode, top_c,
                         budget_frac, local, coef2, coef3, query_pos, block, pool, kv_num, kv_idx,
                         W, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int ssa_project_rows(const float* x, const float* w, int64_t rows, int64_t din,
                                int64_t dout, float* out, ssa_stream_t stream) {
  SSA_REQUIRE(x && w && out, SSA_ERR_INVALID, "project_rows: NULL pointer argument");
  SSA_REQUIRE(rows > 0 && din > 0 && dout > 0, SSA_ERR_INVALID, "project_rows: bad sizes");
  const int64_t total = rows * dout;
  SSA_REQUIRE((total + 255) / 256 < (1ll << 31), SSA_ERR_UNSUPPORTED, "project_rows: too large");
  ssa::project_rows_kernel<<<(unsigned)((total + 255) / 256), 256, 0,
                             static_cast<hipStream_t>(stream)>>>(x, w, rows, din, dout, out);
  return ssa::launch_status("project_rows_kernel");
}

extern "C" int ssa_expand_selection(const int32_t* kv_num, const int32_t* kv_idx, int64_t rows,
                                    int64_t W, int64_t nbk, uint8_t* sel, int32_t* kv_full,
                                    ssa_stream_t stream) {
  SSA_REQUIRE(kv_num && kv_idx, SSA_ERR_INVALID, "expand_selection: NULL list argument");
  SSA_REQUIRE(rows > 0 && W > 0 && nbk > 0, SSA_ERR_INVALID, "expand_selection: bad sizes");
  SSA_REQUIRE(nbk <= ssa::kMaxNbk, SSA_ERR_UNSUPPORTED, "expand_selection: nbk too large");
  SSA_REQUIRE(rows < (1ll << 31), SSA_ERR_UNSUPPORTED, "expand_selection: too many rows");
  if (sel == nullptr && kv_full == nullptr) return SSA_OK;
  ssa::expand_selection_kernel<<<(unsigned)rows, ssa::kSelThreads, 0,
                                 static_cast<hipStream_t>(stream)>>>(kv_num, kv_idx, W, nbk, sel,
                                                                     kv_full);
  return ssa::launch_status("expand_selection_kernel");
}
