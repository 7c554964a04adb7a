// Block-summary kernel: per key block the mean mu, the variance (population or unbiased) and
// optionally the third central moment m3, or per query block the mean q-bar. One workgroup of
// 256 threads streams one block of rows with 16/32-byte coalesced loads, accumulates in fp64 and
// rounds once to fp32 (two passes: the mean, then the centred moments about the fp64 mean; the
// second pass re-reads the block, which is then L2-resident).
//
// Reference semantics: ssa/ssa_kernel.py:78-91 (block_route_budget), :42-44,47 (block_route),
// ssa/gemma_ssa.py:65-82 (_block_stats), ssa/ivf_kernel.py:50-60 (block_means).
#include <type_traits>

#include "common.h"

namespace ssa {
namespace {

constexpr int kSumThreads = 256;
constexpr int kMaxD = 512;

template <int DT>
__device__ inline void load_row8(const char* p, float* out) {
  if constexpr (DT == SSA_F32) {
    const f32x4* q = reinterpret_cast<const f32x4*>(p);
    f32x4 a = q[0], b = q[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[i] = a[i];
      out[4 + i] = b[i];
    }
  } else {
    u32x4 w = *reinterpret_cast<const u32x4*>(p);
    unpack8(w, out, DT == SSA_BF16);
  }
}

// A row's 8 columns as loaded (16-bit: one 16-byte word, unpacked when used), and unpacked.
template <int DT>
struct Raw8 {
  using T = typename std::conditional<DT == SSA_F32, f32x4, u32x4>::type;
  T w[DT == SSA_F32 ? 2 : 1];
};
template <int DT>
__device__ inline void load_raw8(const char* p, Raw8<DT>& r) {
  if constexpr (DT == SSA_F32) {
    const f32x4* q = reinterpret_cast<const f32x4*>(p);
    r.w[0] = q[0];
    r.w[1] = q[1];
  } else {
    r.w[0] = *reinterpret_cast<const u32x4*>(p);
  }
}
template <int DT>
__device__ inline void unpack_raw8(const Raw8<DT>& r, float* out) {
  if constexpr (DT == SSA_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[i] = r.w[0][i];
      out[4 + i] = r.w[1][i];
    }
  } else {
    unpack8(r.w[0], out, DT == SSA_BF16);
  }
}

// Sums the per-thread partials red[q*d + t] over the rpp row groups into colv[t].
__device__ inline void reduce_columns(const double* red, double* colv, int d, int rpp, int tid) {
  for (int t = tid; t < d; t += kSumThreads) {
    double s = 0.0;
    for (int q = 0; q < rpp; ++q) s += red[q * d + t];
    colv[t] = s;
  }
}

// grid (nb, B*H); each thread owns 8 consecutive columns (cv) of every rpp-th row of the block
// (rpp = 256 / (d/8) row groups; with d/8 not dividing 256 the last 256 % (d/8) threads idle).
template <int DT>
__global__ __launch_bounds__(kSumThreads) void block_summary_kernel(
    const char* __restrict__ x, int64_t H, int d, int64_t sb, int64_t sh, int64_t sn,
    int64_t block, int64_t n_rows, int64_t rows_counted, int mode, float* __restrict__ mu,
    float* __restrict__ var, float* __restrict__ m3, int64_t nb) {
  constexpr int ES = DT == SSA_F32 ? 4 : 2;
  __shared__ double red[kSumThreads * 8];
  __shared__ double colv[kMaxD];
  __shared__ double colm[kMaxD];  // fp64 column means

  const int64_t bh = blockIdx.y;
  const int64_t b = bh / H, h = bh % H;
  const int64_t c = blockIdx.x;
  const int ncv = d / 8;
  const int rpp = kSumThreads / ncv;
  const int tid = threadIdx.x;
  const int cv = tid % ncv;
  const int r0 = tid / ncv;
  const bool active = r0 < rpp;

  const int64_t start = c * block;
  int64_t end = start + block;
  if (end > rows_counted) end = rows_counted;
  const int64_t cnt_rows = end > start ? end - start : 0;
  // rows [n_rows, end) are zero rows that count (rows_counted > n_rows): they add nothing to the
  // sums and (0 - mean)^p to the centred moments
  const int64_t rend = end < n_rows ? end : n_rows;
  const int64_t zrows = end - (start > rend ? start : rend);
  const double z = zrows > 0 ? (double)zrows : 0.0;
  const char* base = x + (b * sb + h * sh) * ES + (int64_t)cv * 8 * ES;
  const int64_t out_row = (bh * nb + c) * d;

  // pass 1: column sums
  double acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.0;
  for (int64_t r = start + r0; active && r < rend; r += rpp) {
    float v[8];
    load_row8<DT>(base + r * sn * ES, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] += (double)v[j];
  }
  if (active)
#pragma unroll
    for (int j = 0; j < 8; ++j) red[r0 * d + cv * 8 + j] = acc[j];
  __syncthreads();
  reduce_columns(red, colv, d, rpp, tid);
  __syncthreads();

  if (mode == SSA_STATS_QMEAN) {
    for (int t = tid; t < d; t += kSumThreads) mu[out_row + t] = (float)(colv[t] / (double)block);
    return;
  }
  const double cnt = cnt_rows > 0 ? (double)cnt_rows : 1.0;
  for (int t = tid; t < d; t += kSumThreads) {
    colm[t] = colv[t] / cnt;
    mu[out_row + t] = (float)(colv[t] / cnt);
  }
  double mean[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) mean[j] = colv[cv * 8 + j] / cnt;
  __syncthreads();  // red and colv are reused below

  // pass 2: centred second and third moments about the fp64 mean
  double a2[8], a3[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) a2[j] = a3[j] = 0.0;
  for (int64_t r = start + r0; active && r < rend; r += rpp) {
    float v[8];
    load_row8<DT>(base + r * sn * ES, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      double e = (double)v[j] - mean[j];
      double e2 = e * e;
      a2[j] += e2;
      a3[j] += e2 * e;
    }
  }
  if (var != nullptr) {
    if (active)
#pragma unroll
      for (int j = 0; j < 8; ++j) red[r0 * d + cv * 8 + j] = a2[j];
    __syncthreads();
    reduce_columns(red, colv, d, rpp, tid);
    __syncthreads();
    const double vden = mode == SSA_STATS_UNBIASED ? cnt - 1.0 : cnt;
    for (int t = tid; t < d; t += kSumThreads)
      var[out_row + t] = (float)((colv[t] + z * colm[t] * colm[t]) / vden);
    __syncthreads();
  }
  if (m3 != nullptr) {
    if (active)
#pragma unroll
      for (int j = 0; j < 8; ++j) red[r0 * d + cv * 8 + j] = a3[j];
    __syncthreads();
    reduce_columns(red, colv, d, rpp, tid);
    __syncthreads();
    for (int t = tid; t < d; t += kSumThreads)
      m3[out_row + t] = (float)((colv[t] - z * colm[t] * colm[t] * colm[t]) / cnt);
  }
}

// One wave per block (head dims 64 and 128: NCV = d/8 column groups of 8, RG = 64/NCV row
// groups): lane (rg, cv) streams rows rg, rg + RG, ... of the block with kWaveRows of them in
// flight per step, accumulates its 8 columns in fp64, and the row groups are summed by lane
// exchanges (xor NCV, 2 NCV, ..., 32: every lane ends with its columns' sums) -- no LDS, no
// workgroup barrier. Same two passes and zero-row rules as block_summary_kernel. grid
// (ceil(nb / 4), B*H), 4 waves: wave w takes block 4 blockIdx.x + w.
constexpr int kWaveRows = 8;

template <int DT, int NCV>
__global__ __launch_bounds__(256) void block_summary_wave_kernel(
    const char* __restrict__ x, int64_t H, int64_t sb, int64_t sh, int64_t sn, int64_t block,
    int64_t n_rows, int64_t rows_counted, int mode, float* __restrict__ mu,
    float* __restrict__ var, float* __restrict__ m3, int64_t nb) {
  constexpr int ES = DT == SSA_F32 ? 4 : 2, RG = 64 / NCV, d = NCV * 8;
  const int lane = threadIdx.x & 63;
  const int64_t c = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t nblk = (n_rows + block - 1) / block;
  if (c >= nblk) return;  // (whole waves)
  const int64_t bh = blockIdx.y, b = bh / H, h = bh % H;
  const int cv = lane % NCV, rg = lane / NCV;
  const int64_t start = c * block;
  int64_t end = start + block;
  if (end > rows_counted) end = rows_counted;
  const int64_t cnt_rows = end > start ? end - start : 0;
  const int64_t rend = end < n_rows ? end : n_rows;
  const int64_t zrows = end - (start > rend ? start : rend);
  const double z = zrows > 0 ? (double)zrows : 0.0;
  const char* base = x + (b * sb + h * sh) * ES + (int64_t)cv * 8 * ES;
  const int64_t out_row = (bh * nb + c) * d + cv * 8;
  auto colsum = [&](double (&a)[8]) {
#pragma unroll
    for (int w = NCV; w < 64; w <<= 1)
#pragma unroll
      for (int j = 0; j < 8; ++j) a[j] += lane_xor(a[j], w);
  };
  // pass 1: column sums
  double acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.0;
  for (int64_t r = start + rg; r < rend; r += kWaveRows * RG) {
    Raw8<DT> raw[kWaveRows];
#pragma unroll
    for (int u = 0; u < kWaveRows; ++u)
      if (r + u * RG < rend) load_raw8<DT>(base + (r + u * RG) * sn * ES, raw[u]);
#pragma unroll
    for (int u = 0; u < kWaveRows; ++u)
      if (r + u * RG < rend) {
        float v[8];
        unpack_raw8<DT>(raw[u], v);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += (double)v[j];
      }
  }
  colsum(acc);
  if (mode == SSA_STATS_QMEAN) {
    if (rg == 0)
#pragma unroll
      for (int j = 0; j < 8; ++j) mu[out_row + j] = (float)(acc[j] / (double)block);
    return;
  }
  const double cnt = cnt_rows > 0 ? (double)cnt_rows : 1.0;
  double mean[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) mean[j] = acc[j] / cnt;
  if (rg == 0)
#pragma unroll
    for (int j = 0; j < 8; ++j) mu[out_row + j] = (float)mean[j];
  // pass 2: centred second and third moments about the fp64 mean (the rows again, from L2)
  double a2[8], a3[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) a2[j] = a3[j] = 0.0;
  for (int64_t r = start + rg; r < rend; r += kWaveRows * RG) {
    Raw8<DT> raw[kWaveRows];
#pragma unroll
    for (int u = 0; u < kWaveRows; ++u)
      if (r + u * RG < rend) load_raw8<DT>(base + (r + u * RG) * sn * ES, raw[u]);
#pragma unroll
    for (int u = 0; u < kWaveRows; ++u)
      if (r + u * RG < rend) {
        float v[8];
        unpack_raw8<DT>(raw[u], v);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const double e = (double)v[j] - mean[j];
          const double e2 = e * e;
          a2[j] += e2;
          a3[j] += e2 * e;
        }
      }
  }
  if (var != nullptr) {
    colsum(a2);
    const double vden = mode == SSA_STATS_UNBIASED ? cnt - 1.0 : cnt;
    if (rg == 0)
#pragma unroll
      for (int j = 0; j < 8; ++j) var[out_row + j] = (float)((a2[j] + z * mean[j] * mean[j]) / vden);
  }
  if (m3 != nullptr) {
    colsum(a3);
    if (rg == 0)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        m3[out_row + j] = (float)((a3[j] - z * mean[j] * mean[j] * mean[j]) / cnt);
  }
}

}  // namespace

// Shared by ssa_block_summary and the decode step (which summarises one completed block).
int launch_block_summary(const void* x, int dtype, int64_t B, int64_t H, int64_t n, int64_t d,
                         int64_t sb, int64_t sh, int64_t sn, int64_t block, int64_t n_real,
                         int mode, float* mu, float* var, float* m3, int64_t nb_out,
                         int64_t block_offset, hipStream_t stream) {
  const int64_t nb = (n + block - 1) / block;
  // n_real > n: rows [n, n_real) count as zero rows (capped at the last block's end)
  int64_t rows_counted = mode == SSA_STATS_QMEAN ? n : n_real;
  if (rows_counted > nb * block) rows_counted = nb * block;
  dim3 grid((unsigned)nb, (unsigned)(B * H));
  float* mu_o = mu + block_offset * d;
  float* var_o = var ? var + block_offset * d : nullptr;
  float* m3_o = m3 ? m3 + block_offset * d : nullptr;
  const char* xp = static_cast<const char*>(x);
  if (d == 64 || d == 128) {
    const dim3 gw((unsigned)((nb + 3) / 4), (unsigned)(B * H));
#define SSA_SUMMARY_WAVE(DT)                                                                      \
  do {                                                                                            \
    if (d == 64)                                                                                  \
      block_summary_wave_kernel<DT, 8><<<gw, 256, 0, stream>>>(xp, H, sb, sh, sn, block, n,      \
                                                               rows_counted, mode, mu_o, var_o,  \
                                                               m3_o, nb_out);                    \
    else                                                                                          \
      block_summary_wave_kernel<DT, 16><<<gw, 256, 0, stream>>>(xp, H, sb, sh, sn, block, n,     \
                                                                rows_counted, mode, mu_o, var_o, \
                                                                m3_o, nb_out);                   \
  } while (0)
    switch (dtype) {
      case SSA_F32: SSA_SUMMARY_WAVE(SSA_F32); break;
      case SSA_F16: SSA_SUMMARY_WAVE(SSA_F16); break;
      default: SSA_SUMMARY_WAVE(SSA_BF16); break;
    }
#undef SSA_SUMMARY_WAVE
    return launch_status("block_summary_wave_kernel");
  }
  switch (dtype) {
    case SSA_F32:
      block_summary_kernel<SSA_F32><<<grid, kSumThreads, 0, stream>>>(
          xp, H, (int)d, sb, sh, sn, block, n, rows_counted, mode, mu_o, var_o, m3_o, nb_out);
      break;
    case SSA_F16:
      block_summary_kernel<SSA_F16><<<grid, kSumThreads, 0, stream>>>(
          xp, H, (int)d, sb, sh, sn, block, n, rows_counted, mode, mu_o, var_o, m3_o, nb_out);
      break;
    default:
      block_summary_kernel<SSA_BF16><<<grid, kSumThreads, 0, stream>>>(
          xp, H, (int)d, sb, sh, sn, block, n, rows_counted, mode, mu_o, var_o, m3_o, nb_out);
      break;
  }
  return launch_status("block_summary_kernel");
}

int check_summary_args(const void* x, int dtype, int64_t B, int64_t H, int64_t n, int64_t d,
                       int64_t sb, int64_t sh, int64_t sn, int64_t block) {
  SSA_REQUIRE(x != nullptr, SSA_ERR_INVALID, "block_summary: x is NULL");
  SSA_REQUIRE(dtype_size(dtype) != 0, SSA_ERR_UNSUPPORTED, "block_summary: unknown dtype %d", dtype);
  SSA_REQUIRE(B > 0 && H > 0 && n > 0 && block > 0, SSA_ERR_INVALID,
              "block_summary: B=%lld H=%lld n=%lld block=%lld must be positive", (long long)B,
              (long long)H, (long long)n, (long long)block);
  SSA_REQUIRE(d % 8 == 0 && d >= 8 && d <= kMaxD, SSA_ERR_UNSUPPORTED,
              "block_summary: head_dim %lld unsupported (a multiple of 8, 8..512)",
              (long long)d);
  const int64_t vec = dtype == SSA_F32 ? 4 : 8;  // elements per 16 bytes
  SSA_REQUIRE(aligned16(x) && sb % vec == 0 && sh % vec == 0 && sn % vec == 0,
              SSA_ERR_UNSUPPORTED,
              "block_summary: x must be 16-byte aligned with strides multiple of 16 bytes");
  SSA_REQUIRE((n + block - 1) / block < (1ll << 31) && B * H < 65536, SSA_ERR_UNSUPPORTED,
              "block_summary: grid too large");
  return SSA_OK;
}

}  // namespace ssa

extern "C" int ssa_block_summary(const void* x, int dtype, int64_t B, int64_t H, int64_t n,
                                 int64_t d, int64_t stride_b, int64_t stride_h, int64_t stride_n,
                                 int64_t block, int64_t n_real, int mode, float* mu, float* var,
                                 float* m3, ssa_stream_t stream) {
  SSA_TRY(ssa::check_summary_args(x, dtype, B, H, n, d, stride_b, stride_h, stride_n, block));
  SSA_REQUIRE(mu != nullptr, SSA_ERR_INVALID, "block_summary: mu is NULL");
  SSA_REQUIRE(mode == SSA_STATS_POP || mode == SSA_STATS_UNBIASED || mode == SSA_STATS_QMEAN,
              SSA_ERR_INVALID, "block_summary: unknown mode %d", mode);
  SSA_REQUIRE(mode != SSA_STATS_QMEAN || (var == nullptr && m3 == nullptr), SSA_ERR_INVALID,
              "block_summary: QMEAN mode takes no var/m3 outputs");
  SSA_REQUIRE(n_real > 0, SSA_ERR_INVALID, "block_summary: n_real must be positive");
  const int64_t nb = (n + block - 1) / block;
  return ssa::launch_block_summary(x, dtype, B, H, n, d, stride_b, stride_h, stride_n, block,
                                   n_real, mode, mu, var, m3, nb, 0,
                                   static_cast<hipStream_t>(stream));
}
