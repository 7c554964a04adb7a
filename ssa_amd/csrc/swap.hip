// Tiled forward / backward of the per-row block-sparse softmax attention behind ssa_swap.ssa_masked
// (ssa/ssa_swap.py:32-56), head_dim 64, on v_mfma_f32_32x32x2_f32.
//
// Every query row i has its own selected key blocks (kv_num/kv_idx). The rows are grouped in
// query tiles of 64; row_block_masks_kernel turns the 64 rows' lists into one 64-bit word per
// (query tile, key block): bit r set iff row r of the tile selected the block. The attention
// kernels then walk 64-key tiles and skip a (query tile, key tile) pair whose words are all
// zero; inside a pair a (row, key) entry counts iff the row's bit is set for the key's block and
// key <= row (token causal).
//
//   swap_fwd_kernel   grid (B*Hq*nqt), one 64-row query tile per workgroup: S^T = K Q^T, online
//                     softmax per query column, O^T += V^T P^T; writes O and the row's
//                     natural-log lse.
//   swap_dq_kernel    same grid: recomputes P from lse, dP^T = V dO^T, dS = P (dP - D),
//                     dQ^T += K^T dS^T; also writes D_i = dO_i . O_i for the dk/dv pass.
//   swap_dkdv_kernel  grid (B*Hkv*nkt), one 64-key tile per workgroup, loops the G query heads
//                     and the query tiles at or after the key tile: S = Q K^T, dP = dO V^T,
//                     dV^T += dO^T P, dK^T += Q^T dS.
// Workgroups are issued longest first (the last query tiles, the first key tiles).
// The dq and dk/dv passes each own their outputs (no atomics, deterministic). Inputs of any
// dtype are staged through LDS as fp32; products and sums are fp32 (the reference trains the
// swap in fp32).
//
// MFMA operand layout (32x32x2 f32): lane l supplies A[l%32][l/32] and B[l/32][l%32]; the result
// lane l, register r holds C[(r/4)*8 + (l/32)*4 + r%4][l%32]. The contraction index k of a step
// is assigned freely to the two lane halves, as long as A and B agree: head-dim contractions use
// d = 32*(l/32) + t at step t (contiguous 16-byte LDS reads), key/query contractions use the
// rows the previous product's accumulators already hold in each half.
#include <math.h>

#include "common.h"

namespace ssa {

size_t masked_tiled_workspace(int64_t B, int64_t Hq, int64_t n, int64_t block);

namespace {

constexpr int kLS = 68;                 // LDS row stride (floats): conflict-free 16-byte reads
constexpr int kTileFloats = 64 * kLS;
constexpr int kMaxMaskBlocks = 8192;    // key blocks per sequence (LDS of the mask builder)
constexpr float kLog2eS = 1.4426950408889634f;
constexpr float kLn2S = 0.6931471805599453f;

struct SwapArgs {
  const char* q;
  const char* k;
  const char* v;
  char* o;
  const char* dout;  // strides of o
  float* lse;        // (B*Hq*n)
  float* delta;      // (B*Hq*n)
  void* dq;          // (B, Hq, n, 64) contiguous, fp32 or (grad16) the input type
  void* dk;          // (B, Hkv, n, 64)
  void* dv;
  bool grad16;       // gradients stored in the 16-bit input type (16-bit kernels only)
  int64_t qsb, qsh, qsn, ksb, ksh, ksn, vsb, vsh, vsn, osb, osh, osn;
  int64_t B, Hq, Hkv, G, n, block, nqt, nkt, nb;
  const int32_t* kv_num;
  const int32_t* kv_idx;
  int64_t W;
  unsigned long long* masks;  // (B*Hq, nqt, nb)
  float scale, scale_log2;
};

template <int DT>
__host__ __device__ constexpr int dtype_size_dev() {
  return DT == SSA_F32 ? 4 : 2;
}

__device__ inline f32x16 mfma(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ inline float pair_max(float x) { return fmaxf(x, __shfl_xor(x, 32, 64)); }
__device__ inline float pair_sum(float x) { return x + __shfl_xor(x, 32, 64); }

// 4 consecutive gradient values of a row: fp32, or rounded to the 16-bit input type DT
template <int DT>
__device__ inline void store_grad4(void* base, int64_t off, const f32x4& v, bool grad16) {
  if (DT != SSA_F32 && grad16) {
    unsigned int w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = DT == SSA_BF16 ? (unsigned int)__builtin_bit_cast(unsigned short, (__bf16)v[j])
                            : (unsigned int)__builtin_bit_cast(unsigned short, (_Float16)v[j]);
    uint2 u;
    u.x = w[0] | (w[1] << 16);
    u.y = w[2] | (w[3] << 16);
    *reinterpret_cast<uint2*>(static_cast<unsigned short*>(base) + off) = u;
  } else {
    *reinterpret_cast<f32x4*>(static_cast<float*>(base) + off) = v;
  }
}

// Stages rows [r0, r0 + 64) (rows >= nrows read as zeros) of a (rows, 64) matrix with row stride
// rs elements into LDS as fp32 with 256 threads: row-major into dst and/or transposed into dstT.
template <int DT>
__device__ inline void stage_tile(const char* base, int64_t rs, int64_t r0, int64_t nrows,
                                  float* dst, float* dstT, int tid) {
  if constexpr (DT == SSA_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i, row = c >> 4, col = (c & 15) * 4;
      f32x4 x = {0.0f, 0.0f, 0.0f, 0.0f};
      if (r0 + row < nrows)
        x = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(base) + (r0 + row) * rs + col);
      if (dst) *reinterpret_cast<f32x4*>(dst + row * kLS + col) = x;
      if (dstT) {
#pragma unroll
        for (int j = 0; j < 4; ++j) dstT[(col + j) * kLS + row] = x[j];
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + 256 * i, row = c >> 3, col = (c & 7) * 8;
      u32x4 w = {0u, 0u, 0u, 0u};
      if (r0 + row < nrows)
        w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const unsigned short*>(base) + (r0 + row) * rs + col);
      float f[8];
      unpack8(w, f, DT == SSA_BF16);
      if (dst) {
        *reinterpret_cast<f32x4*>(dst + row * kLS + col) = f32x4{f[0], f[1], f[2], f[3]};
        *reinterpret_cast<f32x4*>(dst + row * kLS + col + 4) = f32x4{f[4], f[5], f[6], f[7]};
      }
      if (dstT) {
#pragma unroll
        for (int j = 0; j < 8; ++j) dstT[(col + j) * kLS + row] = f[j];
      }
    }
  }
}

// 32 consecutive elements [c0, c0 + 32) of one row as fp32 (zeros when !valid).
template <int DT>
__device__ inline void load_row32(const char* base, int64_t off, bool valid, float* out) {
  if constexpr (DT == SSA_F32) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      f32x4 x = {0.0f, 0.0f, 0.0f, 0.0f};
      if (valid) x = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(base) + off + 4 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j) out[4 * i + j] = x[j];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (valid) w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const unsigned short*>(base) + off + 8 * i);
      unpack8(w, out + 8 * i, DT == SSA_BF16);
    }
  }
}

// Stores 4 consecutive fp32 values as DT.
template <int DT>
__device__ inline void store4(char* base, int64_t off, float a, float b, float c, float d) {
  if constexpr (DT == SSA_F32) {
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(base) + off) = f32x4{a, b, c, d};
  } else {
    unsigned short u[4];
    const float x[4] = {a, b, c, d};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (DT == SSA_BF16) u[j] = __builtin_bit_cast(unsigned short, (__bf16)x[j]);
      else u[j] = __builtin_bit_cast(unsigned short, (_Float16)x[j]);
    }
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<u32x2*>(reinterpret_cast<unsigned short*>(base) + off) =
        u32x2{(unsigned)u[0] | ((unsigned)u[1] << 16), (unsigned)u[2] | ((unsigned)u[3] << 16)};
  }
}

// Bits [lo, hi) of a 64-bit word (0 <= lo <= hi <= 64).
__device__ inline unsigned long long bit_range(int lo, int hi) {
  if (hi <= lo) return 0ull;
  const unsigned long long upto = hi >= 64 ? ~0ull : ((1ull << hi) - 1ull);
  return upto & ~((1ull << lo) - 1ull);
}

// For the key tile [k0, k0 + 64): OR of the tile's block words of one query tile (`any`), and
// the keys of the tile selected by query-tile row `r` (bit j = key k0 + j; r < 0: none).
__device__ inline void tile_bits(const unsigned long long* mrow, int64_t k0, int64_t block,
                                 int64_t nb, int r, unsigned long long& any,
                                 unsigned long long& keys) {
  const int64_t c0 = k0 / block;
  int64_t c1 = (k0 + 63) / block;
  if (c1 > nb - 1) c1 = nb - 1;
  any = 0ull;
  keys = 0ull;
  for (int64_t c = c0; c <= c1; ++c) {
    const unsigned long long w = mrow[c];
    any |= w;
    if (r >= 0 && ((w >> r) & 1ull)) {
      const int64_t a = c * block - k0, e = (c + 1) * block - k0;
      keys |= bit_range(a < 0 ? 0 : (int)a, e > 64 ? 64 : (int)e);
    }
  }
}

// grid (B*Hq*nqt), 256 threads: the (query tile, key block) words from the rows' lists.
__global__ __launch_bounds__(256) void row_block_masks_kernel(SwapArgs a) {
  __shared__ unsigned long long mk[kMaxMaskBlocks];
  const int tid = threadIdx.x;
  const int64_t qt = blockIdx.x % a.nqt, bh = blockIdx.x / a.nqt;
  for (int64_t c = tid; c < a.nb; c += 256) mk[c] = 0ull;
  __syncthreads();
  const int64_t q0 = qt * 64;
  for (int64_t idx = tid; idx < 64 * a.W; idx += 256) {
    const int r = (int)(idx / a.W);
    const int64_t j = idx % a.W, row = q0 + r;
    if (row >= a.n) continue;
    const int64_t rid = bh * a.n + row;
    int64_t cnt = a.kv_num[rid];
    if (cnt > a.W) cnt = a.W;
    if (j >= cnt) continue;
    const int64_t c = a.kv_idx[rid * a.W + j];
    if (c < 0 || c >= a.nb || c * a.block > row) continue;  // out of range / not begun: no keys
    atomicOr(&mk[c], 1ull << r);
  }
  __syncthreads();
  unsigned long long* out = a.masks + (bh * a.nqt + qt) * a.nb;
  for (int64_t c = tid; c < a.nb; c += 256) out[c] = mk[c];
}

// Workgroup layout of the three attention kernels: 4 waves, wave w = (x = w & 1, y = w >> 1).
// fwd / dq: x picks the 32 query rows of the 64-row tile, y the 32 keys of each 64-key tile the
// wave contracts over; the two y halves keep separate softmax / gradient state and are merged
// through LDS at the end. dk/dv: x picks the 32 keys, y the 32 query rows of each query tile.

template <int DT>
__global__ __launch_bounds__(256) void swap_fwd_kernel(SwapArgs a) {
  __shared__ float ks[kTileFloats];  // K tile [key][d]
  __shared__ float vt[kTileFloats];  // V tile [d][key]
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hi = lane >> 5, lo = lane & 31;
  const int qh = w & 1, kh = w >> 1;
  const int64_t nbh = a.B * a.Hq;
  const int64_t bh = blockIdx.x % nbh, qt = a.nqt - 1 - blockIdx.x / nbh;  // longest rows first
  const int64_t b = bh / a.Hq, h = bh % a.Hq, kvh = h / a.G;
  const int64_t q0 = qt * 64;
  const int r = 32 * qh + lo;  // this lane's query row in the tile
  const int64_t qi = q0 + r;
  const bool qvalid = qi < a.n;
  float qreg[32];
  load_row32<DT>(a.q, b * a.qsb + h * a.qsh + qi * a.qsn + 32 * hi, qvalid, qreg);
  const unsigned long long* mrow = a.masks + (bh * a.nqt + qt) * a.nb;
  const char* kb = a.k + (b * a.ksb + kvh * a.ksh) * dtype_size_dev<DT>();
  const char* vb = a.v + (b * a.vsb + kvh * a.vsh) * dtype_size_dev<DT>();
  const float sl2 = a.scale_log2;

  float m = -INFINITY, l = 0.0f;
  f32x16 o[2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[x][e] = 0.0f;
  int64_t qlast = q0 + 63;
  if (qlast > a.n - 1) qlast = a.n - 1;
  const int64_t nkt = qlast / 64 + 1;
  for (int64_t kt = 0; kt < nkt; ++kt) {
    const int64_t k0 = kt * 64;
    unsigned long long any, keys;
    tile_bits(mrow, k0, a.block, a.nb, qvalid ? r : -1, any, keys);
    if (any == 0ull) continue;  // same words for every lane: uniform
    __syncthreads();
    stage_tile<DT>(kb, a.ksn, k0, a.n, ks, nullptr, tid);
    stage_tile<DT>(vb, a.vsn, k0, a.n, nullptr, vt, tid);
    __syncthreads();

    f32x16 s;
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = 0.0f;
#pragma unroll
    for (int t4 = 0; t4 < 8; ++t4) {
      const f32x4 a4 = *reinterpret_cast<const f32x4*>(ks + (32 * kh + lo) * kLS + 32 * hi + 4 * t4);
#pragma unroll
      for (int j = 0; j < 4; ++j) s = mfma(a4[j], qreg[4 * t4 + j], s);
    }
    // key of register e: 32*kh + (e/4)*8 + hi*4 + e%4
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int kk = 32 * kh + (e >> 2) * 8 + hi * 4 + (e & 3);
      const bool ok = ((keys >> kk) & 1ull) && (k0 + kk <= qi);
      s[e] = ok ? s[e] * sl2 : -INFINITY;
      mx = fmaxf(mx, s[e]);
    }
    mx = pair_max(mx);
    const float mnew = fmaxf(m, mx);
    const float alpha = mnew == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - mnew);
    float ps = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float p = s[e] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s[e] - mnew);
      s[e] = p;
      ps += p;
    }
    l = l * alpha + ps;
    m = mnew;
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[x][e] *= alpha;
#pragma unroll
    for (int dh = 0; dh < 2; ++dh)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 a4 = *reinterpret_cast<const f32x4*>(vt + (32 * dh + lo) * kLS + 32 * kh + 8 * g + 4 * hi);
#pragma unroll
        for (int j = 0; j < 4; ++j) o[dh] = mfma(a4[j], s[4 * g + j], o[dh]);
      }
  }
  l = pair_sum(l);
  // merge the two key halves: (m, l, O^T) of the kh = 1 waves through LDS
  __syncthreads();
  float* buf = ks;  // 34 x 128 floats
  const int slot = qh * 64 + lane;
  if (kh == 1) {
    buf[slot] = m;
    buf[128 + slot] = l;
#pragma unroll
    for (int x = 0; x < 32; ++x) buf[(2 + x) * 128 + slot] = o[x >> 4][x & 15];
  }
  __syncthreads();
  if (kh == 1 || !qvalid) return;
  const float m1 = buf[slot], l1 = buf[128 + slot];
  const float M = fmaxf(m, m1);
  const float a0 = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - M);
  const float a1 = m1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m1 - M);
  const float lt = l * a0 + l1 * a1;
  const float inv = 1.0f / lt;
  float of[32];
#pragma unroll
  for (int x = 0; x < 32; ++x) of[x] = (o[x >> 4][x & 15] * a0 + buf[(2 + x) * 128 + slot] * a1) * inv;
  const int64_t ooff = b * a.osb + h * a.osh + qi * a.osn;
#pragma unroll
  for (int dh = 0; dh < 2; ++dh)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * dh + 8 * g + 4 * hi, x = 16 * dh + 4 * g;
      store4<DT>(a.o, ooff + d0, of[x], of[x + 1], of[x + 2], of[x + 3]);
    }
  if (hi == 0) a.lse[bh * a.n + qi] = (M + log2f(lt)) * kLn2S;
}

template <int DT>
__global__ __launch_bounds__(256, 2) void swap_dq_kernel(SwapArgs a) {
  __shared__ float ks[kTileFloats];   // K [key][d]
  __shared__ float vs[kTileFloats];   // V [key][d]
  __shared__ float kt_[kTileFloats];  // K [d][key]
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hi = lane >> 5, lo = lane & 31;
  const int qh = w & 1, kh = w >> 1;
  const int64_t nbh = a.B * a.Hq;
  const int64_t bh = blockIdx.x % nbh, qt = a.nqt - 1 - blockIdx.x / nbh;
  const int64_t b = bh / a.Hq, h = bh % a.Hq, kvh = h / a.G;
  const int64_t q0 = qt * 64;
  const int r = 32 * qh + lo;
  const int64_t qi = q0 + r;
  const bool qvalid = qi < a.n;
  float qreg[32], greg[32];
  load_row32<DT>(a.q, b * a.qsb + h * a.qsh + qi * a.qsn + 32 * hi, qvalid, qreg);
  const int64_t ooff = b * a.osb + h * a.osh + qi * a.osn + 32 * hi;
  load_row32<DT>(a.dout, ooff, qvalid, greg);
  float Di;
  {
    float orow[32];
    load_row32<DT>(a.o, ooff, qvalid, orow);
    float acc = 0.0f;
#pragma unroll
    for (int t = 0; t < 32; ++t) acc = fmaf(greg[t], orow[t], acc);
    Di = pair_sum(acc);
  }
  const int64_t rid = bh * a.n + qi;
  const float lse2 = qvalid ? a.lse[rid] * kLog2eS : 0.0f;
  if (qvalid && kh == 0 && hi == 0) a.delta[rid] = Di;
  const unsigned long long* mrow = a.masks + (bh * a.nqt + qt) * a.nb;
  const char* kb = a.k + (b * a.ksb + kvh * a.ksh) * dtype_size_dev<DT>();
  const char* vb = a.v + (b * a.vsb + kvh * a.vsh) * dtype_size_dev<DT>();
  const float sl2 = a.scale_log2;

  f32x16 dqa[2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int e = 0; e < 16; ++e) dqa[x][e] = 0.0f;
  int64_t qlast = q0 + 63;
  if (qlast > a.n - 1) qlast = a.n - 1;
  const int64_t nkt = qlast / 64 + 1;
  for (int64_t kt = 0; kt < nkt; ++kt) {
    const int64_t k0 = kt * 64;
    unsigned long long any, keys;
    tile_bits(mrow, k0, a.block, a.nb, qvalid ? r : -1, any, keys);
    if (any == 0ull) continue;
    __syncthreads();
    stage_tile<DT>(kb, a.ksn, k0, a.n, ks, kt_, tid);
    stage_tile<DT>(vb, a.vsn, k0, a.n, vs, nullptr, tid);
    __syncthreads();

    f32x16 s, dp;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      s[e] = 0.0f;
      dp[e] = 0.0f;
    }
#pragma unroll
    for (int t4 = 0; t4 < 8; ++t4) {
      const f32x4 a4 = *reinterpret_cast<const f32x4*>(ks + (32 * kh + lo) * kLS + 32 * hi + 4 * t4);
      const f32x4 b4 = *reinterpret_cast<const f32x4*>(vs + (32 * kh + lo) * kLS + 32 * hi + 4 * t4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s = mfma(a4[j], qreg[4 * t4 + j], s);
        dp = mfma(b4[j], greg[4 * t4 + j], dp);
      }
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int kk = 32 * kh + (e >> 2) * 8 + hi * 4 + (e & 3);
      const bool ok = ((keys >> kk) & 1ull) && (k0 + kk <= qi);
      const float p = ok ? __builtin_amdgcn_exp2f(fmaf(s[e], sl2, -lse2)) : 0.0f;
      s[e] = p * (dp[e] - Di);  // dS^T
    }
#pragma unroll
    for (int dh = 0; dh < 2; ++dh)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 a4 = *reinterpret_cast<const f32x4*>(kt_ + (32 * dh + lo) * kLS + 32 * kh + 8 * g + 4 * hi);
#pragma unroll
        for (int j = 0; j < 4; ++j) dqa[dh] = mfma(a4[j], s[4 * g + j], dqa[dh]);
      }
  }
  __syncthreads();
  float* buf = ks;  // 32 x 128 floats
  const int slot = qh * 64 + lane;
  if (kh == 1) {
#pragma unroll
    for (int x = 0; x < 32; ++x) buf[x * 128 + slot] = dqa[x >> 4][x & 15];
  }
  __syncthreads();
  if (kh == 1 || !qvalid) return;
#pragma unroll
  for (int dh = 0; dh < 2; ++dh)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * dh + 8 * g + 4 * hi, x = 16 * dh + 4 * g;
      f32x4 val;
#pragma unroll
      for (int j = 0; j < 4; ++j) val[j] = (dqa[dh][4 * g + j] + buf[(x + j) * 128 + slot]) * a.scale;
      store_grad4<SSA_F32>(a.dq, rid * 64 + d0, val, false);
    }
}

// The next query tile >= qt (in order) holding a selected (row, key) pair of key tile k0 for
// head bh, or a.nqt. The workgroup's 256 threads test 256 tiles at a time into a bitmap in
// LDS (act: 4 words; chunk: the first tile of the bitmap held, -1 at first), so a walk over
// mostly unselected tiles costs one round of loads per 256 tiles. Called uniformly.
__device__ inline int64_t next_active_tile(const SwapArgs& a, int64_t bh, int64_t k0, int64_t qt,
                                           unsigned long long* act, int64_t& chunk) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  while (qt < a.nqt) {
    const int64_t c0 = qt & ~int64_t(255);
    if (c0 != chunk) {
      const int64_t t = c0 + tid;
      bool on = false;
      if (t >= k0 / 64 && t < a.nqt) {
        unsigned long long any, unused;
        tile_bits(a.masks + (bh * a.nqt + t) * a.nb, k0, a.block, a.nb, -1, any, unused);
        on = any != 0ull;
      }
      const unsigned long long bal = __ballot(on);
      __syncthreads();  // the previous bitmap is no longer read
      if (lane == 0) act[w] = bal;
      __syncthreads();
      chunk = c0;
    }
    const int r = (int)(qt - c0);
    const unsigned long long rest = act[r >> 6] & (~0ull << (r & 63));
    if (rest != 0ull) return c0 + (r & ~63) + (int64_t)__builtin_ctzll(rest);
    qt = c0 + (r & ~63) + 64;  // no active tile left in this 64-tile word
  }
  return a.nqt;
}

template <int DT>
__global__ __launch_bounds__(256, 2) void swap_dkdv_kernel(SwapArgs a) {
  __shared__ float qs[kTileFloats];   // Q [q][d]
  __shared__ float gs[kTileFloats];   // dO [q][d]
  __shared__ float qtT[kTileFloats];  // Q [d][q]
  __shared__ float gtT[kTileFloats];  // dO [d][q]
  __shared__ float lse_s[64], del_s[64];
  __shared__ unsigned long long act_s[4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hi = lane >> 5, lo = lane & 31;
  const int kq = w & 1, qp = w >> 1;
  const int64_t nbkv = a.B * a.Hkv;
  const int64_t bkv = blockIdx.x % nbkv, kt = blockIdx.x / nbkv;  // most query tiles first
  const int64_t b = bkv / a.Hkv, kvh = bkv % a.Hkv;
  const int64_t k0 = kt * 64;
  const int64_t key = k0 + 32 * kq + lo;
  const bool kvalid = key < a.n;
  float kreg[32], vreg[32];
  load_row32<DT>(a.k, b * a.ksb + kvh * a.ksh + key * a.ksn + 32 * hi, kvalid, kreg);
  load_row32<DT>(a.v, b * a.vsb + kvh * a.vsh + key * a.vsn + 32 * hi, kvalid, vreg);
  const int64_t ck = kvalid ? key / a.block : 0;
  const float sl2 = a.scale_log2;

  f32x16 dka[2], dva[2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      dka[x][e] = 0.0f;
      dva[x][e] = 0.0f;
    }
  for (int64_t g = 0; g < a.G; ++g) {
    const int64_t hq = kvh * a.G + g, bh = b * a.Hq + hq;
    const char* qb = a.q + (b * a.qsb + hq * a.qsh) * dtype_size_dev<DT>();
    const char* gb = a.dout + (b * a.osb + hq * a.osh) * dtype_size_dev<DT>();
    int64_t chunk = -1;
    for (int64_t qt = next_active_tile(a, bh, k0, k0 / 64, act_s, chunk); qt < a.nqt;
         qt = next_active_tile(a, bh, k0, qt + 1, act_s, chunk)) {
      const unsigned long long* mrow = a.masks + (bh * a.nqt + qt) * a.nb;
      const unsigned long long mw = kvalid ? mrow[ck] : 0ull;
      const int64_t q0 = qt * 64;
      __syncthreads();
      stage_tile<DT>(qb, a.qsn, q0, a.n, qs, qtT, tid);
      stage_tile<DT>(gb, a.osn, q0, a.n, gs, gtT, tid);
      if (tid < 64) {
        const bool ok = q0 + tid < a.n;
        lse_s[tid] = ok ? a.lse[bh * a.n + q0 + tid] * kLog2eS : 0.0f;
        del_s[tid] = ok ? a.delta[bh * a.n + q0 + tid] : 0.0f;
      }
      __syncthreads();

      f32x16 s, dp;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        s[e] = 0.0f;
        dp[e] = 0.0f;
      }
#pragma unroll
      for (int t4 = 0; t4 < 8; ++t4) {
        const f32x4 a4 = *reinterpret_cast<const f32x4*>(qs + (32 * qp + lo) * kLS + 32 * hi + 4 * t4);
        const f32x4 b4 = *reinterpret_cast<const f32x4*>(gs + (32 * qp + lo) * kLS + 32 * hi + 4 * t4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          s = mfma(a4[j], kreg[4 * t4 + j], s);
          dp = mfma(b4[j], vreg[4 * t4 + j], dp);
        }
      }
      // query row of register e: 32*qp + (e/4)*8 + hi*4 + e%4 of the tile
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int qq = 32 * qp + (e >> 2) * 8 + hi * 4 + (e & 3);
        const bool ok = ((mw >> qq) & 1ull) && (key <= q0 + qq);
        const float p = ok ? __builtin_amdgcn_exp2f(fmaf(s[e], sl2, -lse_s[qq])) : 0.0f;
        s[e] = p;
        dp[e] = p * (dp[e] - del_s[qq]);  // dS
      }
#pragma unroll
      for (int dh = 0; dh < 2; ++dh)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int off = (32 * dh + lo) * kLS + 32 * qp + 8 * g4 + 4 * hi;
          const f32x4 ga = *reinterpret_cast<const f32x4*>(gtT + off);
          const f32x4 qa = *reinterpret_cast<const f32x4*>(qtT + off);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            dva[dh] = mfma(ga[j], s[4 * g4 + j], dva[dh]);
            dka[dh] = mfma(qa[j], dp[4 * g4 + j], dka[dh]);
          }
        }
    }
  }
  __syncthreads();
  float* bk = qs;  // 32 x 128 floats each
  float* bv = gs;
  const int slot = kq * 64 + lane;
  if (qp == 1) {
#pragma unroll
    for (int x = 0; x < 32; ++x) {
      bk[x * 128 + slot] = dka[x >> 4][x & 15];
      bv[x * 128 + slot] = dva[x >> 4][x & 15];
    }
  }
  __syncthreads();
  if (qp == 1 || !kvalid) return;
  const int64_t krow = (bkv * a.n + key) * 64;
#pragma unroll
  for (int dh = 0; dh < 2; ++dh)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * dh + 8 * g + 4 * hi, x = 16 * dh + 4 * g;
      f32x4 kv4, vv4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        kv4[j] = (dka[dh][4 * g + j] + bk[(x + j) * 128 + slot]) * a.scale;
        vv4[j] = dva[dh][4 * g + j] + bv[(x + j) * 128 + slot];
      }
      store_grad4<SSA_F32>(a.dk, krow + d0, kv4, false);
      store_grad4<SSA_F32>(a.dv, krow + d0, vv4, false);
    }
}

// ---- 16-bit inputs: v_mfma_f32_32x32x16_{bf16,f16} ------------------------------------------
// Tiles stay 16-bit in LDS (row-major stride kRS16, transposed stride kTS16 halves); P and dS are
// rounded to the input type for the second products, as flash attention does. Operand layout
// (32x32x16): lane l supplies A[l%32][8*(l/32) + j] and B[8*(l/32) + j][l%32], j = 0..7.
// Head-dim steps t = 0..3 use d = 32*(l/32) + 8t + j; key (query) steps u = 0..1 over a wave's
// 32 accumulator rows use the rows its registers e = 8u + j hold: 16u + 8*(j/4) + 4*(l/32) + j%4.

constexpr int kRS16 = 72;  // 144 B rows: conflict-free 16-byte reads
constexpr int kTS16 = 68;  // 136 B rows: conflict-free 8-byte reads

template <int DT>
struct Mma16;
template <>
struct Mma16<SSA_BF16> {
  typedef bf16x8 vec;
  __device__ static f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(vec, a),
                                                   __builtin_bit_cast(vec, b), c, 0, 0, 0);
  }
  __device__ static unsigned int bits(float x) { return __builtin_bit_cast(unsigned short, (__bf16)x); }
};
template <>
struct Mma16<SSA_F16> {
  typedef f16x8 vec;
  __device__ static f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(vec, a),
                                                  __builtin_bit_cast(vec, b), c, 0, 0, 0);
  }
  __device__ static unsigned int bits(float x) { return __builtin_bit_cast(unsigned short, (_Float16)x); }
};

// 8 fp32 values (x[0..7]) rounded and packed as one 16-byte operand
template <int DT>
__device__ inline u32x4 pack8(const float* x) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = Mma16<DT>::bits(x[2 * i]) | (Mma16<DT>::bits(x[2 * i + 1]) << 16);
  return r;
}

// Stages rows [r0, r0 + 64) of a 16-bit (rows, 64) matrix without conversion (256 threads).
__device__ inline void stage16(const char* base, int64_t rs, int64_t r0, int64_t nrows,
                               unsigned short* dst, unsigned short* dstT, int tid) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = tid + 256 * i, row = c >> 3, col = (c & 7) * 8;
    u32x4 w = {0u, 0u, 0u, 0u};
    if (r0 + row < nrows)
      w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const unsigned short*>(base) + (r0 + row) * rs + col);
    if (dst) *reinterpret_cast<u32x4*>(dst + row * kRS16 + col) = w;
    if (dstT) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        dstT[(col + j) * kTS16 + row] = (unsigned short)((j & 1) ? (w[j >> 1] >> 16) : (w[j >> 1] & 0xffffu));
    }
  }
}

__device__ inline u32x4 lds16(const unsigned short* p) { return *reinterpret_cast<const u32x4*>(p); }
// halves p[0..3] and p[8..11] of a transposed tile row
__device__ inline u32x4 lds_pair(const unsigned short* p) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 x = *reinterpret_cast<const u32x2*>(p), y = *reinterpret_cast<const u32x2*>(p + 8);
  return u32x4{x[0], x[1], y[0], y[1]};
}

// one row's 32 halves [32*hi, 32*hi + 32) as 4 packed operands (zeros when !valid)
__device__ inline void load_row16(const char* base, int64_t off, bool valid, u32x4* out) {
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    u32x4 w = {0u, 0u, 0u, 0u};
    if (valid) w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const unsigned short*>(base) + off + 8 * t);
    out[t] = w;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void swap_fwd16_kernel(SwapArgs a) {
  // K and V^T tiles (17920 B), later the 34 x 128-float merge buffer (17408 B)
  __shared__ __attribute__((aligned(16))) char smem[64 * kRS16 * 2 + 64 * kTS16 * 2];
  static_assert(64 * kRS16 * 2 + 64 * kTS16 * 2 >= 34 * 128 * 4, "merge buffer");
  unsigned short* ks = reinterpret_cast<unsigned short*>(smem);  // K [key][d]
  unsigned short* vt = ks + 64 * kRS16;                          // V [d][key]
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hi = lane >> 5, lo = lane & 31;
  const int qh = w & 1, kh = w >> 1;
  const int64_t nbh = a.B * a.Hq;
  const int64_t bh = blockIdx.x % nbh, qt = a.nqt - 1 - blockIdx.x / nbh;
  const int64_t b = bh / a.Hq, h = bh % a.Hq, kvh = h / a.G;
  const int64_t q0 = qt * 64;
  const int r = 32 * qh + lo;
  const int64_t qi = q0 + r;
  const bool qvalid = qi < a.n;
  u32x4 qv[4];
  load_row16(a.q, b * a.qsb + h * a.qsh + qi * a.qsn + 32 * hi, qvalid, qv);
  const unsigned long long* mrow = a.masks + (bh * a.nqt + qt) * a.nb;
  const char* kb = a.k + (b * a.ksb + kvh * a.ksh) * 2;
  const char* vb = a.v + (b * a.vsb + kvh * a.vsh) * 2;
  const float sl2 = a.scale_log2;

  float m = -INFINITY, l = 0.0f;
  f32x16 o[2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[x][e] = 0.0f;
  int64_t qlast = q0 + 63;
  if (qlast > a.n - 1) qlast = a.n - 1;
  const int64_t nkt = qlast / 64 + 1;
  for (int64_t kt = 0; kt < nkt; ++kt) {
    const int64_t k0 = kt * 64;
    unsigned long long any, keys;
    tile_bits(mrow, k0, a.block, a.nb, qvalid ? r : -1, any, keys);
    if (any == 0ull) continue;
    __syncthreads();
    stage16(kb, a.ksn, k0, a.n, ks, nullptr, tid);
    stage16(vb, a.vsn, k0, a.n, nullptr, vt, tid);
    __syncthreads();
    f32x16 s;
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      s = Mma16<DT>::mma(lds16(ks + (32 * kh + lo) * kRS16 + 32 * hi + 8 * t), qv[t], s);
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int kk = 32 * kh + (e >> 2) * 8 + hi * 4 + (e & 3);
      const bool ok = ((keys >> kk) & 1ull) && (k0 + kk <= qi);
      s[e] = ok ? s[e] * sl2 : -INFINITY;
      mx = fmaxf(mx, s[e]);
    }
    mx = pair_max(mx);
    const float mnew = fmaxf(m, mx);
    const float alpha = mnew == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - mnew);
    float p[16];
    float ps = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      p[e] = s[e] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s[e] - mnew);
      ps += p[e];
    }
    l = l * alpha + ps;
    m = mnew;
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[x][e] *= alpha;
    const u32x4 p0 = pack8<DT>(p), p1 = pack8<DT>(p + 8);
#pragma unroll
    for (int dh = 0; dh < 2; ++dh) {
      const unsigned short* vrow = vt + (32 * dh + lo) * kTS16 + 32 * kh + 4 * hi;
      o[dh] = Mma16<DT>::mma(lds_pair(vrow), p0, o[dh]);
      o[dh] = Mma16<DT>::mma(lds_pair(vrow + 16), p1, o[dh]);
    }
  }
  l = pair_sum(l);
  __syncthreads();
  float* buf = reinterpret_cast<float*>(smem);  // 34 x 128 floats
  const int slot = qh * 64 + lane;
  if (kh == 1) {
    buf[slot] = m;
    buf[128 + slot] = l;
#pragma unroll
    for (int x = 0; x < 32; ++x) buf[(2 + x) * 128 + slot] = o[x >> 4][x & 15];
  }
  __syncthreads();
  if (kh == 1 || !qvalid) return;
  const float m1 = buf[slot], l1 = buf[128 + slot];
  const float M = fmaxf(m, m1);
  const float a0 = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - M);
  const float a1 = m1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m1 - M);
  const float lt = l * a0 + l1 * a1;
  const float inv = 1.0f / lt;
  float of[32];
#pragma unroll
  for (int x = 0; x < 32; ++x) of[x] = (o[x >> 4][x & 15] * a0 + buf[(2 + x) * 128 + slot] * a1) * inv;
  const int64_t ooff = b * a.osb + h * a.osh + qi * a.osn;
#pragma unroll
  for (int dh = 0; dh < 2; ++dh)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * dh + 8 * g + 4 * hi, x = 16 * dh + 4 * g;
      store4<DT>(a.o, ooff + d0, of[x], of[x + 1], of[x + 2], of[x + 3]);
    }
  if (hi == 0) a.lse[bh * a.n + qi] = (M + log2f(lt)) * kLn2S;
}

template <int DT>
__global__ __launch_bounds__(256) void swap_dq16_kernel(SwapArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[2 * 64 * kRS16 * 2 + 64 * kTS16 * 2];
  static_assert(2 * 64 * kRS16 * 2 + 64 * kTS16 * 2 >= 32 * 128 * 4, "merge buffer");
  unsigned short* ks = reinterpret_cast<unsigned short*>(smem);  // K [key][d]
  unsigned short* vs = ks + 64 * kRS16;                          // V [key][d]
  unsigned short* kt_ = vs + 64 * kRS16;                         // K [d][key]
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hi = lane >> 5, lo = lane & 31;
  const int qh = w & 1, kh = w >> 1;
  const int64_t nbh = a.B * a.Hq;
  const int64_t bh = blockIdx.x % nbh, qt = a.nqt - 1 - blockIdx.x / nbh;
  const int64_t b = bh / a.Hq, h = bh % a.Hq, kvh = h / a.G;
  const int64_t q0 = qt * 64;
  const int r = 32 * qh + lo;
  const int64_t qi = q0 + r;
  const bool qvalid = qi < a.n;
  u32x4 qv[4], gv[4];
  load_row16(a.q, b * a.qsb + h * a.qsh + qi * a.qsn + 32 * hi, qvalid, qv);
  const int64_t ooff = b * a.osb + h * a.osh + qi * a.osn + 32 * hi;
  load_row16(a.dout, ooff, qvalid, gv);
  float Di;
  {
    float orow[32], grow[32];
    load_row32<DT>(a.o, ooff, qvalid, orow);
#pragma unroll
    for (int t = 0; t < 4; ++t) unpack8(gv[t], grow + 8 * t, DT == SSA_BF16);
    float acc = 0.0f;
#pragma unroll
    for (int t = 0; t < 32; ++t) acc = fmaf(grow[t], orow[t], acc);
    Di = pair_sum(acc);
  }
  const int64_t rid = bh * a.n + qi;
  const float lse2 = qvalid ? a.lse[rid] * kLog2eS : 0.0f;
  if (qvalid && kh == 0 && hi == 0) a.delta[rid] = Di;
  const unsigned long long* mrow = a.masks + (bh * a.nqt + qt) * a.nb;
  const char* kb = a.k + (b * a.ksb + kvh * a.ksh) * 2;
  const char* vb = a.v + (b * a.vsb + kvh * a.vsh) * 2;
  const float sl2 = a.scale_log2;

  f32x16 dqa[2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int e = 0; e < 16; ++e) dqa[x][e] = 0.0f;
  int64_t qlast = q0 + 63;
  if (qlast > a.n - 1) qlast = a.n - 1;
  const int64_t nkt = qlast / 64 + 1;
  for (int64_t kt = 0; kt < nkt; ++kt) {
    const int64_t k0 = kt * 64;
    unsigned long long any, keys;
    tile_bits(mrow, k0, a.block, a.nb, qvalid ? r : -1, any, keys);
    if (any == 0ull) continue;
    __syncthreads();
    stage16(kb, a.ksn, k0, a.n, ks, kt_, tid);
    stage16(vb, a.vsn, k0, a.n, vs, nullptr, tid);
    __syncthreads();
    f32x16 s, dp;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      s[e] = 0.0f;
      dp[e] = 0.0f;
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int off = (32 * kh + lo) * kRS16 + 32 * hi + 8 * t;
      s = Mma16<DT>::mma(lds16(ks + off), qv[t], s);
      dp = Mma16<DT>::mma(lds16(vs + off), gv[t], dp);
    }
    float ds[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int kk = 32 * kh + (e >> 2) * 8 + hi * 4 + (e & 3);
      const bool ok = ((keys >> kk) & 1ull) && (k0 + kk <= qi);
      const float p = ok ? __builtin_amdgcn_exp2f(fmaf(s[e], sl2, -lse2)) : 0.0f;
      ds[e] = p * (dp[e] - Di);
    }
    const u32x4 d0 = pack8<DT>(ds), d1 = pack8<DT>(ds + 8);
#pragma unroll
    for (int dh = 0; dh < 2; ++dh) {
      const unsigned short* krow = kt_ + (32 * dh + lo) * kTS16 + 32 * kh + 4 * hi;
      dqa[dh] = Mma16<DT>::mma(lds_pair(krow), d0, dqa[dh]);
      dqa[dh] = Mma16<DT>::mma(lds_pair(krow + 16), d1, dqa[dh]);
    }
  }
  __syncthreads();
  float* buf = reinterpret_cast<float*>(smem);  // 32 x 128 floats
  const int slot = qh * 64 + lane;
  if (kh == 1) {
#pragma unroll
    for (int x = 0; x < 32; ++x) buf[x * 128 + slot] = dqa[x >> 4][x & 15];
  }
  __syncthreads();
  if (kh == 1 || !qvalid) return;
#pragma unroll
  for (int dh = 0; dh < 2; ++dh)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int dd = 32 * dh + 8 * g + 4 * hi, x = 16 * dh + 4 * g;
      f32x4 val;
#pragma unroll
      for (int j = 0; j < 4; ++j) val[j] = (dqa[dh][4 * g + j] + buf[(x + j) * 128 + slot]) * a.scale;
      store_grad4<DT>(a.dq, rid * 64 + dd, val, a.grad16);
    }
}

template <int DT>
__global__ __launch_bounds__(256, 2) void swap_dkdv16_kernel(SwapArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[2 * 64 * kRS16 * 2 + 2 * 64 * kTS16 * 2];
  static_assert(2 * 64 * kRS16 * 2 + 2 * 64 * kTS16 * 2 >= 2 * 32 * 128 * 4, "merge buffers");
  __shared__ float lse_s[64], del_s[64];
  __shared__ unsigned long long act_s[4];
  unsigned short* qs = reinterpret_cast<unsigned short*>(smem);  // Q [q][d]
  unsigned short* gs = qs + 64 * kRS16;                          // dO [q][d]
  unsigned short* qtT = gs + 64 * kRS16;                         // Q [d][q]
  unsigned short* gtT = qtT + 64 * kTS16;                        // dO [d][q]
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hi = lane >> 5, lo = lane & 31;
  const int kq = w & 1, qp = w >> 1;
  const int64_t nbkv = a.B * a.Hkv;
  const int64_t bkv = blockIdx.x % nbkv, kt = blockIdx.x / nbkv;
  const int64_t b = bkv / a.Hkv, kvh = bkv % a.Hkv;
  const int64_t k0 = kt * 64;
  const int64_t key = k0 + 32 * kq + lo;
  const bool kvalid = key < a.n;
  u32x4 kv[4], vv[4];
  load_row16(a.k, b * a.ksb + kvh * a.ksh + key * a.ksn + 32 * hi, kvalid, kv);
  load_row16(a.v, b * a.vsb + kvh * a.vsh + key * a.vsn + 32 * hi, kvalid, vv);
  const int64_t ck = kvalid ? key / a.block : 0;
  const float sl2 = a.scale_log2;

  f32x16 dka[2], dva[2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      dka[x][e] = 0.0f;
      dva[x][e] = 0.0f;
    }
  for (int64_t g = 0; g < a.G; ++g) {
    const int64_t hq = kvh * a.G + g, bh = b * a.Hq + hq;
    const char* qb = a.q + (b * a.qsb + hq * a.qsh) * 2;
    const char* gb = a.dout + (b * a.osb + hq * a.osh) * 2;
    int64_t chunk = -1;
    int64_t qt = next_active_tile(a, bh, k0, k0 / 64, act_s, chunk);
    while (qt < a.nqt) {
      const int64_t nxt = next_active_tile(a, bh, k0, qt + 1, act_s, chunk);
      const unsigned long long* mrow = a.masks + (bh * a.nqt + qt) * a.nb;
      const unsigned long long mw = kvalid ? mrow[ck] : 0ull;
      const int64_t q0 = qt * 64;
      __syncthreads();  // the previous tile's compute is done with the LDS tiles
      stage16(qb, a.qsn, q0, a.n, qs, qtT, tid);
      stage16(gb, a.osn, q0, a.n, gs, gtT, tid);
      if (tid < 64) {
        const bool ok = q0 + tid < a.n;
        lse_s[tid] = ok ? a.lse[bh * a.n + q0 + tid] * kLog2eS : 0.0f;
        del_s[tid] = ok ? a.delta[bh * a.n + q0 + tid] : 0.0f;
      }
      __syncthreads();
      f32x16 s, dp;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        s[e] = 0.0f;
        dp[e] = 0.0f;
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int off = (32 * qp + lo) * kRS16 + 32 * hi + 8 * t;
        s = Mma16<DT>::mma(lds16(qs + off), kv[t], s);
        dp = Mma16<DT>::mma(lds16(gs + off), vv[t], dp);
      }
      float p[16], ds[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int qq = 32 * qp + (e >> 2) * 8 + hi * 4 + (e & 3);
        const bool ok = ((mw >> qq) & 1ull) && (key <= q0 + qq);
        p[e] = ok ? __builtin_amdgcn_exp2f(fmaf(s[e], sl2, -lse_s[qq])) : 0.0f;
        ds[e] = p[e] * (dp[e] - del_s[qq]);
      }
      const u32x4 p0 = pack8<DT>(p), p1 = pack8<DT>(p + 8);
      const u32x4 d0 = pack8<DT>(ds), d1 = pack8<DT>(ds + 8);
#pragma unroll
      for (int dh = 0; dh < 2; ++dh) {
        const int off = (32 * dh + lo) * kTS16 + 32 * qp + 4 * hi;
        dva[dh] = Mma16<DT>::mma(lds_pair(gtT + off), p0, dva[dh]);
        dva[dh] = Mma16<DT>::mma(lds_pair(gtT + off + 16), p1, dva[dh]);
        dka[dh] = Mma16<DT>::mma(lds_pair(qtT + off), d0, dka[dh]);
        dka[dh] = Mma16<DT>::mma(lds_pair(qtT + off + 16), d1, dka[dh]);
      }
      qt = nxt;
    }
  }
  __syncthreads();
  float* bk = reinterpret_cast<float*>(smem);  // 32 x 128 floats each
  float* bv = bk + 32 * 128;
  const int slot = kq * 64 + lane;
  if (qp == 1) {
#pragma unroll
    for (int x = 0; x < 32; ++x) {
      bk[x * 128 + slot] = dka[x >> 4][x & 15];
      bv[x * 128 + slot] = dva[x >> 4][x & 15];
    }
  }
  __syncthreads();
  if (qp == 1 || !kvalid) return;
  const int64_t krow = (bkv * a.n + key) * 64;
#pragma unroll
  for (int dh = 0; dh < 2; ++dh)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int dd = 32 * dh + 8 * g + 4 * hi, x = 16 * dh + 4 * g;
      f32x4 kv4, vv4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        kv4[j] = (dka[dh][4 * g + j] + bk[(x + j) * 128 + slot]) * a.scale;
        vv4[j] = dva[dh][4 * g + j] + bv[(x + j) * 128 + slot];
      }
      store_grad4<DT>(a.dk, krow + dd, kv4, a.grad16);
      store_grad4<DT>(a.dv, krow + dd, vv4, a.grad16);
    }
}

int fill_args(SwapArgs& a, const void* q, const void* k, const void* v, const void* out,
              int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t n, int64_t block,
              const int64_t* strides, const int32_t* kv_num, const int32_t* kv_idx, int64_t W,
              float scale, void* workspace, size_t workspace_bytes) {
  SSA_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out), SSA_ERR_UNSUPPORTED,
              "masked_attn: q, k, v and out must be 16-byte aligned");
  a.q = static_cast<const char*>(q);
  a.k = static_cast<const char*>(k);
  a.v = static_cast<const char*>(v);
  a.o = static_cast<char*>(const_cast<void*>(out));
  a.qsb = strides[0]; a.qsh = strides[1]; a.qsn = strides[2];
  a.ksb = strides[3]; a.ksh = strides[4]; a.ksn = strides[5];
  a.vsb = strides[6]; a.vsh = strides[7]; a.vsn = strides[8];
  a.osb = strides[9]; a.osh = strides[10]; a.osn = strides[11];
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.G = Hq / Hkv; a.n = n; a.block = block;
  a.nqt = (n + 63) / 64;
  a.nkt = a.nqt;
  a.nb = (n + block - 1) / block;
  a.kv_num = kv_num; a.kv_idx = kv_idx; a.W = W;
  a.scale = scale;
  a.scale_log2 = scale * kLog2eS;
  const size_t need = masked_tiled_workspace(B, Hq, n, block);
  SSA_REQUIRE(workspace && workspace_bytes >= need, SSA_ERR_WORKSPACE,
              "masked_attn: workspace needs %zu bytes", need);
  a.masks = static_cast<unsigned long long*>(workspace);
  a.delta = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                     (size_t)B * Hq * a.nqt * a.nb * 8u);
  a.lse = nullptr; a.dout = nullptr; a.dq = a.dk = a.dv = nullptr;
  a.grad16 = false;
  SSA_REQUIRE(B * Hq * a.nqt < (1ll << 31) && B * Hkv * a.nkt < (1ll << 31), SSA_ERR_UNSUPPORTED,
              "masked_attn: grid too large");
  return SSA_OK;
}

}  // namespace

bool masked_tiled_ok(int64_t d, int64_t block, int64_t n) {
  return d == 64 && block >= 1 && (n + block - 1) / block <= kMaxMaskBlocks;
}

size_t masked_tiled_workspace(int64_t B, int64_t Hq, int64_t n, int64_t block) {
  const int64_t nqt = (n + 63) / 64, nb = (n + block - 1) / block;
  return (size_t)B * Hq * nqt * nb * 8u + (size_t)B * Hq * n * 4u;
}

int masked_tiled_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                     int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t n, int64_t block,
                     const int64_t* strides, const int32_t* kv_num, const int32_t* kv_idx,
                     int64_t W, float scale, void* workspace, size_t workspace_bytes,
                     hipStream_t st) {
  SwapArgs a;
  SSA_TRY(fill_args(a, q, k, v, out, dtype, B, Hq, Hkv, n, block, strides, kv_num, kv_idx, W,
                    scale, workspace, workspace_bytes));
  a.lse = lse;
  const unsigned grid = (unsigned)(B * Hq * a.nqt);
  row_block_masks_kernel<<<grid, 256, 0, st>>>(a);
  SSA_TRY(launch_status("row_block_masks_kernel"));
  if (dtype == SSA_F32) swap_fwd_kernel<SSA_F32><<<grid, 256, 0, st>>>(a);
  else if (dtype == SSA_F16) swap_fwd16_kernel<SSA_F16><<<grid, 256, 0, st>>>(a);
  else swap_fwd16_kernel<SSA_BF16><<<grid, 256, 0, st>>>(a);
  return launch_status("swap_fwd_kernel");
}

int masked_tiled_bwd(const void* q, const void* k, const void* v, const void* out,
                     const void* dout, const float* lse, void* dq, void* dk, void* dv,
                     int dtype, int grad_dtype, int flags, int64_t B, int64_t Hq, int64_t Hkv, int64_t n, int64_t block,
                     const int64_t* strides, const int32_t* kv_num, const int32_t* kv_idx,
                     int64_t W, float scale, void* workspace, size_t workspace_bytes,
                     hipStream_t st) {
  SwapArgs a;
  SSA_TRY(fill_args(a, q, k, v, out, dtype, B, Hq, Hkv, n, block, strides, kv_num, kv_idx, W,
                    scale, workspace, workspace_bytes));
  SSA_REQUIRE(aligned16(dout) && aligned16(dq) && aligned16(dk) && aligned16(dv),
              SSA_ERR_UNSUPPORTED, "masked_attn_bwd: dout, dq, dk, dv must be 16-byte aligned");
  a.dout = static_cast<const char*>(dout);
  a.lse = const_cast<float*>(lse);
  SSA_REQUIRE(grad_dtype == SSA_F32 || grad_dtype == dtype, SSA_ERR_INVALID,
              "masked_attn_bwd: gradients must be fp32 or the input type");
  a.dq = dq; a.dk = dk; a.dv = dv;
  a.grad16 = grad_dtype != SSA_F32;
  const unsigned gq = (unsigned)(B * Hq * a.nqt), gk = (unsigned)(B * Hkv * a.nkt);
  if (!(flags & SSA_MASKED_MASKS_READY)) {  // else the forward's masks are in the workspace
    row_block_masks_kernel<<<gq, 256, 0, st>>>(a);
    SSA_TRY(launch_status("row_block_masks_kernel"));
  }
  if (dtype == SSA_F32) {
    swap_dq_kernel<SSA_F32><<<gq, 256, 0, st>>>(a);
    swap_dkdv_kernel<SSA_F32><<<gk, 256, 0, st>>>(a);
  } else if (dtype == SSA_F16) {
    swap_dq16_kernel<SSA_F16><<<gq, 256, 0, st>>>(a);
    swap_dkdv16_kernel<SSA_F16><<<gk, 256, 0, st>>>(a);
  } else {
    swap_dq16_kernel<SSA_BF16><<<gq, 256, 0, st>>>(a);
    swap_dkdv16_kernel<SSA_BF16><<<gk, 256, 0, st>>>(a);
  }
  return launch_status("swap_dkdv_kernel");
}

}  // namespace ssa
