// Block-sparse causal flash attention (prefill) for gfx950.
//
// bf16/fp16 path (d = 64), sparse_attn_dma_kernel<DT, NW, CG, WPE>:
//   a wave owns CG groups of 32 query rows, a workgroup NW waves = one query block (block 64:
//   2 waves x 32 rows) or 128 rows of it (block a multiple of 128: 2 waves x 64 rows, so every
//   LDS operand fragment feeds two MFMAs), walking the block's selected key blocks in 64-key
//   sub-tiles:
//   S^T = K Q^T   on v_mfma_f32_32x32x16_{bf16,f16}: A = K rows (from LDS), B = a wave's Q
//                 fragments (registers, loaded once). The K rows fed to MFMA row m are permuted
//                 (bits 2 and 3 of m swapped) so that each lane's 16 accumulators of a 32-key
//                 tile hold two runs of 8 consecutive keys -- exactly the B-operand layout of
//                 the next product, so P never leaves registers.
//   online softmax in fp32 (exp2 with scale*log2e folded into one FMA; lazy rescale: the running
//                 max only moves when a row's max exceeds it by more than 2^8),
//   O^T += V^T P^T on MFMA: A = V^T rows (LDS), B = P^T (registers, bf16/fp16).
// K and V^T sub-tiles go HBM -> LDS directly (global_load_lds_dwordx4, no staging registers)
// into a 2-stage ring with an XOR swizzle (16-byte chunk c of row r at c ^ ((r >> 1) & 7)): the
// 16 lanes of one ds_read_b128 phase hit all 64 banks once. V is transposed once per call into
// the workspace so V^T sub-tiles are contiguous 16-byte runs of keys. Row sums of the rounded P
// use v_dot2 against ones; row max / sum across the two 32-lane halves use v_permlane32_swap.
// Each wave's block list is held in a register window read with v_readlane. Workgroups are
// dispatched heaviest query blocks first, and the query heads sharing a key head for the same
// query block are placed on the same XCD (their shared tiles hit its L2).
//
// fp32 path: a single-wave VALU kernel (one query row per lane), K/V sub-tiles of 64 keys in LDS.
//
// Semantics: FlexAttention with BlockMask.from_kv_blocks(kv_num, kv_idx, block) and
// mask_mod = (kv <= q) & (kv < n) -- ssa/ssa_kernel.py:33-34,125-126; ssa/gemma_ssa.py:159-162,179.
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "common.h"

namespace ssa {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleSlack = 8.0f;
// Rows whose scores provably stay within +-fast_bound<DT>() (log2 units) take the softmax without
// a running max. The bounded path pre-scales q by scale*log2e and rounds it to fp16 for the QK
// product (bf16 inputs: against the fp16 copy of K written by the key-norm pass, exact for
// |k| < 2^16), so a score moves by at most 2^-11 |q| |k| scale log2e < 2^-11 * bound = 1/64
// log2 unit at the bound of 32 -- a change of at most 1.1 % in one P, 2.2 % in the ratio of two
// (typically ~0.1 %: the 64 elements' rounding errors have random signs); the fp32-scaled
// scores of the exact path and of FlexAttention carry no such error. A key-norm limit of 4096
// keeps the fp16 rounding of tiny q elements (absolute 2^-25) and the fp16 copy's range out of
// the error. P = 2^s is packed into the PV input type. bf16 has fp32's exponent range. fp16's
// largest finite value is 65504 < 2^16: an fp16 row takes P = 2^(s - m0), m0 the largest score
// of its first sub-tile (a lower bound of its maximum: the row's largest P is >= 1, so P below
// 2^-24, flushed to 0, is negligible beside it), which stays finite unless a later score
// exceeds m0 + 16; a row whose sum l comes out non-finite sends its query block to the exact
// launch. Rows beyond the bound take the exact running-max path, whose scores are the fp32
// products scaled in fp32.
constexpr float kFastBoundBf16 = 32.0f;
constexpr float kFastBoundF16 = 32.0f;
constexpr float kKeyNormLimit = 4096.0f;
// Step of the clock-rotated list walk (bounded launch, lists of <= 128 entries): roughly the time
// a workgroup spends on one K / V^T sub-tile with the device full, measured at C3 (4 waves x 32
// rows, 128-row workgroups: best at 1.5-2 us) and C5 (8 waves x 32 rows: 2-3 us); in
// s_memrealtime ticks (100 MHz).
constexpr int64_t kRotTicks128 = 200;
constexpr int64_t kRotTicks256 = 250;
template <int DT>
__device__ constexpr float fast_bound() {
  return DT == SSA_F16 ? kFastBoundF16 : kFastBoundBf16;
}
// Key norms enter the bound per 64-key tile: tile t of key head bk holds the largest squared key
// norm of rows 64t..64t+63 at tmax2[bk * ntile + t]. A workgroup bounds its scores with the tiles
// it attends only, so its choice of path depends on no key it does not read (in particular on no
// key after its query block).

struct AttnParams {
  const char* q;
  const char* k;
  const char* k16;  // fp16 copy of bf16 K (B, Hkv, n_pad, 64) in the workspace (bounded rows)
  const char* v;   // natural V (fp32 path)
  const char* vt;  // V^T workspace (B, Hkv, 64, n_pad) (16-bit path)
  char* o;
  int64_t qsb, qsh, qsn, ksb, ksh, ksn, vsb, vsh, vsn, osb, osh, osn;
  int64_t B, Hq, Hkv, G, n, n_pad, block, nbq;
  const int32_t* kv_num;
  const int32_t* kv_idx;
  int64_t W;
  float scale_log2;
  float* lse;
  const float* tmax2;  // per-tile maxima of the squared key norms (NULL: exact path only)
  int64_t ntile;       // 64-key tiles per key head (n_pad / 64)
  int* unbounded;      // per (b, kv head): set by mode 1 when one of its workgroups is not bounded
                       // (or, fp16, overflowed)
  int64_t rot_ticks;   // bounded launch, lists of <= 128 entries: s_memrealtime ticks per sub-tile
                       // step of the clock-rotated list walk (0: every walk starts at entry 0)
  bool rotate;         // host: rotate the walks (SSA_ATTN_ROTATE)
  int* redo;           // per (b, kv head, query block): set by mode 1 when a workgroup of the
                       // query block is not bounded or (fp16) a row of it overflowed; the exact
                       // launch then redoes the query block for every query head of the key head
  int64_t qsub;   // query sub-tiles per query block
  int64_t total;  // logical workgroups
  int64_t group;  // logical workgroups placed together on one XCD
};

// Logical work item of a physical workgroup: XCD x = pid % 8 receives consecutive runs of
// `group` logical items, runs interleaved across the 8 XCDs.
__device__ inline int64_t logical_id(int64_t pid, int64_t group) {
  const int64_t x = pid & 7, s = pid >> 3;
  return ((s / group) * 8 + x) * group + (s % group);
}

// Permutation of a 32-key group: MFMA row m loads key sigma(m) (bits 2 and 3 swapped).
__device__ inline int sigma32(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

template <int DT>
struct Mfma;
template <>
struct Mfma<SSA_BF16> {
  typedef bf16x8 vec;
  static __device__ inline f32x16 mma(const vec& a, const vec& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ inline vec from_bits(const u32x4& w) { return __builtin_bit_cast(vec, w); }
  static __device__ inline vec pack(const float* p) {
    vec r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = (__bf16)p[j];
    return r;
  }
  static __device__ inline unsigned int pack2(float a, float b) {
    unsigned short lo = __builtin_bit_cast(unsigned short, (__bf16)a);
    unsigned short hi = __builtin_bit_cast(unsigned short, (__bf16)b);
    return (unsigned int)lo | ((unsigned int)hi << 16);
  }
  // acc + sum of the 8 packed values, on v_dot2_f32_bf16 against ones
  static __device__ inline float rowsum(const vec& v, float acc) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    const u32x4 w = __builtin_bit_cast(u32x4, v);
    const v2 one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const unsigned int wi = w[i];  // (bit_cast of a vector-element subscript mis-lowers)
      acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, wi), one, acc, false);
    }
    return acc;
  }
};
template <>
struct Mfma<SSA_F16> {
  typedef f16x8 vec;
  static __device__ inline f32x16 mma(const vec& a, const vec& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ inline vec from_bits(const u32x4& w) { return __builtin_bit_cast(vec, w); }
  static __device__ inline vec pack(const float* p) {
    vec r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = (_Float16)p[j];
    return r;
  }
  static __device__ inline unsigned int pack2(float a, float b) {
    unsigned short lo = __builtin_bit_cast(unsigned short, (_Float16)a);
    unsigned short hi = __builtin_bit_cast(unsigned short, (_Float16)b);
    return (unsigned int)lo | ((unsigned int)hi << 16);
  }
  // acc + sum of the 8 packed values, on v_dot2_f32_f16 against ones
  static __device__ inline float rowsum(const vec& v, float acc) {
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    const u32x4 w = __builtin_bit_cast(u32x4, v);
    const v2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const unsigned int wi = w[i];
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, wi), one, acc, false);
    }
    return acc;
  }
};

__device__ inline unsigned int pack2_f16(float a, float b) {
  const unsigned short lo = __builtin_bit_cast(unsigned short, (_Float16)a);
  const unsigned short hi = __builtin_bit_cast(unsigned short, (_Float16)b);
  return (unsigned int)lo | ((unsigned int)hi << 16);
}

// Key-norm bound of the attention call: the largest squared norm of key rows k0..k0+63 of one
// key head (rows >= n count 0) into its tile's slot; the first tile's workgroup also clears the
// head's unbounded flag for the mode-1 launch, and the tile starting a query block its redo flag. 256 threads; lanes 8r..8r+7 of a pass read row
// r's 8 16-byte chunks.
struct KeyNorm {
  const unsigned short* k;  // NULL: no key norms
  int64_t ksb, ksh, ksn;
  bool bf16;
  float* tmax2;    // (B*Hkv, ntile)
  int* unbounded;  // (B*Hkv)
  int64_t ntile;
  int* redo;       // (B*Hkv, nbq): cleared here, one entry per query block (block a multiple of 64)
  int64_t block, nbq;
  unsigned short* k16;  // bf16 keys: their fp16 copy (B*Hkv, n_pad, 64), rows >= n zero (else NULL)
  int64_t n_pad;
};

__device__ inline void key_tile_norm_max(const KeyNorm& kn, int64_t b, int64_t kvh,
                                         int64_t Hkv, int64_t k0, int64_t n) {
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const unsigned short* base = kn.k + b * kn.ksb + kvh * kn.ksh;
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int q = tid + 256 * j;
    const int row = q >> 3, ch = q & 7;
    float acc = 0.0f;
    u32x4 h = {0u, 0u, 0u, 0u};
    if (k0 + row < n) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(base + (k0 + row) * kn.ksn + ch * 8);
      float x[8];
      unpack8(w, x, kn.bf16);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = fmaf(x[e], x[e], acc);
      // fp16 holds every bf16 value of magnitude in [2^-14, 2^16) exactly (8 significant bits
      // in 11); smaller ones move by at most 2^-25, larger ones overflow -- tiles with such keys
      // fail the bounded rows' key-norm limit, so the exact path (which reads k) takes them
#pragma unroll
      for (int e = 0; e < 4; ++e) h[e] = pack2_f16(x[2 * e], x[2 * e + 1]);
    }
    if (kn.k16 != nullptr)
      *reinterpret_cast<u32x4*>(kn.k16 + ((b * Hkv + kvh) * kn.n_pad + k0 + row) * 64 + ch * 8) = h;
    acc += __shfl_xor(acc, 1, 64);
    acc += __shfl_xor(acc, 2, 64);
    acc += __shfl_xor(acc, 4, 64);
    mx = fmaxf(mx, acc);
  }
#pragma unroll
  for (int off = 8; off <= 32; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  if (tid == 0) {
    const int64_t bk = b * Hkv + kvh;
    kn.tmax2[bk * kn.ntile + k0 / 64] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    if (k0 == 0) kn.unbounded[bk] = 0;
    if (kn.redo != nullptr && k0 % kn.block == 0) kn.redo[bk * kn.nbq + k0 / kn.block] = 0;
  }
}

// Key norms alone (V^T supplied by the caller). grid (n_pad/64, B*Hkv).
__global__ __launch_bounds__(256) void key_norm_max_kernel(KeyNorm kn, int64_t Hkv, int64_t n) {
  const int64_t bk = blockIdx.y;
  key_tile_norm_max(kn, bk / Hkv, bk % Hkv, Hkv, (int64_t)blockIdx.x * 64, n);
}

// V (B, Hkv, n, d) -> V^T (B, Hkv, d, n_pad), zero for keys >= n, in 64 x 64 tiles (head dims
// 64 z .. 64 z + 63 of keys 64 x ..); with kn.k set (head dim 64), also the key-norm bound of the
// same 64 rows. grid (n_pad/64, B*Hkv, d/64).
__global__ __launch_bounds__(256) void transpose_v_kernel(const char* __restrict__ v,
                                                          char* __restrict__ vt, int64_t Hkv,
                                                          int64_t n, int64_t n_pad, int64_t vsb,
                                                          int64_t vsh, int64_t vsn, int64_t d,
                                                          KeyNorm kn) {
  __shared__ unsigned short t[64][64 + 2];
  const int64_t bk = blockIdx.y;
  const int64_t b = bk / Hkv, kvh = bk % Hkv;
  const int64_t k0 = (int64_t)blockIdx.x * 64;
  const int64_t z = blockIdx.z;
  const int tid = threadIdx.x;
  if (kn.k != nullptr) key_tile_norm_max(kn, b, kvh, Hkv, k0, n);
  const unsigned short* src =
      reinterpret_cast<const unsigned short*>(v) + b * vsb + kvh * vsh + z * 64;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int q = tid + 256 * j;
    const int row = q >> 3, ch = q & 7;
    u32x4 w = {0u, 0u, 0u, 0u};
    if (k0 + row < n) w = *reinterpret_cast<const u32x4*>(src + (k0 + row) * vsn + ch * 8);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      t[row][ch * 8 + 2 * e] = (unsigned short)(w[e] & 0xffffu);
      t[row][ch * 8 + 2 * e + 1] = (unsigned short)(w[e] >> 16);
    }
  }
  __syncthreads();
  unsigned short* dst = reinterpret_cast<unsigned short*>(vt) + (bk * d + z * 64) * n_pad;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int q = tid + 256 * j;
    const int drow = q >> 3, kch = q & 7;
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = (unsigned int)t[kch * 8 + 2 * e][drow] |
             ((unsigned int)t[kch * 8 + 2 * e + 1][drow] << 16);
    *reinterpret_cast<u32x4*>(dst + drow * n_pad + k0 + kch * 8) = w;
  }
}

// Workgroup barrier once this wave's LDS DMA (global_load_lds) has landed. __syncthreads() is not
// enough: its workgroup-scope release fence waits for LDS and store traffic (lgkmcnt) only, not
// for the loads that write LDS asynchronously (vmcnt) -- the compiler's own tracking of them
// inserted the vmcnt(0) in some builds of the tile loop and not in others. The "memory" clobber
// keeps the compiler from moving LDS or global accesses across it.
__device__ inline void dma_barrier() {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Max / sum of a value with its partner lane (lane ^ 32) without an LDS round trip:
// permlane32_swap(x, x) returns {x of lanes 0-31 (both halves), x of lanes 32-63 (both halves)}.
__device__ inline float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// fp32 path: one wave per 64 query rows, one row per lane. grid = logical items (no remap).
__global__ __launch_bounds__(64) void sparse_attn_f32_kernel(AttnParams p) {
  __shared__ __attribute__((aligned(16))) float Ks[64][64];
  __shared__ __attribute__((aligned(16))) float Vs[64][64];
  int64_t L = blockIdx.x;
  const int64_t qs = L % p.qsub;
  L /= p.qsub;
  const int64_t h = L % p.Hq;
  L /= p.Hq;
  const int64_t b = L % p.B;
  L /= p.B;
  const int64_t i = p.nbq - 1 - L;
  const int64_t kvh = h / p.G;
  const int lane = threadIdx.x;
  const int64_t q0 = i * p.block + qs * 64;
  if (q0 >= p.n) return;
  const int64_t qmax = q0 + 63 < p.n - 1 ? q0 + 63 : p.n - 1;
  const int64_t qpos = q0 + lane;

  const float* qp = reinterpret_cast<const float*>(p.q) + b * p.qsb + h * p.qsh + qpos * p.qsn;
  float qv[64], ov[64];
#pragma unroll
  for (int e = 0; e < 64; ++e) {
    qv[e] = qpos < p.n ? qp[e] : 0.0f;
    ov[e] = 0.0f;
  }
  const float* kbase = reinterpret_cast<const float*>(p.k) + b * p.ksb + kvh * p.ksh;
  const float* vbase = reinterpret_cast<const float*>(p.v) + b * p.vsb + kvh * p.vsh;
  const int64_t row = (b * p.Hq + h) * p.nbq + i;
  int cnt = p.kv_num[row];
  if (cnt > p.W) cnt = (int)p.W;
  if (cnt < 0) cnt = 0;
  const int32_t* list = p.kv_idx + row * p.W;
  const int S = (int)(p.block / 64);
  float m_run = -INFINITY, l_run = 0.0f;
  const float c2 = p.scale_log2;
  for (int t = 0; t < cnt * S; ++t) {
    const int32_t c = list[t / S];
    if (c < 0 || (int64_t)c >= p.nbq) continue;
    const int64_t key0 = (int64_t)c * p.block + (int64_t)(t % S) * 64;
    if (key0 > qmax || key0 >= p.n) continue;
    __syncthreads();
    for (int e = lane; e < 64 * 64; e += 64) {
      const int kr = e >> 6, kc = e & 63;
      const bool in = key0 + kr < p.n;
      Ks[kr][kc] = in ? kbase[(key0 + kr) * p.ksn + kc] : 0.0f;
      Vs[kr][kc] = in ? vbase[(key0 + kr) * p.vsn + kc] : 0.0f;
    }
    __syncthreads();
    float sv[64];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 64; ++j) {
      float s = 0.0f;
#pragma unroll
      for (int e = 0; e < 64; e += 4) {
        const f32x4 kk = *reinterpret_cast<const f32x4*>(&Ks[j][e]);
        s = fmaf(qv[e], kk[0], s);
        s = fmaf(qv[e + 1], kk[1], s);
        s = fmaf(qv[e + 2], kk[2], s);
        s = fmaf(qv[e + 3], kk[3], s);
      }
      const int64_t key = key0 + j;
      if (key > qpos || key >= p.n) s = -INFINITY;
      sv[j] = s;
      mx = fmaxf(mx, s);
    }
    const float m_new = fmaxf(m_run, mx * c2);
    if (m_new > m_run) {
      const float alpha = exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int e = 0; e < 64; ++e) ov[e] *= alpha;
      m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;
#pragma unroll
    for (int j = 0; j < 64; ++j) {
      const float pj = exp2f(fmaf(sv[j], c2, -m_use));
      l_run += pj;
#pragma unroll
      for (int e = 0; e < 64; e += 4) {
        const f32x4 vv = *reinterpret_cast<const f32x4*>(&Vs[j][e]);
        ov[e] = fmaf(pj, vv[0], ov[e]);
        ov[e + 1] = fmaf(pj, vv[1], ov[e + 1]);
        ov[e + 2] = fmaf(pj, vv[2], ov[e + 2]);
        ov[e + 3] = fmaf(pj, vv[3], ov[e + 3]);
      }
    }
  }
  if (qpos < p.n) {
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    float* op = reinterpret_cast<float*>(p.o) + b * p.osb + h * p.osh + qpos * p.osn;
#pragma unroll
    for (int e = 0; e < 64; ++e) op[e] = ov[e] * inv;
    if (p.lse != nullptr)
      p.lse[(b * p.Hq + h) * p.n + qpos] =
          l_run > 0.0f ? (m_run + log2f(l_run)) * kLn2 : -INFINITY;
  }
}

// 16-byte chunk c of an LDS tile row r of RB bytes is stored at chunk c ^ swz<RB>(r): the 16
// lanes served together by one ds_read_b128 of an MFMA operand (16 distinct rows r0..r0+15, the
// same logical chunk) then hit all 64 banks once -- their addresses are distinct mod 256 bytes:
// RB = 128 (two rows per 256 bytes): row parity x chunk ^ ((r >> 1) & 7); RB = 64: r & 3 x
// chunk ^ ((r >> 2) & 3); RB >= 256 (rows a multiple of 256 bytes): chunk ^ (r & 15).
template <int RB>
__device__ inline int swz(int r) {
  if constexpr (RB == 64) return (r >> 2) & 3;
  else if constexpr (RB == 128) return (r >> 1) & 7;
  else return r & 15;
}

// A wave owns CG groups of 32 query rows (every LDS operand fragment feeds CG MFMAs); a workgroup
// of NW waves owns ROWS = 32*CG*NW rows of one query block and walks its selected key blocks in
// KT-key sub-tiles (KT = 64, or 32 for head dim 256). K sub-tiles (KT rows of D elements) and V^T
// sub-tiles (D rows of KT keys), swizzled, go HBM -> LDS directly (global_load_lds_dwordx4, no
// staging registers) into a 2-stage ring, one barrier per sub-tile.
// MODE 0: every workgroup, exact online softmax. MODE 1: only workgroups whose rows are all
// bounded (P = 2^S without a running max). MODE 2: only the others, exact. Modes 1 and 2 are
// launched back to back and together cover every workgroup (head dim 64 only).
template <int DT, int NW, int CG, int WPE, int MODE, int D = 64, int KT = 64, bool REG = false>
__global__ __launch_bounds__(NW * 64, WPE) void sparse_attn_dma_kernel(AttnParams p) {
  using M = Mfma<DT>;
  typedef typename M::vec vec;
  // bounded rows of bf16 inputs: S^T = K Q^T on fp16 operands (the fp16 copy of K, q scale log2e
  // rounded to fp16); every other product in the input type
  constexpr bool K16 = MODE == 1 && DT == SSA_BF16;
  using MQ = Mfma<K16 ? SSA_F16 : DT>;
  static_assert(D % 64 == 0 && (KT == 32 || KT == 64), "head dim a multiple of 64, KT 32 or 64");
  static_assert(MODE == 0 || D == 64, "the bounded-row path is built for head dim 64");
  constexpr int TILE = KT * D * 2;    // bytes of one K or V^T sub-tile
  constexpr int KRB = D * 2;          // bytes of a K tile row (one key)
  constexpr int VRB = KT * 2;         // bytes of a V^T tile row (one head dim)
  constexpr int KD = D / 16;          // 16-element k-steps of the QK product
  constexpr int DTN = D / 32;         // 32-row output tiles of the PV product
  constexpr int TT = KT / 32;         // 32-key groups of a sub-tile
  constexpr int SS = KT / 16;         // 16-key steps of the PV product
  constexpr int ROWS = 32 * CG * NW;  // query rows per workgroup
  constexpr int LPW = TILE / 1024 / NW;  // 1 KB load instructions per wave per operand per sub-tile
  static_assert(LPW >= 1 && TILE % (1024 * NW) == 0, "sub-tile loads must split over the waves");
  __shared__ __attribute__((aligned(1024))) unsigned char kst0[TILE];
  __shared__ __attribute__((aligned(1024))) unsigned char vst0[TILE];
  __shared__ __attribute__((aligned(1024))) unsigned char kst1[TILE];
  __shared__ __attribute__((aligned(1024))) unsigned char vst1[TILE];

  const int64_t L0 = logical_id(blockIdx.x, p.group);
  if (L0 >= p.total) return;
  int64_t L = L0;
  const int64_t qs = L % p.qsub;
  L /= p.qsub;
  const int64_t hg = L % p.G;
  L /= p.G;
  const int64_t kvh = L % p.Hkv;
  L /= p.Hkv;
  const int64_t b = L % p.B;
  L /= p.B;
  const int64_t i = p.nbq - 1 - L;
  const int64_t h = kvh * p.G + hg;
  if constexpr (MODE == 2) {
    // mode 1 completed every query block of this head, or this one
    if (p.unbounded[b * p.Hkv + kvh] == 0) return;
    if (p.redo[(b * p.Hkv + kvh) * p.nbq + i] == 0) return;
  }

  const int64_t q0 = i * p.block + qs * ROWS;
  if (q0 >= p.n) return;
  const int64_t qmax = q0 + ROWS - 1 < p.n - 1 ? q0 + ROWS - 1 : p.n - 1;

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, col = lane & 31;
  const int64_t qw0 = q0 + w * 32 * CG;  // first query row of this wave
  int qpos[CG];  // 32-bit (the host checks n < 2^31)
#pragma unroll
  for (int c = 0; c < CG; ++c) qpos[c] = (int)qw0 + 32 * c + col;
  // REMAT: the fp16 bounded-row build (its m0 offset takes the last registers of the 128-VGPR
  // budget) re-forms the lane's query row and K row offset from the lane index where the tile
  // loop and the epilogue use them; kept live across the loop they spilled. The other builds
  // keep them hoisted (re-forming costs ~11 VALU instructions per sub-tile).
  constexpr bool REMAT = MODE == 1 && DT == SSA_F16;
  auto qrow = [&](int c) -> int {
    int ln = lane;
    if constexpr (REMAT) asm volatile("" : "+v"(ln));
    return (int)qw0 + 32 * c + (ln & 31);
  };

  const int64_t row = (b * p.Hq + h) * p.nbq + i;
  int cnt = p.kv_num[row];
  if (cnt > p.W) cnt = (int)p.W;
  if (cnt < 0) cnt = 0;
  const int32_t* list = p.kv_idx + row * p.W;
  const int S = (int)(p.block / KT);

  // Q fragments (B operands of S^T = K Q^T) of the column groups
  vec qf[CG][KD];
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    const unsigned short* src = reinterpret_cast<const unsigned short*>(p.q) + b * p.qsb +
                                h * p.qsh + qpos[c] * p.qsn + half * 8;
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
      u32x4 wv = {0u, 0u, 0u, 0u};
      if (qpos[c] < p.n) wv = *reinterpret_cast<const u32x4*>(src + kd * 16);
      qf[c][kd] = M::from_bits(wv);
    }
  }

  // Bounded rows: when |q| |k|max scale log2e < fast_bound<DT>() for every row of the wave, the
  // scores (log2 units) lie in (-bound, bound), so P = 2^S needs no running max. Q is then
  // pre-scaled by scale log2e (rounded to the input type) and the softmax is exp2 of the raw
  // MFMA output; numerator and denominator share the implicit max 0.
  constexpr bool fast = MODE == 1;
  constexpr bool OFS = fast && DT == SSA_F16;  // fp16 bounded rows: scores offset by m0 (above)
  int e0 = 0;  // first list entry walked (REG: rotated by the clock, below)
  if constexpr (MODE == 1) {
    __shared__ int wg_bounded, wg_e0;
    // largest squared key norm over the tiles this workgroup attends (its list's blocks, tiles
    // starting at or before its last query row)
    float km2 = 0.0f;
    {
      const float* tm = p.tmax2 + (b * p.Hkv + kvh) * p.ntile;
      const int64_t tpb = p.block / 64;  // tiles per key block
      for (int e = lane; e < cnt; e += 64) {
        const int32_t c = list[e];
        if (c < 0 || (int64_t)c >= p.nbq) continue;
        for (int64_t t = 0; t < tpb; ++t)
          if ((int64_t)c * p.block + t * 64 <= qmax) km2 = fmaxf(km2, tm[(int64_t)c * tpb + t]);
      }
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) km2 = fmaxf(km2, __shfl_xor(km2, off, 64));
    }
    bool ok = true;
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      float qn2 = 0.0f;
#pragma unroll
      for (int kd = 0; kd < KD; ++kd)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float x = (float)qf[c][kd][j];
          qn2 = fmaf(x, x, qn2);
        }
      qn2 = pair_sum(qn2);
      const float qn = sqrtf(qn2);
      ok = ok && (p.scale_log2 * qn * sqrtf(km2) < fast_bound<DT>()) &&
           (sqrtf(km2) < kKeyNormLimit) && (p.scale_log2 * qn < 1.0e4f);
    }
    if (tid == 0) {
      wg_bounded = 1;
      int e = 0;
      if (REG && p.rot_ticks > 0 && cnt > 0) {
        // the walk starts at the list position the clock points to: with a period of cnt*S*rot
        // ticks (rot ~ one sub-tile step), workgroups resident together read the same part of
        // their (ascending) lists at the same time, wherever they started, so the key blocks
        // they share are fetched once into L2 / MALL for all of them
        const uint64_t per = (uint64_t)cnt * (uint64_t)S * (uint64_t)p.rot_ticks;
        e = (int)((__builtin_amdgcn_s_memrealtime() % per) / ((uint64_t)S * (uint64_t)p.rot_ticks));
      }
      wg_e0 = e;
    }
    __syncthreads();
    if (!__all(ok) && lane == 0) wg_bounded = 0;
    __syncthreads();
    e0 = wg_e0;
    if (wg_bounded == 0) {  // the exact launch takes this query block
      if (tid == 0) {
        p.redo[(b * p.Hkv + kvh) * p.nbq + i] = 1;
        p.unbounded[b * p.Hkv + kvh] = 1;
      }
      return;
    }
    {
#pragma unroll
      for (int c = 0; c < CG; ++c)
#pragma unroll
        for (int kd = 0; kd < KD; ++kd) {
          float x[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) x[j] = (float)qf[c][kd][j] * p.scale_log2;
          qf[c][kd] = __builtin_bit_cast(vec, MQ::pack(x));
        }
    }
  }

  // K rows: the input, or (K16) its fp16 copy, contiguous rows of 64
  const int64_t ksn = K16 ? 64 : p.ksn;
  const unsigned short* kbase =
      K16 ? reinterpret_cast<const unsigned short*>(p.k16) + (b * p.Hkv + kvh) * p.n_pad * 64
          : reinterpret_cast<const unsigned short*>(p.k) + b * p.ksb + kvh * p.ksh;
  const unsigned short* vtbase =
      reinterpret_cast<const unsigned short*>(p.vt) + (b * p.Hkv + kvh) * D * p.n_pad;

  // Load plan: instruction j of wave w fills 1 KB of the tile at LDS offset j*1024*NW + w*1024:
  // K rows j*KR*NW + w*KR + [0, KR) (KR = 1024 / KRB keys), V^T rows j*VR*NW + w*VR + [0, VR)
  // (VR = 1024 / VRB head dims); lane -> row lr (+ j*KR*NW), physical chunk = lane % chunks per
  // row, loading logical chunk physical ^ swz(row) (the swizzles repeat every 16 rows, so the
  // chunk of instruction j depends on j only when it advances by a row count not a multiple of
  // 16: K rows at head dim 256).
  constexpr int KR = 1024 / KRB, VR = 1024 / VRB, KC = KRB / 16, VC = VRB / 16;
  const int lr = w * KR + lane / KC;
  const int vr = w * VR + lane / VC;
  static_assert((VR * NW) % 16 == 0, "V^T rows per load instruction keep the swizzle");
  const int vc = (lane % VC) ^ swz<VRB>(vr);
  const uint32_t vgo = (uint32_t)(vr * p.n_pad + vc * 8);
  const int64_t kstep = KR * NW * ksn, vstep = VR * NW * p.n_pad;

  // Tile cursor over the row's block list: entry ce, sub-tile cs (key0 = list[ce]*block + cs*KT).
  // The list is held 64 entries at a time in one VGPR (entry lbase + j in lane j), read with
  // v_readlane: no memory wait per sub-tile. Key arithmetic is 32-bit (the host checks n < 2^31).
  const int n32 = (int)p.n, blk32 = (int)p.block, nbq32 = (int)p.nbq, qmax32 = (int)qmax;
  int lbase = 0;
  int32_t lreg = lane < cnt ? list[lane] : -1;
  // REG (the host launches it for lists of at most 128 entries): entries 64..127 in a second
  // register, no reload, so the walk can start anywhere in the list and wrap around
  int32_t lreg1 = -1;
  if constexpr (REG) lreg1 = 64 + lane < cnt ? list[64 + lane] : -1;
  int ce = e0, cs = -1, kk = 0;  // kk: entries walked (REG: entry ce = e0 + kk mod cnt)
  // advances the cursor to the next tile that starts at or before the last query row and before
  // n; returns its first key, or -1 past the list
  auto next_tile = [&]() -> int {
    while (true) {
      int c;
      if constexpr (REG) {
        if (++cs == S) {
          cs = 0;
          ++kk;
          if (++ce == cnt) ce = 0;
        }
        if (kk >= cnt) return -1;
        c = ce < 64 ? __builtin_amdgcn_readlane(lreg, ce) : __builtin_amdgcn_readlane(lreg1, ce - 64);
      } else {
        if (++cs == S) {
          cs = 0;
          ++ce;
        }
        if (ce >= cnt) return -1;
        if (ce - lbase >= 64) {  // wave-uniform; once per 64 list entries
          lbase = ce;
          lreg = ce + lane < cnt ? list[ce + lane] : -1;
        }
        c = __builtin_amdgcn_readlane(lreg, ce - lbase);
      }
      if (c >= 0 && c < nbq32) {
        const int k0 = c * blk32 + cs * KT;
        if (k0 <= qmax32 && k0 < n32) return k0;
      }
      cs = S - 1;  // later sub-tiles of this entry start later still (or the entry is invalid)
    }
  };
  auto issue = [&](unsigned char* kdst, unsigned char* vdst, int key0) {
    const unsigned short* kt = kbase + key0 * ksn;
    const unsigned short* vt = vtbase + key0;
    if (key0 + KT <= n32) {
      int ln = lane;  // (REMAT: re-formed on each call)
      if constexpr (REMAT) asm volatile("" : "+v"(ln));
      const int lrr = w * KR + ln / KC;
      const uint32_t klr = (uint32_t)lrr * (uint32_t)ksn;
#pragma unroll
      for (int j = 0; j < LPW; ++j) {
        const int lcj = (ln % KC) ^ swz<KRB>(lrr + j * KR * NW);
        __builtin_amdgcn_global_load_lds(kt + j * kstep + (klr + (uint32_t)(lcj * 8)),
                                         kdst + j * 1024 * NW + w * 1024, 16, 0, 0);
      }
    } else {  // ragged tail: rows >= n re-read row n-1 (their scores are masked)
#pragma unroll
      for (int j = 0; j < LPW; ++j) {
        int64_t r = key0 + j * KR * NW + lr;
        if (r > p.n - 1) r = p.n - 1;
        const int lcj = (lane % KC) ^ swz<KRB>(lr + j * KR * NW);
        __builtin_amdgcn_global_load_lds(kbase + r * ksn + lcj * 8,
                                         kdst + j * 1024 * NW + w * 1024, 16, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < LPW; ++j)
      __builtin_amdgcn_global_load_lds(vt + j * vstep + vgo, vdst + j * 1024 * NW + w * 1024,
                                       16, 0, 0);
  };

  // per-lane LDS read offsets: K row tt*32 + sigma32(col), V^T row dt*32 + col; chunk
  // (2*step + half) ^ swz(row) (the swizzles repeat every 16 rows); tt / dt add 32 rows (an
  // immediate).
  const int krow = sigma32(col);
  uint32_t koff[KD], voff[SS];
#pragma unroll
  for (int s = 0; s < KD; ++s)
    koff[s] = (uint32_t)(krow * KRB + (((2 * s + half) ^ swz<KRB>(krow)) * 16));
#pragma unroll
  for (int s = 0; s < SS; ++s)
    voff[s] = (uint32_t)(col * VRB + (((2 * s + half) ^ swz<VRB>(col)) * 16));

  f32x16 oacc[DTN][CG];  // [dt][c]
#pragma unroll
  for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
    for (int c = 0; c < CG; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[dt][c][r] = 0.0f;
  float m_run[CG], l_part[CG];
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    m_run[c] = fast ? 0.0f : -INFINITY;
    l_part[c] = 0.0f;
  }
  bool have_m0 = !OFS;  // OFS: m_run holds m0 once the first sub-tile set it
  const float c2 = p.scale_log2;
  // Exact path, bf16 (XO): the running max is taken on a wave's first sub-tile only; later
  // sub-tiles reuse it as the offset of P = 2^(s - m) (bf16 P has fp32's exponent range, so a
  // later score may exceed m by up to ~100 log2 units before anything overflows). A workgroup
  // with a row whose sum or output left that range walks its list again with the per-sub-tile
  // running max (xo_pass false).
  constexpr bool XO = !fast && DT == SSA_BF16;
  // raised wave priority around the exact path's MFMA phases: kept for head dims 128 / 256; at 64
  // the default priority is 1.5-2 % faster since the max is no longer taken every sub-tile
  constexpr bool PRIO = !fast && D != 64;

  // SKIPC (std::true_type): the running max is not taken for this sub-tile (XO)
  auto compute = [&](const unsigned char* ks, const unsigned char* vs, int key0, auto skipc) {
    constexpr bool SKIP = decltype(skipc)::value;
    // ---- S^T = K Q^T ----
    u32x4 ka[TT][KD];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int kd = 0; kd < KD; ++kd)
        ka[tt][kd] = *reinterpret_cast<const u32x4*>(ks + koff[kd] + tt * (32 * KRB));
    f32x16 sacc[TT][CG];  // [tt][c]
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int c = 0; c < CG; ++c) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[tt][c][r] = OFS ? -m_run[c] : 0.0f;
#pragma unroll
        for (int kd = 0; kd < KD; ++kd)
          sacc[tt][c] = MQ::mma(MQ::from_bits(ka[tt][kd]),
                                __builtin_bit_cast(typename MQ::vec, qf[c][kd]), sacc[tt][c]);
      }
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    // V^T fragments of the first two key steps, in flight during the softmax
    u32x4 va[SS][DTN];
#pragma unroll
    for (int s = 0; s < (SS < 2 ? SS : 2); ++s)
#pragma unroll
      for (int dt = 0; dt < DTN; ++dt)
        va[s][dt] = *reinterpret_cast<const u32x4*>(vs + voff[s] + dt * (32 * VRB));
    // ---- mask (diagonal / ragged tail sub-tiles only) ----
    if (key0 + KT - 1 > (int)qw0 || key0 + KT > n32) {
#pragma unroll
      for (int c = 0; c < CG; ++c) {
        const int lim_q = qrow(c) - key0;
        const int lim_n = n32 - 1 - key0;
        const int lim = lim_q < lim_n ? lim_q : lim_n;
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = tt * 32 + (r >> 3) * 16 + half * 8 + (r & 7);
            if (key > lim) sacc[tt][c][r] = -INFINITY;
          }
      }
    }
    if constexpr (fast) {  // ---- bounded rows: P^T = 2^(S^T), O^T += V^T P^T ----
      if constexpr (OFS) {
        if (!have_m0) {  // first sub-tile: m0 = its largest score per row, subtracted here (the
                         // later sub-tiles start their accumulators at -m0)
#pragma unroll
          for (int c = 0; c < CG; ++c) {
            float mx = -INFINITY;
#pragma unroll
            for (int tt = 0; tt < TT; ++tt)
#pragma unroll
              for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[tt][c][r]);
            mx = pair_max(mx);
            m_run[c] = mx == -INFINITY ? 0.0f : mx;
#pragma unroll
            for (int tt = 0; tt < TT; ++tt)
#pragma unroll
              for (int r = 0; r < 16; ++r) sacc[tt][c][r] -= m_run[c];
          }
          have_m0 = true;
        }
      }
#pragma unroll
      for (int s = 0; s < SS; ++s) {
        if (s + 2 < SS) {
#pragma unroll
          for (int dt = 0; dt < DTN; ++dt)
            va[(s + 2) % SS][dt] = *reinterpret_cast<const u32x4*>(vs + voff[(s + 2) % SS] + dt * (32 * VRB));
        }
        vec pb[CG];
#pragma unroll
        for (int c = 0; c < CG; ++c) {
          float pv[8];
#pragma unroll
          for (int j = 0; j < 8; ++j)
            pv[j] = __builtin_amdgcn_exp2f(sacc[s >> 1][c][8 * (s & 1) + j]);
          pb[c] = M::pack(pv);
          l_part[c] = M::rowsum(pb[c], l_part[c]);
        }
#pragma unroll
        for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
          for (int c = 0; c < CG; ++c)
            oacc[dt][c] = M::mma(M::from_bits(va[s][dt]), pb[c], oacc[dt][c]);
      }
      return;
    }
    // ---- online softmax (lazy rescale; XO: on a wave's first sub-tile only) ----
    float m_use[CG];
    if constexpr (!SKIP) {
      float m_cand[CG];
      bool grew[CG];
      bool any_grew = false;
#pragma unroll
      for (int c = 0; c < CG; ++c) {
        float mx = -INFINITY;
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[tt][c][r]);
        mx = pair_max(mx);
        m_cand[c] = mx * c2;
        grew[c] = m_cand[c] > m_run[c] + kRescaleSlack;
        any_grew = any_grew || grew[c];
      }
      if (__any(any_grew)) {
#pragma unroll
        for (int c = 0; c < CG; ++c) {
          const float alpha = grew[c] ? __builtin_amdgcn_exp2f(m_run[c] - m_cand[c]) : 1.0f;
          l_part[c] *= alpha;
#pragma unroll
          for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[dt][c][r] *= alpha;
          m_run[c] = grew[c] ? m_cand[c] : m_run[c];
        }
      }
    }
#pragma unroll
    for (int c = 0; c < CG; ++c) m_use[c] = m_run[c] == -INFINITY ? 0.0f : m_run[c];
    // ---- P^T (registers) and O^T += V^T P^T ----
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < SS; ++s) {
      if (s + 2 < SS) {
#pragma unroll
        for (int dt = 0; dt < DTN; ++dt)
          va[(s + 2) % SS][dt] = *reinterpret_cast<const u32x4*>(vs + voff[(s + 2) % SS] + dt * (32 * VRB));
      }
      vec pb[CG];
#pragma unroll
      for (int c = 0; c < CG; ++c) {
        float pv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          pv[j] = __builtin_amdgcn_exp2f(fmaf(sacc[s >> 1][c][8 * (s & 1) + j], c2, -m_use[c]));
        pb[c] = M::pack(pv);
        l_part[c] = M::rowsum(pb[c], l_part[c]);
      }
#pragma unroll
      for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
        for (int c = 0; c < CG; ++c)
          oacc[dt][c] = M::mma(M::from_bits(va[s][dt]), pb[c], oacc[dt][c]);
    }
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
  };

  // 2-stage ring, statically unrolled by two so each LDS access names its stage's array.
  // (the cursor advances before each barrier: scalar work off the path from the barrier to
  // the next tile's loads)
  const int wlast = (int)qw0 + 32 * CG - 1;  // this wave's last query row
  const std::false_type take_max;
  // the whole walk with the running max of every sub-tile (XO: the second walk)
  [[maybe_unused]] auto walk = [&]() {
    int key0 = next_tile();
    if (key0 >= 0) issue(kst0, vst0, key0);
    while (key0 >= 0) {
      int key0n = next_tile();
      dma_barrier();  // stage 0 landed for all waves; stage 1 no longer read
      if (key0n >= 0) issue(kst1, vst1, key0n);
      if (key0 <= wlast) compute(kst0, vst0, key0, take_max);
      key0 = key0n;
      if (key0 < 0) break;
      key0n = next_tile();
      dma_barrier();  // stage 1 landed; stage 0 no longer read
      if (key0n >= 0) issue(kst0, vst0, key0n);
      if (key0 <= wlast) compute(kst1, vst1, key0, take_max);
      key0 = key0n;
    }
  };
  // XO: the running max of the walk's first sub-tile only (in list order every wave computes
  // it: its key blocks start at or before the query block's first row; a wave that does not
  // keeps m = -inf, offsets by 0, and overflows into the second walk if its scores are large)
  [[maybe_unused]] auto walk_xo = [&]() {
    const std::true_type skip_max;
    int key0 = next_tile();
    if (key0 < 0) return;
    issue(kst0, vst0, key0);
    int key0n = next_tile();
    dma_barrier();
    if (key0n >= 0) issue(kst1, vst1, key0n);
    if (key0 <= wlast) compute(kst0, vst0, key0, take_max);
    key0 = key0n;
    while (key0 >= 0) {
      key0n = next_tile();
      dma_barrier();  // stage 1 landed; stage 0 no longer read
      if (key0n >= 0) issue(kst0, vst0, key0n);
      if (key0 <= wlast) compute(kst1, vst1, key0, skip_max);
      key0 = key0n;
      if (key0 < 0) break;
      key0n = next_tile();
      dma_barrier();  // stage 0 landed; stage 1 no longer read
      if (key0n >= 0) issue(kst1, vst1, key0n);
      if (key0 <= wlast) compute(kst0, vst0, key0, skip_max);
      key0 = key0n;
    }
  };
  if constexpr (XO) {
    __shared__ int wg_ovf;
    if (tid == 0) wg_ovf = 0;
    walk_xo();
    // a row whose sum reached 2^100 (a later score ~100 log2 units above its first sub-tile's
    // maximum) or whose output accumulators overflowed: the workgroup walks again with the
    // per-sub-tile running max
    bool bad = false;
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      const float lt = pair_sum(l_part[c]);
      bool ok = lt < 0x1p100f;
#pragma unroll
      for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) ok = ok && fabsf(oacc[dt][c][r]) < INFINITY;
      if (qrow(c) < n32 && !ok) bad = true;
    }
    __syncthreads();  // (orders the flag's clear before the writes below)
    if (__any(bad) && lane == 0) wg_ovf = 1;
    __syncthreads();  // every wave is also past its last LDS read of the walk
    if (wg_ovf) {     // workgroup-uniform
      ce = e0;
      cs = -1;
      kk = 0;
      if (lbase != 0) {
        lbase = 0;
        lreg = lane < cnt ? list[lane] : -1;
      }
#pragma unroll
      for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
        for (int c = 0; c < CG; ++c)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[dt][c][r] = 0.0f;
#pragma unroll
      for (int c = 0; c < CG; ++c) {
        m_run[c] = -INFINITY;
        l_part[c] = 0.0f;
      }
      walk();
    }
  } else {
    int key0 = next_tile();
    if (key0 >= 0) issue(kst0, vst0, key0);
    while (key0 >= 0) {
      int key0n = next_tile();
      dma_barrier();  // stage 0 landed for all waves; stage 1 no longer read
      if (key0n >= 0) issue(kst1, vst1, key0n);
      if (key0 <= wlast) compute(kst0, vst0, key0, take_max);
      key0 = key0n;
      if (key0 < 0) break;
      key0n = next_tile();
      dma_barrier();  // stage 1 landed; stage 0 no longer read
      if (key0n >= 0) issue(kst0, vst0, key0n);
      if (key0 <= wlast) compute(kst1, vst1, key0, take_max);
      key0 = key0n;
    }
  }

  // ---- epilogue: O = O^T / l ----
  if constexpr (OFS) {  // a row whose P overflowed fp16: its query block goes to the exact launch
    bool bad = false;
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      const float lt = pair_sum(l_part[c]);  // (every lane: a cross-lane sum)
      if (qrow(c) < n32 && !(lt < INFINITY)) bad = true;
    }
    if (__any(bad) && lane == 0) {
      p.redo[(b * p.Hkv + kvh) * p.nbq + i] = 1;
      p.unbounded[b * p.Hkv + kvh] = 1;
    }
  }
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    const float l_tot = pair_sum(l_part[c]);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    const int qr = qrow(c);
    if (qr < n32) {
      unsigned short* op =
          reinterpret_cast<unsigned short*>(p.o) + b * p.osb + h * p.osh + qr * p.osn;
#pragma unroll
      for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const int d0 = dt * 32 + rg * 8 + half * 4;
          uint2 wv;
          wv.x = M::pack2(oacc[dt][c][4 * rg] * inv, oacc[dt][c][4 * rg + 1] * inv);
          wv.y = M::pack2(oacc[dt][c][4 * rg + 2] * inv, oacc[dt][c][4 * rg + 3] * inv);
          *reinterpret_cast<uint2*>(op + d0) = wv;
        }
      if (p.lse != nullptr && half == 0)
        p.lse[(b * p.Hq + h) * p.n + qr] =
            l_tot > 0.0f ? (m_run[c] + log2f(l_tot)) * kLn2 : -INFINITY;
    }
  }
}

// Wide head dims (d = 128 NW, e.g. 512): a 32-key sub-tile of K and V^T is 64 KB at d = 512, so
// an LDS ring of them would leave one workgroup per CU. Here the head dim is split across the NW
// waves of a workgroup instead -- wave w owns dims [128 w, 128 w + 128) of one 32-row query group
// -- and each wave loads its K and V^T fragments from global memory straight into registers
// (their reuse across query groups and the query heads of a key head is L2's). Each wave
// contracts its dims into a partial S^T = K Q^T (32 keys x 32 rows, the K rows permuted as in
// sparse_attn_dma_kernel so P^T never leaves registers); the NW partials are summed through LDS
// in wave order, so every wave holds the same fp32 scores, runs the same online softmax (exact
// path: running max, fp32-scaled scores) and multiplies the same P into its dims of O.
template <int DT, int NW>
__global__ __launch_bounds__(NW * 64, 2) void sparse_attn_wide_kernel(AttnParams p) {
  using M = Mfma<DT>;
  typedef typename M::vec vec;
  constexpr int D = 128 * NW;
  constexpr int KD = 8;   // 16-dim k-steps of a wave's 128 dims
  constexpr int DTN = 4;  // 32-dim output tiles of a wave's 128 dims
  constexpr int KT = 32;  // keys per sub-tile
  __shared__ float sx[2][NW][16][64];  // partial scores [parity][wave][accumulator][lane]

  const int64_t L0 = logical_id(blockIdx.x, p.group);
  if (L0 >= p.total) return;
  int64_t L = L0;
  const int64_t qs = L % p.qsub;
  L /= p.qsub;
  const int64_t hg = L % p.G;
  L /= p.G;
  const int64_t kvh = L % p.Hkv;
  L /= p.Hkv;
  const int64_t b = L % p.B;
  L /= p.B;
  const int64_t i = p.nbq - 1 - L;
  const int64_t h = kvh * p.G + hg;
  const int64_t q0 = i * p.block + qs * 32;
  if (q0 >= p.n) return;
  const int64_t qmax = q0 + 31 < p.n - 1 ? q0 + 31 : p.n - 1;

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, col = lane & 31;
  const int qpos = (int)q0 + col;  // 32-bit (the host checks n < 2^31)
  const int d0 = 128 * w;          // this wave's first head dim
  const int64_t row = (b * p.Hq + h) * p.nbq + i;
  int cnt = p.kv_num[row];
  if (cnt > p.W) cnt = (int)p.W;
  if (cnt < 0) cnt = 0;
  const int32_t* list = p.kv_idx + row * p.W;
  const int S = (int)(p.block / KT);

  // Q fragments of this wave's dims (B operands of S^T = K Q^T)
  vec qf[KD];
  {
    const unsigned short* src = reinterpret_cast<const unsigned short*>(p.q) + b * p.qsb +
                                h * p.qsh + (int64_t)qpos * p.qsn + d0 + half * 8;
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
      u32x4 wv = {0u, 0u, 0u, 0u};
      if (qpos < p.n) wv = *reinterpret_cast<const u32x4*>(src + kd * 16);
      qf[kd] = M::from_bits(wv);
    }
  }
  const unsigned short* kbase = reinterpret_cast<const unsigned short*>(p.k) + b * p.ksb +
                                kvh * p.ksh + d0 + half * 8;
  const unsigned short* vtbase = reinterpret_cast<const unsigned short*>(p.vt) +
                                 (b * p.Hkv + kvh) * (int64_t)D * p.n_pad +
                                 (int64_t)(d0 + col) * p.n_pad + half * 8;
  const int krow = sigma32(col);

  const int n32 = (int)p.n, blk32 = (int)p.block, nbq32 = (int)p.nbq, qmax32 = (int)qmax;
  int lbase = 0;
  int32_t lreg = lane < cnt ? list[lane] : -1;
  int ce = 0, cs = -1;
  auto next_tile = [&]() -> int {
    while (true) {
      if (++cs == S) {
        cs = 0;
        ++ce;
      }
      if (ce >= cnt) return -1;
      if (ce - lbase >= 64) {  // wave-uniform; once per 64 list entries
        lbase = ce;
        lreg = ce + lane < cnt ? list[ce + lane] : -1;
      }
      const int c = __builtin_amdgcn_readlane(lreg, ce - lbase);
      if (c >= 0 && c < nbq32) {
        const int k0 = c * blk32 + cs * KT;
        if (k0 <= qmax32 && k0 < n32) return k0;
      }
      cs = S - 1;
    }
  };

  f32x16 oacc[DTN];
#pragma unroll
  for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.0f;
  float m_run = -INFINITY, l_part = 0.0f;
  const float c2 = p.scale_log2;
  int par = 0;
  for (int key0 = next_tile(); key0 >= 0; key0 = next_tile()) {
    // ---- partial S^T over this wave's dims ----
    int kr = key0 + krow;
    if (kr > n32 - 1) kr = n32 - 1;  // ragged tail: re-read row n-1 (masked below)
    const unsigned short* kp = kbase + (int64_t)kr * p.ksn;
    u32x4 ka[KD];
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) ka[kd] = *reinterpret_cast<const u32x4*>(kp + kd * 16);
    u32x4 va[2][DTN];
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int dt = 0; dt < DTN; ++dt)
        va[st][dt] = *reinterpret_cast<const u32x4*>(vtbase + (int64_t)dt * 32 * p.n_pad + key0 +
                                                     st * 16);
    f32x16 sacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sacc[r] = 0.0f;
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) sacc = M::mma(M::from_bits(ka[kd]), qf[kd], sacc);
    // ---- the NW partials summed in wave order (identical in every wave) ----
#pragma unroll
    for (int r = 0; r < 16; ++r) sx[par][w][r][lane] = sacc[r];
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float x = sx[par][0][r][lane];
#pragma unroll
      for (int u = 1; u < NW; ++u) x += sx[par][u][r][lane];
      sacc[r] = x;
    }
    par ^= 1;  // the next tile writes the other buffer (a wave reaches it only after every wave
               // has passed this tile's barrier, i.e. finished reading the buffer it overwrites
               // two tiles later)
    // ---- mask (diagonal / ragged tail sub-tiles) ----
    if (key0 + KT - 1 > (int)q0 || key0 + KT > n32) {
      const int lim_q = qpos - key0, lim_n = n32 - 1 - key0;
      const int lim = lim_q < lim_n ? lim_q : lim_n;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = (r >> 3) * 16 + half * 8 + (r & 7);
        if (key > lim) sacc[r] = -INFINITY;
      }
    }
    // ---- online softmax (lazy rescale) ----
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[r]);
    mx = pair_max(mx);
    const float m_cand = mx * c2;
    if (m_cand > m_run + kRescaleSlack) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_cand);
      l_part *= alpha;
#pragma unroll
      for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
      m_run = m_cand;
    }
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;
    // ---- P^T (registers) and O^T += V^T P^T over this wave's dims ----
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      float pv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) pv[j] = __builtin_amdgcn_exp2f(fmaf(sacc[8 * st + j], c2, -m_use));
      const vec pb = M::pack(pv);
      l_part = M::rowsum(pb, l_part);
#pragma unroll
      for (int dt = 0; dt < DTN; ++dt) oacc[dt] = M::mma(M::from_bits(va[st][dt]), pb, oacc[dt]);
    }
  }

  // ---- epilogue: this wave's dims of O = O^T / l ----
  const float l_tot = pair_sum(l_part);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (qpos < n32) {
    unsigned short* op = reinterpret_cast<unsigned short*>(p.o) + b * p.osb + h * p.osh +
                         (int64_t)qpos * p.osn + d0;
#pragma unroll
    for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int e0 = dt * 32 + rg * 8 + half * 4;
        uint2 wv;
        wv.x = M::pack2(oacc[dt][4 * rg] * inv, oacc[dt][4 * rg + 1] * inv);
        wv.y = M::pack2(oacc[dt][4 * rg + 2] * inv, oacc[dt][4 * rg + 3] * inv);
        *reinterpret_cast<uint2*>(op + e0) = wv;
      }
    if (p.lse != nullptr && w == 0 && half == 0)
      p.lse[(b * p.Hq + h) * p.n + qpos] = l_tot > 0.0f ? (m_run + log2f(l_tot)) * kLn2 : -INFINITY;
  }
}

// Logical work items of a launch whose workgroups own `rows` query rows (a divisor of the block,
// or the whole block 64): query sub-tiles per query block, the run of items placed together on
// one XCD (the query heads of a key head for one query block), and the grid (a multiple of 8
// runs, so every XCD receives whole runs).
inline int64_t set_rows(AttnParams& p, int64_t rows) {
  p.qsub = p.block == 64 ? 1 : p.block / rows;
  p.group = p.G * p.qsub;
  p.total = p.nbq * p.B * p.Hkv * p.G * p.qsub;
  return (p.total + 8 * p.group - 1) / (8 * p.group) * (8 * p.group);
}

template <int DT>
int launch_mfma(AttnParams& p, int64_t d, hipStream_t stream) {
  // head dim 64: 2 waves x 32 rows per workgroup for block 64 (one query block); otherwise the
  // bounded launch runs 4 waves x 32 rows (block 128) or 8 waves x 32 rows (a multiple of 256:
  // a whole 256-row query block, so each K / V^T sub-tile is read once per query block) and the
  // exact launch 4 waves x 32 rows; head dims 128 / 256 (exact path): 2 or 4 waves x 32 rows
  const bool b64 = p.block == 64;
  int64_t grid = set_rows(p, 128);
  SSA_REQUIRE(grid < (1ll << 31), SSA_ERR_UNSUPPORTED, "sparse_attn: grid too large");
  if (d == 128) {
    if (b64) sparse_attn_dma_kernel<DT, 2, 1, 2, 0, 128, 64><<<(unsigned)grid, 128, 0, stream>>>(p);
    else sparse_attn_dma_kernel<DT, 4, 1, 2, 0, 128, 64><<<(unsigned)grid, 256, 0, stream>>>(p);
  } else if (d == 256) {
    if (b64) sparse_attn_dma_kernel<DT, 2, 1, 1, 0, 256, 32><<<(unsigned)grid, 128, 0, stream>>>(p);
    else sparse_attn_dma_kernel<DT, 4, 1, 1, 0, 256, 32><<<(unsigned)grid, 256, 0, stream>>>(p);
  } else if (p.tmax2 == nullptr) {
    if (b64) sparse_attn_dma_kernel<DT, 2, 1, 2, 0><<<(unsigned)grid, 128, 0, stream>>>(p);
    else sparse_attn_dma_kernel<DT, 4, 1, 4, 0><<<(unsigned)grid, 256, 0, stream>>>(p);
  } else if (b64) {
    sparse_attn_dma_kernel<DT, 2, 1, 2, 1><<<(unsigned)grid, 128, 0, stream>>>(p);
    sparse_attn_dma_kernel<DT, 2, 1, 2, 2><<<(unsigned)grid, 128, 0, stream>>>(p);
  } else {
    // 32 rows per wave, 4 waves per SIMD (one score-fragment set per wave in 128 VGPRs: at C3
    // 4-6 % faster than 2 waves x 64 rows for the bounded rows, 2-3 % for the exact path); the
    // exact launch redoes the query blocks the bounded launch flagged
    if (p.block % 256 == 0) {
      const int64_t g1 = set_rows(p, 256);
      SSA_REQUIRE(g1 < (1ll << 31), SSA_ERR_UNSUPPORTED, "sparse_attn: grid too large");
      p.rot_ticks = p.rotate ? kRotTicks256 : 0;
      if (p.W <= 128)
        sparse_attn_dma_kernel<DT, 8, 1, 4, 1, 64, 64, true><<<(unsigned)g1, 512, 0, stream>>>(p);
      else
        sparse_attn_dma_kernel<DT, 8, 1, 4, 1><<<(unsigned)g1, 512, 0, stream>>>(p);
    } else if (p.W <= 128) {
      p.rot_ticks = p.rotate ? kRotTicks128 : 0;
      sparse_attn_dma_kernel<DT, 4, 1, 4, 1, 64, 64, true><<<(unsigned)grid, 256, 0, stream>>>(p);
    } else {
      sparse_attn_dma_kernel<DT, 4, 1, 4, 1><<<(unsigned)grid, 256, 0, stream>>>(p);
    }
    grid = set_rows(p, 128);
    sparse_attn_dma_kernel<DT, 4, 1, 4, 2><<<(unsigned)grid, 256, 0, stream>>>(p);
  }
  return launch_status("sparse_attn_dma_kernel");
}

}  // namespace
}  // namespace ssa

namespace ssa {
namespace {
// bytes of the fp16 key copy (bf16 inputs at head dim 64: the bounded rows' QK operand)
size_t k16_bytes(int dtype, int64_t B, int64_t Hkv, int64_t n_pad, int64_t d) {
  if (dtype != SSA_BF16 || d != 64) return 0;
  return ((size_t)B * (size_t)Hkv * (size_t)n_pad * 64u * 2u + 255) / 256 * 256;
}
}  // namespace
}  // namespace ssa

namespace ssa {
namespace {
// The per-(k, v) part of an attention call, into its workspace: V^T (unless vt_ready) and, with
// `norms` (16-bit, head dim 64), the key-norm pass -- the fp16 copy of K (bf16), the per-tile
// key-norm maxima and the cleared unbounded / redo flags -- fused with the transpose when both run.
int attn_prepare(const void* k, const void* v, int dtype, int64_t B, int64_t Hkv, int64_t n,
                 int64_t d, int64_t block, int64_t ksb, int64_t ksh, int64_t ksn, int64_t vsb,
                 int64_t vsh, int64_t vsn, void* workspace, bool vt_ready, bool norms,
                 hipStream_t st) {
  const int64_t nbq = (n + block - 1) / block, n_pad = nbq * block, ntile = n_pad / 64;
  const size_t vt_bytes = ((size_t)B * Hkv * d * n_pad * 2u + 255) / 256 * 256;
  const size_t k16b = k16_bytes(dtype, B, Hkv, n_pad, d);
  if (!norms) {
    if (!vt_ready) {
      KeyNorm none{};
      const dim3 tz((unsigned)(n_pad / 64), (unsigned)(B * Hkv), (unsigned)(d / 64));
      transpose_v_kernel<<<tz, 256, 0, st>>>(static_cast<const char*>(v),
                                             static_cast<char*>(workspace), Hkv, n, n_pad, vsb,
                                             vsh, vsn, d, none);
      return launch_status("transpose_v_kernel");
    }
    return SSA_OK;
  }
  unsigned short* k16 =
      k16b ? reinterpret_cast<unsigned short*>(static_cast<char*>(workspace) + vt_bytes) : nullptr;
  float* tmax2 = reinterpret_cast<float*>(static_cast<char*>(workspace) + vt_bytes + k16b);
  int* unbounded = reinterpret_cast<int*>(tmax2 + B * Hkv * ntile);
  int* redo = unbounded + B * Hkv;
  KeyNorm kn{static_cast<const unsigned short*>(k), ksb, ksh, ksn, dtype == SSA_BF16, tmax2,
             unbounded, ntile, redo, block, nbq, k16, n_pad};
  const dim3 tg((unsigned)(n_pad / 64), (unsigned)(B * Hkv));
  if (vt_ready) {
    key_norm_max_kernel<<<tg, 256, 0, st>>>(kn, Hkv, n);
    return launch_status("key_norm_max_kernel");
  }
  // V^T and the key norms in one pass
  transpose_v_kernel<<<tg, 256, 0, st>>>(static_cast<const char*>(v), static_cast<char*>(workspace),
                                         Hkv, n, n_pad, vsb, vsh, vsn, 64, kn);
  return launch_status("transpose_v_kernel");
}
}  // namespace
}  // namespace ssa

extern "C" size_t ssa_sparse_attn_workspace_size(int dtype, int64_t B, int64_t Hkv, int64_t n,
                                                 int64_t d, int64_t block) {
  if (dtype == SSA_F32 || block <= 0) return 0;
  const int64_t n_pad = (n + block - 1) / block * block;
  const size_t vt = ((size_t)B * (size_t)Hkv * (size_t)d * (size_t)n_pad * 2u + 255) / 256 * 256;
  // V^T, then (bf16, head dim 64) the fp16 copy of K, then the per-tile key-norm maxima
  // (float), one unbounded-workgroup flag (int) per key head and one redo flag (int) per
  // (key head, query block)
  const size_t tail = (size_t)(B * Hkv * (n_pad / 64) + B * Hkv + B * Hkv * (n_pad / block)) * 4u;
  return vt + ssa::k16_bytes(dtype, B, Hkv, n_pad, d) + (tail + 255) / 256 * 256;
}

extern "C" int ssa_sparse_attn_prepare(const void* k, const void* v, int dtype, int64_t B,
                                       int64_t Hkv, int64_t n, int64_t d, int64_t block,
                                       const int64_t* strides, void* workspace,
                                       size_t workspace_bytes, ssa_stream_t stream) {
  using namespace ssa;
  SSA_REQUIRE(k && v && strides && workspace, SSA_ERR_INVALID,
              "attn_prepare: NULL pointer argument");
  SSA_REQUIRE(dtype == SSA_F16 || dtype == SSA_BF16, SSA_ERR_UNSUPPORTED,
              "attn_prepare: 16-bit dtypes only");
  SSA_REQUIRE(B > 0 && Hkv > 0 && n > 0, SSA_ERR_INVALID, "attn_prepare: sizes must be positive");
  SSA_REQUIRE(d == 64 || d == 128 || d == 256 || d == 512, SSA_ERR_UNSUPPORTED,
              "attn_prepare: head_dim must be 64, 128, 256 or 512");
  SSA_REQUIRE(block == 64 || (block > 0 && block % 128 == 0), SSA_ERR_UNSUPPORTED,
              "attn_prepare: block %lld unsupported (64 or a multiple of 128)", (long long)block);
  SSA_REQUIRE(n + block < (1ll << 31), SSA_ERR_UNSUPPORTED, "attn_prepare: n too large");
  for (int s = 0; s < 6; ++s)
    SSA_REQUIRE(strides[s] % 8 == 0, SSA_ERR_UNSUPPORTED,
                "attn_prepare: stride %d (%lld) not a multiple of 16 bytes", s,
                (long long)strides[s]);
  SSA_REQUIRE(aligned16(k) && aligned16(v) && aligned16(workspace), SSA_ERR_UNSUPPORTED,
              "attn_prepare: tensors must be 16-byte aligned");
  const size_t need = ssa_sparse_attn_workspace_size(dtype, B, Hkv, n, d, block);
  SSA_REQUIRE(workspace_bytes >= need, SSA_ERR_WORKSPACE,
              "attn_prepare: workspace needs %zu bytes", need);
  const int64_t n_pad = (n + block - 1) / block * block;
  SSA_REQUIRE(B * Hkv < 65536 && n_pad / 64 < (1ll << 31), SSA_ERR_UNSUPPORTED,
              "attn_prepare: grid too large");
  return attn_prepare(k, v, dtype, B, Hkv, n, d, block, strides[0], strides[1], strides[2],
                      strides[3], strides[4], strides[5], workspace, false, d == 64,
                      static_cast<hipStream_t>(stream));
}

extern "C" int ssa_transpose_v(const void* v, int dtype, int64_t B, int64_t Hkv, int64_t n,
                               int64_t d, int64_t block, int64_t stride_b, int64_t stride_h,
                               int64_t stride_n, void* vt, size_t vt_bytes, ssa_stream_t stream) {
  using namespace ssa;
  SSA_REQUIRE(v && vt, SSA_ERR_INVALID, "transpose_v: NULL pointer argument");
  SSA_REQUIRE(dtype == SSA_F16 || dtype == SSA_BF16, SSA_ERR_UNSUPPORTED,
              "transpose_v: 16-bit dtypes only");
  SSA_REQUIRE(B > 0 && Hkv > 0 && n > 0 && block > 0, SSA_ERR_INVALID, "transpose_v: bad sizes");
  SSA_REQUIRE(d == 64 || d == 128 || d == 256 || d == 512, SSA_ERR_UNSUPPORTED,
              "transpose_v: head_dim must be 64, 128, 256 or 512");
  SSA_REQUIRE(block % 64 == 0, SSA_ERR_UNSUPPORTED, "transpose_v: block must be a multiple of 64");
  SSA_REQUIRE(aligned16(v) && aligned16(vt) && stride_b % 8 == 0 && stride_h % 8 == 0 &&
                  stride_n % 8 == 0,
              SSA_ERR_UNSUPPORTED, "transpose_v: 16-byte alignment required");
  const size_t need = ssa_sparse_attn_workspace_size(dtype, B, Hkv, n, d, block);
  SSA_REQUIRE(vt_bytes >= need, SSA_ERR_WORKSPACE, "transpose_v: needs %zu bytes", need);
  const int64_t n_pad = (n + block - 1) / block * block;
  SSA_REQUIRE(B * Hkv < 65536 && n_pad / 64 < (1ll << 31), SSA_ERR_UNSUPPORTED,
              "transpose_v: grid too large");
  dim3 tg((unsigned)(n_pad / 64), (unsigned)(B * Hkv), (unsigned)(d / 64));
  KeyNorm none{};
  transpose_v_kernel<<<tg, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const char*>(v), static_cast<char*>(vt), Hkv, n, n_pad, stride_b, stride_h,
      stride_n, d, none);
  return launch_status("transpose_v_kernel");
}

extern "C" int ssa_sparse_attn_fwd(const void* q, const void* k, const void* v, void* out,
                                   int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t n,
                                   int64_t d, int64_t block, const int64_t* strides,
                                   const int32_t* kv_num, const int32_t* kv_idx, int64_t W,
                                   float scale, float* lse, int flags, void* workspace,
                                   size_t workspace_bytes, ssa_stream_t stream) {
  using namespace ssa;
  SSA_REQUIRE(q && k && v && out && strides && kv_num && kv_idx, SSA_ERR_INVALID,
              "sparse_attn: NULL pointer argument");
  SSA_REQUIRE(dtype == SSA_F32 || dtype == SSA_F16 || dtype == SSA_BF16, SSA_ERR_UNSUPPORTED,
              "sparse_attn: unknown dtype %d", dtype);
  SSA_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && n > 0 && W > 0, SSA_ERR_INVALID,
              "sparse_attn: sizes must be positive");
  SSA_REQUIRE(Hq % Hkv == 0, SSA_ERR_INVALID, "sparse_attn: Hq not a multiple of Hkv");
  SSA_REQUIRE(d == 64 || ((d == 128 || d == 256 || d == 512) && dtype != SSA_F32),
              SSA_ERR_UNSUPPORTED,
              "sparse_attn: head_dim %lld unsupported (64; 128, 256 and 512 for 16-bit inputs)",
              (long long)d);
  SSA_REQUIRE(block == 64 || (block > 0 && block % 128 == 0), SSA_ERR_UNSUPPORTED,
              "sparse_attn: block %lld unsupported (64 or a multiple of 128)", (long long)block);
  SSA_REQUIRE(B * Hq < (1ll << 24), SSA_ERR_UNSUPPORTED, "sparse_attn: too many heads");
  SSA_REQUIRE(n + block < (1ll << 31), SSA_ERR_UNSUPPORTED,
              "sparse_attn: n = %lld too large (key positions are 32-bit)", (long long)n);
  SSA_REQUIRE((flags & ~(SSA_ATTN_VT_READY | SSA_ATTN_ROTATE | SSA_ATTN_EXACT |
                          SSA_ATTN_PREPARED)) == 0,
              SSA_ERR_INVALID,
              "sparse_attn: unknown flags");
  const int64_t vec = dtype == SSA_F32 ? 4 : 8;
  for (int s = 0; s < 12; ++s)
    SSA_REQUIRE(strides[s] % vec == 0, SSA_ERR_UNSUPPORTED,
                "sparse_attn: stride %d (%lld) not a multiple of 16 bytes", s,
                (long long)strides[s]);
  SSA_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out), SSA_ERR_UNSUPPORTED,
              "sparse_attn: tensors must be 16-byte aligned");
  SSA_REQUIRE(scale > 0.0f && isfinite(scale), SSA_ERR_INVALID, "sparse_attn: scale must be > 0");

  AttnParams p;
  p.q = static_cast<const char*>(q);
  p.k = static_cast<const char*>(k);
  p.v = static_cast<const char*>(v);
  p.o = static_cast<char*>(out);
  p.qsb = strides[0]; p.qsh = strides[1]; p.qsn = strides[2];
  p.ksb = strides[3]; p.ksh = strides[4]; p.ksn = strides[5];
  p.vsb = strides[6]; p.vsh = strides[7]; p.vsn = strides[8];
  p.osb = strides[9]; p.osh = strides[10]; p.osn = strides[11];
  p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.G = Hq / Hkv; p.n = n; p.block = block;
  p.nbq = (n + block - 1) / block;
  p.n_pad = p.nbq * block;
  p.kv_num = kv_num; p.kv_idx = kv_idx; p.W = W;
  p.scale_log2 = scale * kLog2e;
  p.lse = lse;
  hipStream_t st = static_cast<hipStream_t>(stream);

  p.tmax2 = nullptr;
  p.unbounded = nullptr;
  p.redo = nullptr;
  p.k16 = nullptr;
  p.rot_ticks = 0;
  p.rotate = (flags & SSA_ATTN_ROTATE) != 0;
  p.ntile = p.n_pad / 64;
  if (dtype == SSA_F32) {
    p.vt = nullptr;
    p.qsub = block / 64;
    p.group = 1;
    p.total = p.nbq * B * Hq * p.qsub;
    SSA_REQUIRE(p.total < (1ll << 31), SSA_ERR_UNSUPPORTED, "sparse_attn: grid too large");
    sparse_attn_f32_kernel<<<(unsigned)p.total, 64, 0, st>>>(p);
    return launch_status("sparse_attn_f32_kernel");
  }
  const size_t need = ssa_sparse_attn_workspace_size(dtype, B, Hkv, n, d, block);
  SSA_REQUIRE(workspace != nullptr && workspace_bytes >= need && aligned16(workspace),
              SSA_ERR_WORKSPACE, "sparse_attn: workspace needs %zu bytes (16-byte aligned)", need);
  p.vt = static_cast<const char*>(workspace);
  SSA_REQUIRE(B * Hkv < 65536 && p.n_pad / 64 < (1ll << 31), SSA_ERR_UNSUPPORTED,
              "sparse_attn: grid too large");
  // after V^T: the fp16 copy of K (bf16, head dim 64), the per-tile key-norm maxima, then mode
  // 1's unbounded flags (all written by the key-norm pass, every entry; by ssa_sparse_attn_prepare
  // for a SSA_ATTN_PREPARED call)
  const size_t vt_bytes = ((size_t)B * Hkv * d * p.n_pad * 2u + 255) / 256 * 256;
  const size_t k16b = k16_bytes(dtype, B, Hkv, p.n_pad, d);
  const bool norms = d == 64 && !(flags & SSA_ATTN_EXACT);
  if (!(flags & SSA_ATTN_PREPARED))
    SSA_TRY(attn_prepare(k, v, dtype, B, Hkv, n, d, block, p.ksb, p.ksh, p.ksn, p.vsb, p.vsh,
                         p.vsn, workspace, (flags & SSA_ATTN_VT_READY) != 0, norms, st));
  if (!norms) {  // exact path only
    if (d == 512) {  // head dim split across 4 waves, 32 query rows per workgroup
      p.qsub = block / 32;
      p.group = p.G * p.qsub;
      p.total = p.nbq * B * Hkv * p.G * p.qsub;
      const int64_t grid = (p.total + 8 * p.group - 1) / (8 * p.group) * (8 * p.group);
      SSA_REQUIRE(grid < (1ll << 31), SSA_ERR_UNSUPPORTED, "sparse_attn: grid too large");
      if (dtype == SSA_BF16) sparse_attn_wide_kernel<SSA_BF16, 4><<<(unsigned)grid, 256, 0, st>>>(p);
      else sparse_attn_wide_kernel<SSA_F16, 4><<<(unsigned)grid, 256, 0, st>>>(p);
      return launch_status("sparse_attn_wide_kernel");
    }
    if (dtype == SSA_BF16) return launch_mfma<SSA_BF16>(p, d, st);
    return launch_mfma<SSA_F16>(p, d, st);
  }
  float* tmax2 = reinterpret_cast<float*>(static_cast<char*>(workspace) + vt_bytes + k16b);
  p.tmax2 = tmax2;
  p.unbounded = reinterpret_cast<int*>(tmax2 + B * Hkv * p.ntile);
  p.redo = p.unbounded + B * Hkv;
  p.k16 = k16b ? static_cast<const char*>(workspace) + vt_bytes : nullptr;
  if (dtype == SSA_BF16) return launch_mfma<SSA_BF16>(p, 64, st);
  return launch_mfma<SSA_F16>(p, 64, st);
}
