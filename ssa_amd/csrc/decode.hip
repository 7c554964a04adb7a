// Routed decode: one query token per head attends the keys <= pos of its selected blocks.
//
// decode_partial_kernel: one wave per (query row, selected block) -- the gather is split over
//   every selected block of every head, so a step's ~30 MB of K/V are read by ~1000 waves in
//   parallel. Each wave computes its block's scores (one key per lane per pass, 16-byte row
//   loads; for blocks of <= 128 keys the V rows are loaded before the scores), the block's max /
//   sum in fp32 and its unnormalised output row, and writes (m, l, o) to the workspace.
// decode_combine_kernel: merges a row's partials with the usual max-rescaling (4 waves per row).
// decode_step: append the new token and convert the query rows (one launch) -> summarise a
//   just-completed block -> route the query over the complete blocks (route_impl,
//   SSA_ROUTE_QUERY) -> partial -> combine.
//
// Reference: ssa/ivf_decode.py:49-62 (decode_attend), :128-136 (per-step body);
// ssa/gemma_ssa.py:85-137,225-240 (exact per-query router and softmax at q_len = 1).
#include <math.h>

#include <mutex>

#include "common.h"

namespace ssa {

int launch_block_summary(const void* x, int dtype, int64_t B, int64_t H, int64_t n, int64_t d,
                         int64_t sb, int64_t sh, int64_t sn, int64_t block, int64_t n_real,
                         int mode, float* mu, float* var, float* m3, int64_t nb_out,
                         int64_t block_offset, hipStream_t stream);
int route_impl(const void* rows, int rows_dt, const float* mu, const float* var, const float* m3,
               int64_t B,
               int64_t Hq, int64_t Hkv, int64_t nbq, int64_t nbk, int64_t d, int mode,
               int64_t top_c, float budget_frac, int64_t local, float coef2, float coef3,
               int64_t query_pos, int64_t block, int64_t pool, int32_t* kv_num, int32_t* kv_idx,
               int64_t W, void* workspace, size_t workspace_bytes, hipStream_t stream);

bool masked_tiled_ok(int64_t d, int64_t block, int64_t n);
size_t masked_tiled_workspace(int64_t B, int64_t Hq, int64_t n, int64_t block);
int masked_tiled_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                     int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t n, int64_t block,
                     const int64_t* strides, const int32_t* kv_num, const int32_t* kv_idx,
                     int64_t W, float scale, void* workspace, size_t workspace_bytes,
                     hipStream_t st);
int masked_tiled_bwd(const void* q, const void* k, const void* v, const void* out,
                     const void* dout, const float* lse, void* dq, void* dk, void* dv,
                     int dtype, int grad_dtype, int flags, int64_t B, int64_t Hq, int64_t Hkv,
                     int64_t n, int64_t block,
                     const int64_t* strides, const int32_t* kv_num, const int32_t* kv_idx,
                     int64_t W, float scale, void* workspace, size_t workspace_bytes,
                     hipStream_t st);

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kMaxDecodeBlock = 1024;
constexpr int kMaxDecodeD = 512;

struct DecodeParams {
  const char* q;
  const char* k;
  const char* v;
  char* o;
  int64_t qsb, qsh, qsn, ksb, ksh, ksn, vsb, vsh, vsn, osb, osh, osn;
  int64_t B, Hq, G, nq, cap, d, block, pos;
  const int32_t* kv_num;
  const int32_t* kv_idx;
  int64_t W;
  float scale_log2;
  float* part;  // (B*Hq*nq, W, d + 2): m, l, o[d]
  float* lse;   // optional (B*Hq*nq): natural-log sum of exp of the scaled scores of the row
  // decode step with the append folded in: the token at pos is not yet in the caches; its key /
  // value rows are read from k_new / v_new (B, Hkv, d), and one workgroup per key head writes
  // them into the caches (no workgroup of the launch reads cache row pos)
  int fused_append = 0;
  const char* k_new = nullptr;
  const char* v_new = nullptr;
  int64_t knb = 0, knh = 0, vnb = 0, vnh = 0;
};

template <int DT>
__device__ inline float load_elem(const char* base, int64_t idx) {
  if constexpr (DT == SSA_F32) return reinterpret_cast<const float*>(base)[idx];
  else {
    unsigned short u = reinterpret_cast<const unsigned short*>(base)[idx];
    if constexpr (DT == SSA_BF16) return __uint_as_float((unsigned int)u << 16);
    else return (float)__builtin_bit_cast(_Float16, u);
  }
}

template <int DT>
__device__ inline void store_elem(char* base, int64_t idx, float x) {
  if constexpr (DT == SSA_F32) reinterpret_cast<float*>(base)[idx] = x;
  else if constexpr (DT == SSA_BF16)
    reinterpret_cast<unsigned short*>(base)[idx] = __builtin_bit_cast(unsigned short, (__bf16)x);
  else
    reinterpret_cast<unsigned short*>(base)[idx] = __builtin_bit_cast(unsigned short, (_Float16)x);
}

__device__ inline float wave_max(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, 64));
  return x;
}
__device__ inline float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// Partial softmax attention of query row (b, h, r) over key block c: (m, l, o[d]) into part.
template <int DT>
__device__ inline void block_partial(const DecodeParams& p, float* part, float* qs, float* ps,
                                     int64_t b, int64_t h, int64_t kvh, int64_t r, int64_t pos,
                                     int64_t c) {
  const int lane = threadIdx.x;
  const int d = (int)p.d;
  const int64_t key0 = c * p.block;
  int64_t key1 = key0 + p.block;
  if (key1 > pos + 1) key1 = pos + 1;
  if (key1 > p.cap) key1 = p.cap;
  const int nk = (int)(key1 - key0);
  // PV lane layout (16-bit): key group kg = lane / 8, 16-byte chunk ch = lane % 8 of the V row.
  // Blocks of at most 8 * kPre keys with d <= 64 load their V rows up front, in flight while the
  // scores are computed.
  constexpr int kPre = 16;
  const int kg = lane >> 3, ch = lane & 7;
  const int64_t voff = b * p.vsb + kvh * p.vsh;
  const int64_t koff = b * p.ksb + kvh * p.ksh;
  const bool pre = DT != SSA_F32 && d <= 64 && nk <= 8 * kPre;
  // row pointers of key `key` (the token being appended comes from k_new / v_new)
  constexpr int es = DT == SSA_F32 ? 4 : 2;
  const int64_t newkey = p.fused_append ? pos : -1;
  auto krow = [&](int64_t key) -> const char* {
    return key == newkey ? p.k_new + (b * p.knb + kvh * p.knh) * es : p.k + (koff + key * p.ksn) * es;
  };
  auto vrow = [&](int64_t key) -> const char* {
    return key == newkey ? p.v_new + (b * p.vnb + kvh * p.vnh) * es : p.v + (voff + key * p.vsn) * es;
  };
  u32x4 vpre[kPre];
  if constexpr (DT != SSA_F32) {
    if (pre) {
#pragma unroll
      for (int t = 0; t < kPre; ++t) {
        const int kk = kg + 8 * t;
        vpre[t] = u32x4{0u, 0u, 0u, 0u};
        if (kk < nk && ch * 8 < d)
          vpre[t] = *reinterpret_cast<const u32x4*>(
              reinterpret_cast<const unsigned short*>(vrow(key0 + kk)) + ch * 8);
      }
    }
  }

  const char* qb = p.q;
  const int64_t qoff = b * p.qsb + h * p.qsh + r * p.qsn;
  for (int e = lane; e < d; e += 64) qs[e] = load_elem<DT>(qb, qoff + e);
  __syncthreads();

  float mloc = -INFINITY;
  for (int kk = lane; kk < nk; kk += 64) {
    const char* kr = krow(key0 + kk);
    float s = 0.0f;
    if constexpr (DT == SSA_F32) {
      for (int e = 0; e < d; e += 4) {
        const f32x4 kv = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(kr) + e);
        s = fmaf(qs[e], kv[0], s);
        s = fmaf(qs[e + 1], kv[1], s);
        s = fmaf(qs[e + 2], kv[2], s);
        s = fmaf(qs[e + 3], kv[3], s);
      }
    } else {
      for (int e = 0; e < d; e += 8) {
        const u32x4 w =
            *reinterpret_cast<const u32x4*>(reinterpret_cast<const unsigned short*>(kr) + e);
        float kv[8];
        unpack8(w, kv, DT == SSA_BF16);
#pragma unroll
        for (int t = 0; t < 8; ++t) s = fmaf(qs[e + t], kv[t], s);
      }
    }
    const float sl = s * p.scale_log2;
    ps[kk] = sl;
    mloc = fmaxf(mloc, sl);
  }
  const float m = wave_max(mloc);
  __syncthreads();
  float lloc = 0.0f;
  for (int kk = lane; kk < nk; kk += 64) {
    const float pk = exp2f(ps[kk] - m);
    ps[kk] = pk;
    lloc += pk;
  }
  const float l = wave_sum(lloc);
  __syncthreads();
  if constexpr (DT == SSA_F32) {
    for (int e = lane; e < d; e += 64) {
      float acc = 0.0f;
      for (int kk = 0; kk < nk; ++kk)
        acc = fmaf(ps[kk], load_elem<DT>(vrow(key0 + kk), e), acc);
      part[2 + e] = acc;
    }
  } else if (pre) {  // the prefetched V rows; the 8 key groups summed with shuffles
    float acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = 0.0f;
#pragma unroll
    for (int t = 0; t < kPre; ++t) {
      const int kk = kg + 8 * t;
      if (kk < nk) {
        float vv[8];
        unpack8(vpre[t], vv, DT == SSA_BF16);
        const float pk = ps[kk];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = fmaf(pk, vv[e], acc[e]);
      }
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      float x = acc[t];
      x += __shfl_xor(x, 8, 64);
      x += __shfl_xor(x, 16, 64);
      x += __shfl_xor(x, 32, 64);
      acc[t] = x;
    }
    if (kg == 0 && ch * 8 < d)
#pragma unroll
      for (int t = 0; t < 8; ++t) part[2 + ch * 8 + t] = acc[t];
  } else {
    // 8 keys per pass, 16-byte V row loads; the 8 key groups are summed with shuffles.
    for (int e0 = 0; e0 < d; e0 += 64) {
      const bool on = e0 + ch * 8 < d;
      float acc[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[t] = 0.0f;
      if (on) {
#pragma unroll 4
        for (int kk = kg; kk < nk; kk += 8) {
          const u32x4 wv = *reinterpret_cast<const u32x4*>(
              reinterpret_cast<const unsigned short*>(vrow(key0 + kk)) + e0 + ch * 8);
          float vv[8];
          unpack8(wv, vv, DT == SSA_BF16);
          const float pk = ps[kk];
#pragma unroll
          for (int t = 0; t < 8; ++t) acc[t] = fmaf(pk, vv[t], acc[t]);
        }
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        float x = acc[t];
        x += __shfl_xor(x, 8, 64);
        x += __shfl_xor(x, 16, 64);
        x += __shfl_xor(x, 32, 64);
        acc[t] = x;
      }
      if (kg == 0 && on)
#pragma unroll
        for (int t = 0; t < 8; ++t) part[2 + e0 + ch * 8 + t] = acc[t];
    }
  }
  if (lane == 0) {
    part[0] = m;
    part[1] = l;
  }
}

// grid (B*Hq*nq), 4 waves per row: wave w merges partials [w * q, (w + 1) * q) of the row (q =
// ceil(cnt / 4)) with the usual max-rescaling, loading 8 partial rows at a time (one memory
// latency per batch, not per partial); the waves' sums are then added through LDS.
template <int DT>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeParams p) {
  __shared__ float red[4][kMaxDecodeD];
  __shared__ float sm[4];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t rowid = blockIdx.x;
  int cnt = p.kv_num[rowid];
  if (cnt > p.W) cnt = (int)p.W;
  if (cnt < 0) cnt = 0;
  const int64_t stride = p.d + 2;
  const float* rp = p.part + rowid * p.W * stride;
  float M = -INFINITY;
  for (int j = tid; j < cnt; j += 256) M = fmaxf(M, rp[j * stride]);
  M = wave_max(M);
  if (lane == 0) sm[wv] = M;
  __syncthreads();
  M = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
  __syncthreads();
  const int qn = (cnt + 3) / 4;
  const int ja = wv * qn, jz = ja + qn < cnt ? ja + qn : cnt;
  float L = 0.0f;
  float acc[kMaxDecodeD / 64];
#pragma unroll
  for (int k = 0; k < kMaxDecodeD / 64; ++k) acc[k] = 0.0f;
  for (int j0 = ja; j0 < jz; j0 += 64) {
    const int jl = j0 + lane;
    float mj = -INFINITY, lj = 0.0f;
    if (jl < jz) {
      mj = rp[jl * stride];
      lj = rp[jl * stride + 1];
    }
    const float wl = mj == -INFINITY ? 0.0f : exp2f(mj - M);  // empty partials: weight 0
    L += lj * wl;
    const int jn = jz - j0 < 64 ? jz - j0 : 64;
    for (int jb = 0; jb < jn; jb += 8) {
#pragma unroll
      for (int k = 0; k < kMaxDecodeD / 64; ++k) {
        if (64 * k >= p.d) break;  // uniform
        float x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const bool in = jb + u < jn && lane + 64 * k < p.d;
          x[u] = in ? rp[(j0 + jb + u) * stride + 2 + lane + 64 * k] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) acc[k] = fmaf(x[u], __shfl(wl, (jb + u) & 63, 64), acc[k]);
      }
    }
  }
  L = wave_sum(L);
  if (lane == 0) sm[wv] = L;
#pragma unroll
  for (int k = 0; k < kMaxDecodeD / 64; ++k)
    if (lane + 64 * k < p.d) red[wv][lane + 64 * k] = acc[k];
  __syncthreads();
  L = sm[0] + sm[1] + sm[2] + sm[3];
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  const int64_t bh = rowid / p.nq, r = rowid % p.nq;
  const int64_t b = bh / p.Hq, h = bh % p.Hq;
  for (int e = tid; e < p.d; e += 256)
    store_elem<DT>(p.o, b * p.osb + h * p.osh + r * p.osn + e,
                   (red[0][e] + red[1][e] + red[2][e] + red[3][e]) * inv);
  if (p.lse != nullptr && tid == 0) p.lse[rowid] = L > 0.0f ? (M + log2f(L)) * kLn2 : -INFINITY;
}

// grid (rows * W): block x handles selected block j = x % W of query row x / W, one wave each.
template <int DT>
__global__ __launch_bounds__(64) void decode_partial_kernel(DecodeParams p) {
  __shared__ float qs[kMaxDecodeD];
  __shared__ float ps[kMaxDecodeBlock];
  const int lane = threadIdx.x;
  const int64_t j = blockIdx.x % p.W;
  const int64_t rowid = blockIdx.x / p.W;  // (b*Hq + h)*nq + r
  const int64_t bh = rowid / p.nq, r = rowid % p.nq;
  const int64_t b = bh / p.Hq, h = bh % p.Hq, kvh = h / p.G;
  const int64_t pos = p.pos + r;
  const int d = (int)p.d;
  float* part = p.part + (rowid * p.W + j) * (p.d + 2);

  int cnt = p.kv_num[rowid];
  if (cnt > p.W) cnt = (int)p.W;
  const int32_t* list = p.kv_idx + rowid * p.W;
  bool empty = j >= cnt;
  int64_t c = 0;
  if (!empty) {
    c = list[j];
    const int64_t nblk = (p.cap + p.block - 1) / p.block;
    if (c < 0 || c >= nblk || c * p.block > pos) empty = true;
    for (int64_t jj = 0; jj < j && !empty; ++jj)  // a repeated id is attended once
      if (list[jj] == c) empty = true;
  }
  if (empty) {
    if (lane == 0) {
      part[0] = -INFINITY;
      part[1] = 0.0f;
    }
    for (int e = lane; e < d; e += 64) part[2 + e] = 0.0f;
  } else {
    block_partial<DT>(p, part, qs, ps, b, h, kvh, r, pos, c);
  }
  // folded append: workgroup (j = 0) of the first query head of each key head writes the new
  // token into the caches; every read of that row in this launch comes from k_new / v_new
  if (p.fused_append && j == 0 && r == 0 && h % p.G == 0) {
    for (int e = lane; e < d; e += 64) {
      store_elem<DT>(const_cast<char*>(p.k), b * p.ksb + kvh * p.ksh + pos * p.ksn + e,
                     load_elem<DT>(p.k_new, b * p.knb + kvh * p.knh + e));
      store_elem<DT>(const_cast<char*>(p.v), b * p.vsb + kvh * p.vsh + pos * p.vsn + e,
                     load_elem<DT>(p.v_new, b * p.vnb + kvh * p.vnh + e));
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Backward of the per-row block-sparse softmax attention (ssa_swap.ssa_masked): for query row i
// with output O_i, upstream gradient dO_i and log-sum-exp lse_i, over its selected keys j <= pos:
//   P_ij = exp(scale q_i.k_j - lse_i), dP_ij = dO_i.v_j, D_i = dO_i.O_i, dS_ij = P_ij (dP_ij - D_i)
//   dq_i += scale sum_j dS_ij k_j,  dk_j += scale dS_ij q_i,  dv_j += P_ij dO_i.
// One wave per (row, selected block) as in the forward; dq/dk/dv are fp32 and accumulated with
// atomics (summation order varies from run to run at the last bit).
// ---------------------------------------------------------------------------------------------
struct BwdParams {
  DecodeParams f;       // q, k, v, out (as o), strides, lists, sizes of the forward
  const char* dout;     // upstream gradient, strides of out
  const float* lse;
  const float* delta;   // D_i (B*Hq*nq)
  float* dq;            // (B, Hq, nq, d) fp32 contiguous
  float* dk;            // (B, Hkv, cap, d) fp32 contiguous
  float* dv;
  int64_t Hkv;
};

// D_i = dO_i . O_i. grid (rows), one wave each.
template <int DT>
__global__ __launch_bounds__(64) void masked_delta_kernel(BwdParams bp) {
  const DecodeParams& p = bp.f;
  const int64_t rowid = blockIdx.x;
  const int64_t bh = rowid / p.nq, r = rowid % p.nq;
  const int64_t b = bh / p.Hq, h = bh % p.Hq;
  const int64_t off = b * p.osb + h * p.osh + r * p.osn;
  float acc = 0.0f;
  for (int e = threadIdx.x; e < p.d; e += 64)
    acc = fmaf(load_elem<DT>(bp.dout, off + e), load_elem<DT>(p.o, off + e), acc);
  acc = wave_sum(acc);
  if (threadIdx.x == 0) const_cast<float*>(bp.delta)[rowid] = acc;
}

__global__ __launch_bounds__(256) void zero_f32_kernel(float* x, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    x[i] = 0.0f;
}

// grid (rows * W), one wave per (row, selected block).
template <int DT>
__global__ __launch_bounds__(64) void masked_bwd_kernel(BwdParams bp) {
  const DecodeParams& p = bp.f;
  __shared__ float qs[kMaxDecodeD];
  __shared__ float gs[kMaxDecodeD];  // dO_i
  __shared__ float ps[kMaxDecodeBlock];
  __shared__ float dss[kMaxDecodeBlock];
  const int lane = threadIdx.x;
  const int64_t j = blockIdx.x % p.W;
  const int64_t rowid = blockIdx.x / p.W;
  const int64_t bh = rowid / p.nq, r = rowid % p.nq;
  const int64_t b = bh / p.Hq, h = bh % p.Hq, kvh = h / p.G;
  const int64_t pos = p.pos + r;
  const int d = (int)p.d;
  int cnt = p.kv_num[rowid];
  if (cnt > p.W) cnt = (int)p.W;
  if (j >= cnt) return;
  const int32_t* list = p.kv_idx + rowid * p.W;
  const int64_t c = list[j];
  const int64_t nblk = (p.cap + p.block - 1) / p.block;
  if (c < 0 || c >= nblk || c * p.block > pos) return;
  for (int64_t jj = 0; jj < j; ++jj)  // a repeated id is attended (and differentiated) once
    if (list[jj] == c) return;
  const int64_t key0 = c * p.block;
  int64_t key1 = key0 + p.block;
  if (key1 > pos + 1) key1 = pos + 1;
  if (key1 > p.cap) key1 = p.cap;
  const int nk = (int)(key1 - key0);
  const float lse2 = bp.lse[rowid] * kLog2e;  // log2 domain
  const float Di = bp.delta[rowid];
  const float scale = p.scale_log2 / kLog2e;

  const int64_t qoff = b * p.qsb + h * p.qsh + r * p.qsn;
  const int64_t goff = b * p.osb + h * p.osh + r * p.osn;
  for (int e = lane; e < d; e += 64) {
    qs[e] = load_elem<DT>(p.q, qoff + e);
    gs[e] = load_elem<DT>(bp.dout, goff + e);
  }
  __syncthreads();
  const int64_t koff = b * p.ksb + kvh * p.ksh, voff = b * p.vsb + kvh * p.vsh;
  for (int kk = lane; kk < nk; kk += 64) {
    float s = 0.0f, dp = 0.0f;
    const int64_t kr = koff + (key0 + kk) * p.ksn, vr = voff + (key0 + kk) * p.vsn;
    for (int e = 0; e < d; ++e) {
      s = fmaf(qs[e], load_elem<DT>(p.k, kr + e), s);
      dp = fmaf(gs[e], load_elem<DT>(p.v, vr + e), dp);
    }
    const float pk = exp2f(s * p.scale_log2 - lse2);
    ps[kk] = pk;
    dss[kk] = pk * (dp - Di);
  }
  __syncthreads();
  // dq_i (lane = head dim): scale * sum_j dS_ij k_j
  const int64_t dqoff = rowid * p.d;
  for (int e = lane; e < d; e += 64) {
    float acc = 0.0f;
    for (int kk = 0; kk < nk; ++kk) acc = fmaf(dss[kk], load_elem<DT>(p.k, koff + (key0 + kk) * p.ksn + e), acc);
    atomicAdd(bp.dq + dqoff + e, scale * acc);
  }
  // dk_j += scale dS_ij q_i, dv_j += P_ij dO_i (lane = head dim, coalesced rows)
  const int64_t kvrow = (b * bp.Hkv + kvh) * p.cap;
  for (int kk = 0; kk < nk; ++kk) {
    const float dsk = scale * dss[kk], pk = ps[kk];
    float* dkr = bp.dk + (kvrow + key0 + kk) * p.d;
    float* dvr = bp.dv + (kvrow + key0 + kk) * p.d;
    for (int e = lane; e < d; e += 64) {
      if (dsk != 0.0f) atomicAdd(dkr + e, dsk * qs[e]);
      if (pk != 0.0f) atomicAdd(dvr + e, pk * gs[e]);
    }
  }
}

// Element strides of the append: new token rows (b,h) and caches (b,h,n).
struct AppendStrides {
  int64_t knb, knh, vnb, vnh, kcb, kch, kcn, vcb, vch, vcn;
};

// One launch for the per-step preparation. grid (B*Hq): block (b, h) converts query row (b, h)
// to contiguous fp32 (the router's rows), and the first query head of each key head also writes
// k_new/v_new (B, Hkv, d) into the caches at row pos.
template <int DT>
__global__ __launch_bounds__(64) void decode_prep_kernel(const char* q, float* qf, const char* kn,
                                                         const char* vn, char* kc, char* vc,
                                                         int64_t Hq, int64_t G, int64_t d,
                                                         int64_t qsb, int64_t qsh, int64_t pos,
                                                         AppendStrides st) {
  const int64_t r = blockIdx.x;
  const int64_t b = r / Hq, h = r % Hq;
  for (int e = threadIdx.x; e < d; e += 64) qf[r * d + e] = load_elem<DT>(q, b * qsb + h * qsh + e);
  if (h % G != 0) return;
  const int64_t kvh = h / G;
  for (int e = threadIdx.x; e < d; e += 64) {
    store_elem<DT>(kc, b * st.kcb + kvh * st.kch + pos * st.kcn + e,
                   load_elem<DT>(kn, b * st.knb + kvh * st.knh + e));
    store_elem<DT>(vc, b * st.vcb + kvh * st.vch + pos * st.vcn + e,
                   load_elem<DT>(vn, b * st.vnb + kvh * st.vnh + e));
  }
}

int run_attend(int dtype, DecodeParams& p, hipStream_t stream) {
  const int64_t rows = p.B * p.Hq * p.nq;
  SSA_REQUIRE(rows * p.W < (1ll << 31), SSA_ERR_UNSUPPORTED, "decode: grid too large");
  const unsigned g1 = (unsigned)(rows * p.W);
  switch (dtype) {
    case SSA_F32: decode_partial_kernel<SSA_F32><<<g1, 64, 0, stream>>>(p); break;
    case SSA_F16: decode_partial_kernel<SSA_F16><<<g1, 64, 0, stream>>>(p); break;
    default: decode_partial_kernel<SSA_BF16><<<g1, 64, 0, stream>>>(p); break;
  }
  SSA_TRY(launch_status("decode_partial_kernel"));
  const unsigned g2 = (unsigned)rows;
  switch (dtype) {
    case SSA_F32: decode_combine_kernel<SSA_F32><<<g2, 256, 0, stream>>>(p); break;
    case SSA_F16: decode_combine_kernel<SSA_F16><<<g2, 256, 0, stream>>>(p); break;
    default: decode_combine_kernel<SSA_BF16><<<g2, 256, 0, stream>>>(p); break;
  }
  return launch_status("decode_combine_kernel");
}

int check_decode(int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t nq, int64_t cap,
                 int64_t d, int64_t block, int64_t pos, int64_t W, const int64_t* strides,
                 int nstrides) {
  SSA_REQUIRE(dtype == SSA_F32 || dtype == SSA_F16 || dtype == SSA_BF16, SSA_ERR_UNSUPPORTED,
              "decode: unknown dtype %d", dtype);
  SSA_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && nq > 0 && cap > 0 && W > 0 && block > 0,
              SSA_ERR_INVALID, "decode: sizes must be positive");
  SSA_REQUIRE(Hq % Hkv == 0, SSA_ERR_INVALID, "decode: Hq not a multiple of Hkv");
  SSA_REQUIRE(pos >= 0 && pos + nq <= cap, SSA_ERR_INVALID,
              "decode: query positions [%lld,%lld) outside the cache [0,%lld)", (long long)pos,
              (long long)(pos + nq), (long long)cap);
  SSA_REQUIRE(d % 8 == 0 && d >= 8 && d <= kMaxDecodeD, SSA_ERR_UNSUPPORTED,
              "decode: head_dim %lld unsupported (multiple of 8, <= %d)", (long long)d, kMaxDecodeD);
  SSA_REQUIRE(block <= kMaxDecodeBlock, SSA_ERR_UNSUPPORTED, "decode: block > %d", kMaxDecodeBlock);
  SSA_REQUIRE(W < 65536, SSA_ERR_UNSUPPORTED, "decode: W too large");
  const int64_t vec = dtype == SSA_F32 ? 4 : 8;
  for (int s = 0; s < nstrides; ++s)
    SSA_REQUIRE(strides[s] % vec == 0, SSA_ERR_UNSUPPORTED,
                "decode: stride %d not a multiple of 16 bytes", s);
  return SSA_OK;
}

}  // namespace
}  // namespace ssa

extern "C" size_t ssa_decode_attend_workspace_size(int64_t B, int64_t Hq, int64_t nq, int64_t W,
                                                   int64_t d) {
  return (size_t)B * (size_t)Hq * (size_t)nq * (size_t)W * (size_t)(d + 2) * 4u;
}

extern "C" int ssa_decode_attend(const void* q, const void* k, const void* v, void* out, int dtype,
                                 int64_t B, int64_t Hq, int64_t Hkv, int64_t nq, int64_t cap,
                                 int64_t d, int64_t block, int64_t pos, const int64_t* strides,
                                 const int32_t* kv_num, const int32_t* kv_idx, int64_t W,
                                 float scale, void* workspace, size_t workspace_bytes,
                                 ssa_stream_t stream) {
  using namespace ssa;
  SSA_REQUIRE(q && k && v && out && strides && kv_num && kv_idx, SSA_ERR_INVALID,
              "decode_attend: NULL pointer argument");
  SSA_TRY(check_decode(dtype, B, Hq, Hkv, nq, cap, d, block, pos, W, strides, 12));
  SSA_REQUIRE(aligned16(k) && aligned16(v), SSA_ERR_UNSUPPORTED,
              "decode_attend: caches must be 16-byte aligned");
  const size_t need = ssa_decode_attend_workspace_size(B, Hq, nq, W, d);
  SSA_REQUIRE(workspace && workspace_bytes >= need, SSA_ERR_WORKSPACE,
              "decode_attend: workspace needs %zu bytes", need);
  SSA_REQUIRE(scale > 0.0f, SSA_ERR_INVALID, "decode_attend: scale must be > 0");
  DecodeParams p;
  p.q = static_cast<const char*>(q);
  p.k = static_cast<const char*>(k);
  p.v = static_cast<const char*>(v);
  p.o = static_cast<char*>(out);
  p.qsb = strides[0]; p.qsh = strides[1]; p.qsn = strides[2];
  p.ksb = strides[3]; p.ksh = strides[4]; p.ksn = strides[5];
  p.vsb = strides[6]; p.vsh = strides[7]; p.vsn = strides[8];
  p.osb = strides[9]; p.osh = strides[10]; p.osn = strides[11];
  p.B = B; p.Hq = Hq; p.G = Hq / Hkv; p.nq = nq; p.cap = cap; p.d = d; p.block = block;
  p.pos = pos;
  p.kv_num = kv_num; p.kv_idx = kv_idx; p.W = W;
  p.scale_log2 = scale * kLog2e;
  p.part = static_cast<float*>(workspace);
  p.lse = nullptr;
  return run_attend(dtype, p, static_cast<hipStream_t>(stream));
}

extern "C" size_t ssa_decode_step_workspace_size(int64_t B, int64_t Hq, int64_t cap, int64_t d,
                                                 int64_t block, int64_t W) {
  const int64_t nbk = block > 0 ? (cap + block - 1) / block : 0;
  size_t qf = (size_t)B * Hq * d * 4u;
  qf = (qf + 255) / 256 * 256;
  size_t keys = (size_t)B * Hq * nbk * 4u;
  keys = (keys + 255) / 256 * 256;
  return qf + keys + ssa_decode_attend_workspace_size(B, Hq, 1, W, d);
}

namespace {
// The body of ssa_decode_step and ssa_decode_step_static: `workspace` is the caller's buffer or
// the library's static scratch.
int decode_step_impl(const void* q, const void* k_new, const void* v_new, void* kcache,
                     void* vcache, float* mu, float* var, void* out, int dtype, int64_t B,
                     int64_t Hq, int64_t Hkv, int64_t cap, int64_t d, int64_t block, int64_t pos,
                     const int64_t* strides, int64_t top_c, float budget_frac, int64_t local,
                     float coef2, float scale, int32_t* kv_num, int32_t* kv_idx, int64_t W,
                     void* workspace, size_t workspace_bytes, ssa_stream_t stream) {
  using namespace ssa;
  SSA_REQUIRE(q && k_new && v_new && kcache && vcache && mu && var && out && strides && kv_num &&
                  kv_idx,
              SSA_ERR_INVALID, "decode_step: NULL pointer argument");
  SSA_TRY(check_decode(dtype, B, Hq, Hkv, 1, cap, d, block, pos, W, strides, 14));
  SSA_REQUIRE(aligned16(kcache) && aligned16(vcache), SSA_ERR_UNSUPPORTED,
              "decode_step: caches must be 16-byte aligned");
  SSA_REQUIRE(scale > 0.0f, SSA_ERR_INVALID, "decode_step: scale must be > 0");
  const size_t need = ssa_decode_step_workspace_size(B, Hq, cap, d, block, W);
  SSA_REQUIRE(workspace && workspace_bytes >= need, SSA_ERR_WORKSPACE,
              "decode_step: workspace needs %zu bytes", need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nbk = (cap + block - 1) / block;
  const int es = dtype_size(dtype);
  char* ws = static_cast<char*>(workspace);
  const size_t qf_bytes = ((size_t)B * Hq * d * 4u + 255) / 256 * 256;
  const size_t key_bytes = ((size_t)B * Hq * nbk * 4u + 255) / 256 * 256;
  float* qf = reinterpret_cast<float*>(ws);
  void* keys = ws + qf_bytes;
  float* part = reinterpret_cast<float*>(ws + qf_bytes + key_bytes);

  // 1. append the new token and convert the query rows (one launch) -- unless the step can fold
  //    the append into the attend launch: no block completes at pos (its summary would need the
  //    token in the cache first) and the query rows are contiguous, so the router reads them as
  //    they are
  const bool completes = (pos + 1) % block == 0;
  const bool fold = !completes && strides[1] == d && strides[0] == Hq * d;
  AppendStrides as;
  as.knb = strides[2]; as.knh = strides[3]; as.vnb = strides[4]; as.vnh = strides[5];
  as.kcb = strides[6]; as.kch = strides[7]; as.kcn = strides[8];
  as.vcb = strides[9]; as.vch = strides[10]; as.vcn = strides[11];
  const char* kn = static_cast<const char*>(k_new);
  const char* vn = static_cast<const char*>(v_new);
  char* kc = static_cast<char*>(kcache);
  char* vc = static_cast<char*>(vcache);
  const unsigned gr = (unsigned)(B * Hq);
  const char* qc = static_cast<const char*>(q);
  const int64_t G = Hq / Hkv;
  if (!fold) {
    switch (dtype) {
      case SSA_F32:
        decode_prep_kernel<SSA_F32><<<gr, 64, 0, st>>>(qc, qf, kn, vn, kc, vc, Hq, G, d, strides[0],
                                                        strides[1], pos, as);
        break;
      case SSA_F16:
        decode_prep_kernel<SSA_F16><<<gr, 64, 0, st>>>(qc, qf, kn, vn, kc, vc, Hq, G, d, strides[0],
                                                        strides[1], pos, as);
        break;
      default:
        decode_prep_kernel<SSA_BF16><<<gr, 64, 0, st>>>(qc, qf, kn, vn, kc, vc, Hq, G, d, strides[0],
                                                         strides[1], pos, as);
        break;
    }
    SSA_TRY(launch_status("decode_prep_kernel"));
  }

  // 2. a block completed at pos: its population summary becomes routable
  if ((pos + 1) % block == 0) {
    const int64_t c = pos / block;
    const char* blk = kc + c * block * as.kcn * es;
    SSA_TRY(launch_block_summary(blk, dtype, B, Hkv, block, d, as.kcb, as.kch, as.kcn, block, block,
                                 SSA_STATS_POP, mu, var, nullptr, nbk, c, st));
  }

  // 3. route the queries over the complete blocks
  SSA_TRY(route_impl(fold ? static_cast<const void*>(qc) : qf, fold ? dtype : SSA_F32, mu, var,
                     nullptr, B, Hq, Hkv, 1, nbk, d, SSA_ROUTE_QUERY, top_c, budget_frac, local,
                     coef2, 0.0f, pos, block, 1, kv_num, kv_idx, W, keys, key_bytes, st));

  // 4. attend
  DecodeParams p;
  p.q = qc;
  p.k = kc;
  p.v = vc;
  p.o = static_cast<char*>(out);
  p.qsb = strides[0]; p.qsh = strides[1]; p.qsn = 0;
  p.ksb = as.kcb; p.ksh = as.kch; p.ksn = as.kcn;
  p.vsb = as.vcb; p.vsh = as.vch; p.vsn = as.vcn;
  p.osb = strides[12]; p.osh = strides[13]; p.osn = 0;
  p.B = B; p.Hq = Hq; p.G = Hq / Hkv; p.nq = 1; p.cap = cap; p.d = d; p.block = block;
  p.pos = pos;
  p.kv_num = kv_num; p.kv_idx = kv_idx; p.W = W;
  p.scale_log2 = scale * kLog2e;
  p.part = part;
  p.lse = nullptr;
  if (fold) {
    p.fused_append = 1;
    p.k_new = kn;
    p.v_new = vn;
    p.knb = as.knb; p.knh = as.knh; p.vnb = as.vnb; p.vnh = as.vnh;
  }
  return run_attend(dtype, p, st);
}

// Scratch of ssa_decode_step_static: device memory the library itself holds, one copy on every
// device it runs on, for the process's lifetime. In host code `decode_scratch` names a host-side
// stand-in, not the device copy: kernels and copies use the address hipGetSymbolAddress returns
// for the device, looked up once per device (with that device current) and kept in
// g_scratch_ptr.
__device__ __align__(256) unsigned char decode_scratch[SSA_DECODE_STATIC_SCRATCH_BYTES];
constexpr int kMaxScratchDevices = 256;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

int scratch_of_device(hipStream_t st, void** ptr) {
  using namespace ssa;
  int dev = -1;
  if (st != nullptr) {
    SSA_TRY(hip_status(hipStreamGetDevice(st, &dev), "hipStreamGetDevice"));
  } else {
    SSA_TRY(hip_status(hipGetDevice(&dev), "hipGetDevice"));
  }
  SSA_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, SSA_ERR_UNSUPPORTED,
              "decode_step_static: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    SSA_TRY(hip_status(hipGetDevice(&cur), "hipGetDevice"));
    if (cur != dev) SSA_TRY(hip_status(hipSetDevice(dev), "hipSetDevice"));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(decode_scratch));
    if (cur != dev) SSA_TRY(hip_status(hipSetDevice(cur), "hipSetDevice"));
    SSA_TRY(hip_status(e, "hipGetSymbolAddress(decode_scratch)"));
    SSA_REQUIRE(p != nullptr, SSA_ERR_HIP, "decode_step_static: no scratch address on device %d",
                dev);
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return SSA_OK;
}
}  // namespace

extern "C" int ssa_decode_step(const void* q, const void* k_new, const void* v_new, void* kcache,
                               void* vcache, float* mu, float* var, void* out, int dtype,
                               int64_t B, int64_t Hq, int64_t Hkv, int64_t cap, int64_t d,
                               int64_t block, int64_t pos, const int64_t* strides, int64_t top_c,
                               float budget_frac, int64_t local, float coef2, float scale,
                               int32_t* kv_num, int32_t* kv_idx, int64_t W, void* workspace,
                               size_t workspace_bytes, ssa_stream_t stream) {
  return decode_step_impl(q, k_new, v_new, kcache, vcache, mu, var, out, dtype, B, Hq, Hkv, cap, d,
                          block, pos, strides, top_c, budget_frac, local, coef2, scale, kv_num,
                          kv_idx, W, workspace, workspace_bytes, stream);
}

extern "C" int ssa_decode_step_static(const void* q, const void* k_new, const void* v_new,
                                      void* kcache, void* vcache, float* mu, float* var,
                                      void* out, int dtype, int64_t B, int64_t Hq, int64_t Hkv,
                                      int64_t cap, int64_t d, int64_t block, int64_t pos,
                                      const int64_t* strides, int64_t top_c, float budget_frac,
                                      int64_t local, float coef2, float scale, int32_t* kv_num,
                                      int32_t* kv_idx, int64_t W, ssa_stream_t stream) {
  using namespace ssa;
  const size_t need = ssa_decode_step_workspace_size(B, Hq, cap, d, block, W);
  SSA_REQUIRE(need <= (size_t)SSA_DECODE_STATIC_SCRATCH_BYTES, SSA_ERR_WORKSPACE,
              "decode_step_static: this step needs %zu bytes of scratch, more than the static "
              "%zu (use ssa_decode_step with a workspace)",
              need, (size_t)SSA_DECODE_STATIC_SCRATCH_BYTES);
  void* ws = nullptr;
  SSA_TRY(scratch_of_device(static_cast<hipStream_t>(stream), &ws));
  return decode_step_impl(q, k_new, v_new, kcache, vcache, mu, var, out, dtype, B, Hq, Hkv, cap, d,
                          block, pos, strides, top_c, budget_frac, local, coef2, scale, kv_num,
                          kv_idx, W, ws, (size_t)SSA_DECODE_STATIC_SCRATCH_BYTES, stream);
}

extern "C" size_t ssa_masked_attn_workspace_size(int64_t B, int64_t Hq, int64_t n, int64_t W,
                                                 int64_t d, int64_t block) {
  if (ssa::masked_tiled_ok(d, block, n)) return ssa::masked_tiled_workspace(B, Hq, n, block);
  return ssa_decode_attend_workspace_size(B, Hq, n, W, d) + (size_t)B * Hq * n * 4u;
}

namespace {
int masked_params(ssa::DecodeParams& p, const void* q, const void* k, const void* v,
                  const void* out, int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t n,
                  int64_t d, int64_t block, const int64_t* strides, const int32_t* kv_num,
                  const int32_t* kv_idx, int64_t W, float scale) {
  using namespace ssa;
  SSA_REQUIRE(q && k && v && out && strides && kv_num && kv_idx, SSA_ERR_INVALID,
              "masked_attn: NULL pointer argument");
  SSA_TRY(check_decode(dtype, B, Hq, Hkv, n, n, d, block, 0, W, strides, 12));
  SSA_REQUIRE(aligned16(k) && aligned16(v), SSA_ERR_UNSUPPORTED,
              "masked_attn: k and v must be 16-byte aligned");
  SSA_REQUIRE(scale > 0.0f, SSA_ERR_INVALID, "masked_attn: scale must be > 0");
  p.q = static_cast<const char*>(q);
  p.k = static_cast<const char*>(k);
  p.v = static_cast<const char*>(v);
  p.o = static_cast<char*>(const_cast<void*>(out));
  p.qsb = strides[0]; p.qsh = strides[1]; p.qsn = strides[2];
  p.ksb = strides[3]; p.ksh = strides[4]; p.ksn = strides[5];
  p.vsb = strides[6]; p.vsh = strides[7]; p.vsn = strides[8];
  p.osb = strides[9]; p.osh = strides[10]; p.osn = strides[11];
  p.B = B; p.Hq = Hq; p.G = Hq / Hkv; p.nq = n; p.cap = n; p.d = d; p.block = block;
  p.pos = 0;
  p.kv_num = kv_num; p.kv_idx = kv_idx; p.W = W;
  p.scale_log2 = scale * kLog2e;
  return SSA_OK;
}
}  // namespace

extern "C" int ssa_masked_attn_fwd(const void* q, const void* k, const void* v, void* out,
                                   float* lse, int dtype, int64_t B, int64_t Hq, int64_t Hkv,
                                   int64_t n, int64_t d, int64_t block, const int64_t* strides,
                                   const int32_t* kv_num, const int32_t* kv_idx, int64_t W,
                                   float scale, void* workspace, size_t workspace_bytes,
                                   ssa_stream_t stream) {
  using namespace ssa;
  DecodeParams p;
  SSA_TRY(masked_params(p, q, k, v, out, dtype, B, Hq, Hkv, n, d, block, strides, kv_num, kv_idx,
                        W, scale));
  SSA_REQUIRE(lse != nullptr, SSA_ERR_INVALID, "masked_attn_fwd: lse is NULL");
  if (masked_tiled_ok(d, block, n))
    return masked_tiled_fwd(q, k, v, out, lse, dtype, B, Hq, Hkv, n, block, strides, kv_num,
                            kv_idx, W, scale, workspace, workspace_bytes,
                            static_cast<hipStream_t>(stream));
  const size_t need = ssa_decode_attend_workspace_size(B, Hq, n, W, d);
  SSA_REQUIRE(workspace && workspace_bytes >= need, SSA_ERR_WORKSPACE,
              "masked_attn_fwd: workspace needs %zu bytes", need);
  p.part = static_cast<float*>(workspace);
  p.lse = lse;
  return run_attend(dtype, p, static_cast<hipStream_t>(stream));
}

extern "C" int ssa_masked_attn_bwd(const void* q, const void* k, const void* v, const void* out,
                                   const void* dout, const float* lse, void* dq, void* dk,
                                   void* dv, int dtype, int grad_dtype, int flags, int64_t B,
                                   int64_t Hq, int64_t Hkv,
                                   int64_t n, int64_t d, int64_t block, const int64_t* strides,
                                   const int32_t* kv_num, const int32_t* kv_idx, int64_t W,
                                   float scale, void* workspace, size_t workspace_bytes,
                                   ssa_stream_t stream) {
  using namespace ssa;
  BwdParams bp;
  SSA_TRY(masked_params(bp.f, q, k, v, out, dtype, B, Hq, Hkv, n, d, block, strides, kv_num,
                        kv_idx, W, scale));
  SSA_REQUIRE(dout && lse && dq && dk && dv, SSA_ERR_INVALID, "masked_attn_bwd: NULL gradient");
  SSA_REQUIRE((flags & ~SSA_MASKED_MASKS_READY) == 0, SSA_ERR_INVALID,
              "masked_attn_bwd: unknown flags");
  if (masked_tiled_ok(d, block, n))
    return masked_tiled_bwd(q, k, v, out, dout, lse, dq, dk, dv, dtype, grad_dtype, flags, B, Hq,
                            Hkv, n, block,
                            strides, kv_num, kv_idx, W, scale, workspace, workspace_bytes,
                            static_cast<hipStream_t>(stream));
  SSA_REQUIRE(grad_dtype == SSA_F32, SSA_ERR_UNSUPPORTED,
              "masked_attn_bwd: the per-row path (d != 64) accumulates fp32 gradients only");
  const size_t need = (size_t)B * Hq * n * 4u;
  SSA_REQUIRE(workspace && workspace_bytes >= need, SSA_ERR_WORKSPACE,
              "masked_attn_bwd: workspace needs %zu bytes", need);
  bp.f.part = nullptr;
  bp.f.lse = nullptr;
  bp.dout = static_cast<const char*>(dout);
  bp.lse = lse;
  bp.delta = static_cast<const float*>(workspace);
  bp.dq = static_cast<float*>(dq);
  bp.dk = static_cast<float*>(dk);
  bp.dv = static_cast<float*>(dv);
  bp.Hkv = Hkv;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t rows = B * Hq * n;
  SSA_REQUIRE(rows * W < (1ll << 31), SSA_ERR_UNSUPPORTED, "masked_attn_bwd: grid too large");
  const int64_t nq_el = rows * d, nk_el = B * Hkv * n * d;
  zero_f32_kernel<<<(unsigned)((nq_el + 255) / 256 < 4096 ? (nq_el + 255) / 256 : 4096), 256, 0, st>>>(bp.dq, nq_el);
  zero_f32_kernel<<<(unsigned)((nk_el + 255) / 256 < 4096 ? (nk_el + 255) / 256 : 4096), 256, 0, st>>>(bp.dk, nk_el);
  zero_f32_kernel<<<(unsigned)((nk_el + 255) / 256 < 4096 ? (nk_el + 255) / 256 : 4096), 256, 0, st>>>(bp.dv, nk_el);
  SSA_TRY(launch_status("zero_f32_kernel"));
  const unsigned g1 = (unsigned)rows, g2 = (unsigned)(rows * W);
  switch (dtype) {
    case SSA_F32:
      masked_delta_kernel<SSA_F32><<<g1, 64, 0, st>>>(bp);
      masked_bwd_kernel<SSA_F32><<<g2, 64, 0, st>>>(bp);
      break;
    case SSA_F16:
      masked_delta_kernel<SSA_F16><<<g1, 64, 0, st>>>(bp);
      masked_bwd_kernel<SSA_F16><<<g2, 64, 0, st>>>(bp);
      break;
    default:
      masked_delta_kernel<SSA_BF16><<<g1, 64, 0, st>>>(bp);
      masked_bwd_kernel<SSA_BF16><<<g2, 64, 0, st>>>(bp);
      break;
  }
  return launch_status("masked_bwd_kernel");
}
