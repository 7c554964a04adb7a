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

#include <type_traits>

#include <mutex>

#include "common.h"
#include "select.h"

namespace ssa {

typedef float f32x2 __attribute__((ext_vector_type(2)));

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
  for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, lane_xor(x, off));
  return x;
}
__device__ inline float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += lane_xor(x, off);
  return x;
}


// Stores of a partial result: plain, or (FUSED) relaxed agent-scope atomic stores, which are
// performed at the device's coherence point, so a workgroup on another XCD can read them with
// agent-scope loads once the writer's stores have completed.
template <bool FUSED>
__device__ inline void put_part(float* p, float x) {
  if constexpr (FUSED) __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = x;
}

// Partial softmax attention of query row (b, h, r) over key block c (keys [kofs, kofs + kcnt)
// of the block; kcnt < 0: the whole block): (m, l, o[d]) into part, computed by one wave (qs,
// ps: that wave's LDS); a range without keys at or before pos stores the empty partial
// (m = -inf, l = 0, o = 0). FUSED: the wave is one of several in its workgroup (wave-local LDS
// ordering); COH: the partial is stored with put_part<true> (else plain stores, e.g. into LDS).
template <int DT, bool FUSED = false, int KPRE = 16, bool COH = FUSED>
__device__ inline void block_partial(const DecodeParams& p, float* part, float* qs, float* ps,
                                     int64_t b, int64_t h, int64_t kvh, int64_t r, int64_t pos,
                                     int64_t c, int64_t kofs = 0, int64_t kcnt = -1) {
  const int lane = threadIdx.x & 63;
  auto lds_sync = []() {
    if constexpr (FUSED) wave_lds_sync();
    else __syncthreads();
  };
  const int d = (int)p.d;
  const int64_t key0 = c * p.block + kofs;
  int64_t key1 = c * p.block + p.block;
  if (kcnt >= 0 && key0 + kcnt < key1) key1 = key0 + kcnt;
  if (key1 > pos + 1) key1 = pos + 1;
  if (key1 > p.cap) key1 = p.cap;
  const int nk = (int)(key1 - key0);
  if (nk <= 0) {
    if (lane == 0) {
      put_part<COH>(&part[0], -INFINITY);
      put_part<COH>(&part[1], 0.0f);
    }
    for (int e = lane; e < d; e += 64) put_part<COH>(&part[2 + e], 0.0f);
    return;
  }
  // PV lane layout (16-bit): key group kg = lane / 8, 16-byte chunk ch = lane % 8 of the V row.
  // Ranges of at most 8 * kPre keys with d <= 64 load their V rows up front, in flight while the
  // scores are computed.
  constexpr int kPre = KPRE;
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
  const char* qb = p.q;
  const int64_t qoff = b * p.qsb + h * p.qsh + r * p.qsn;
  // FUSED: the query elements are loaded first and staged after the K / V loads are issued, so
  // that staging waits for the query only
  float qx[2] = {0.0f, 0.0f};
  if constexpr (FUSED) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
      if (lane + 64 * u < d) qx[u] = load_elem<DT>(qb, qoff + lane + 64 * u);
  }
  u32x4 vpre[kPre];
  if constexpr (DT != SSA_F32) {
    if (pre) {
      if constexpr (FUSED) {  // unconditional loads (past the block: its last key, unused)
        const int chc = ch * 8 < d ? ch : d / 8 - 1;
#pragma unroll
        for (int t = 0; t < kPre; ++t) {
          const int kk = kg + 8 * t < nk ? kg + 8 * t : nk - 1;
          vpre[t] = *reinterpret_cast<const u32x4*>(
              reinterpret_cast<const unsigned short*>(vrow(key0 + kk)) + chc * 8);
        }
      } else {
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
  }

  // FUSED (one wave of several per CU: registers to spare): the K rows of such a block are
  // loaded with the V rows and in their layout (lane: chunk ch of key kg + 8t; a load instruction
  // reads 8 whole 128-byte rows), before the query row is staged
  u32x4 kpre[kPre];
  if constexpr (FUSED && DT != SSA_F32) {
    if (pre) {
      const int chc = ch * 8 < d ? ch : d / 8 - 1;
#pragma unroll
      for (int t = 0; t < kPre; ++t) {
        const int kk = kg + 8 * t < nk ? kg + 8 * t : nk - 1;
        kpre[t] = *reinterpret_cast<const u32x4*>(
            reinterpret_cast<const unsigned short*>(krow(key0 + kk)) + chc * 8);
      }
    }
  }

  if constexpr (FUSED) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
      if (lane + 64 * u < d) qs[lane + 64 * u] = qx[u];
  } else {
    for (int e = lane; e < d; e += 64) qs[e] = load_elem<DT>(qb, qoff + e);
  }
  lds_sync();

  float mloc = -INFINITY;
  // FUSED 16-bit ranges in the K / V layout above: lane (kg, ch) forms the 8-dim partial dots of
  // its kPre keys kg + 8t, and three halving exchanges over the 8 lanes of its key group (xor 4,
  // 2, 1) leave it the full dots of keys kg + 8t for t = V ch + i, i < V = kPre / 8; their exps
  // go to ps
  bool done = false;
  float lsum = 0.0f;
  if constexpr (FUSED && DT != SSA_F32) {
    if (pre) {
      float qv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) qv[u] = ch * 8 < d ? qs[ch * 8 + u] : 0.0f;
      float sc[kPre];
#pragma unroll
      for (int t = 0; t < kPre; ++t) {
        float kv[8];
        unpack8(kpre[t], kv, DT == SSA_BF16);
        float a = 0.0f;
#pragma unroll
        for (int u = 0; u < 8; ++u) a = fmaf(qv[u], kv[u], a);
        sc[t] = a;
      }
      constexpr int V = kPre / 8;  // full dots per lane at the end
#pragma unroll
      for (int w = 4; w >= 1; w >>= 1) {  // keep the half of the values whose t bit = ch bit w
        const bool hi = (ch & w) != 0;
#pragma unroll
        for (int i = 0; i < V * w; ++i) {
          const float keep = hi ? sc[i + V * w] : sc[i];
          const float send = hi ? sc[i] : sc[i + V * w];
          sc[i] = keep + lane_xor(send, w);
        }
      }
      float sl[V];
#pragma unroll
      for (int i = 0; i < V; ++i) {
        sl[i] = sc[i] * p.scale_log2;
        if (kg + 8 * (V * ch + i) < nk) mloc = fmaxf(mloc, sl[i]);
      }
      const float m = wave_max(mloc);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const int kk = kg + 8 * (V * ch + i);
        const float pk = kk < nk ? exp2f(sl[i] - m) : 0.0f;
        if (kk < nk) ps[kk] = pk;
        lsum += pk;
      }
      mloc = m;
      done = true;
    }
  }
  for (int kk = lane; kk < nk && !done; kk += 64) {
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
  const float m = done ? mloc : wave_max(mloc);
  lds_sync();
  float lloc = lsum;
  for (int kk = lane; kk < nk && !done; kk += 64) {
    const float pk = exp2f(ps[kk] - m);
    ps[kk] = pk;
    lloc += pk;
  }
  const float l = wave_sum(lloc);
  lds_sync();
  if constexpr (DT == SSA_F32) {
    for (int e = lane; e < d; e += 64) {
      float acc = 0.0f;
      for (int kk = 0; kk < nk; ++kk)
        acc = fmaf(ps[kk], load_elem<DT>(vrow(key0 + kk), e), acc);
      put_part<COH>(&part[2 + e], acc);
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
      x += lane_xor(x, 8);
      x += lane_xor(x, 16);
      x += lane_xor(x, 32);
      acc[t] = x;
    }
    if (kg == 0 && ch * 8 < d)
#pragma unroll
      for (int t = 0; t < 8; ++t) put_part<COH>(&part[2 + ch * 8 + t], acc[t]);
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
        x += lane_xor(x, 8);
        x += lane_xor(x, 16);
        x += lane_xor(x, 32);
        acc[t] = x;
      }
      if (kg == 0 && on)
#pragma unroll
        for (int t = 0; t < 8; ++t) put_part<COH>(&part[2 + e0 + ch * 8 + t], acc[t]);
    }
  }
  if (lane == 0) {
    put_part<COH>(&part[0], m);
    put_part<COH>(&part[1], l);
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
// Fused decode step: two launches per step.
// decode_route_kernel<DT, DQ, NW>: grid (ceil(ncand / (16 NW)), B*Hkv), NW waves of 16
//   candidates. A workgroup scores a chunk of 16 NW candidate blocks (64, 128 or 256: the
//   smallest whose lists the merge below can hold, spreading the scoring over the most CUs) of one
//   key head for all G query rows of that head -- exact: fp64 sums over the head
//   dim from the fp32 operands (q, fl32(q*q) broadcast from LDS), the fp32 score assembled as
//   route_score_kernel does -- and keeps each row's chunk top-K by (key desc, block asc) with the
//   chunk's K-th key. A chunk's top-K holds every candidate of the chunk that can be in the
//   row's top-K (one it drops has K candidates of its chunk ranked above it). Workgroup (0, 0)
//   also clears the arrival counters of the attend launch.
// decode_attend_fused_kernel: grid (ceil(W / 4), B*Hq), 8 waves. Every workgroup of a row merges
//   the row's chunk lists: T_lb, a lower bound of the row's K-th key from the chunks' sorted
//   lists, keeps only entries >= T_lb (every member of the top-K) in LDS; one wave finds the
//   K-th key T, takes keys > T and ties at T by lowest block index, and sorts the taken blocks
//   below the local range ascending, followed by the own block and its `local` predecessors (a
//   block-wide radix search and bitmaps above 512 survivors). Waves w and w + 4 then attend the
//   two halves of slot 4*blockIdx.x + w of the list (block_partial) and store their partials
//   with agent-scope stores; after each wave's stores have completed, an agent-scope arrival
//   counter per row picks the row's last workgroup, which reads the partials with agent-scope
//   loads, combines them, and writes the output row and (kv_num, kv_idx).
// ---------------------------------------------------------------------------------------------
constexpr int kDChunk = 256;     // largest chunk of candidate blocks per route workgroup
constexpr int kDTop = 64;        // largest keep of the fused step
constexpr int kDMaxRows = 16;    // query rows per key head (G)
constexpr int kDMaxD = 128;      // head dim
constexpr int kDMaxBlock = 512;  // keys per block
constexpr int kDSurv = 8192;     // merged entries held in LDS (nchunk * K <= kDSurv)
constexpr int kDMaxChunks = 128; // chunks whose r-th keys bound the row's K-th key
constexpr int kDBitWords = 1024; // bitmap words: blocks <= own < 32768
constexpr int kDMaxW = 128;

struct FusedStep {
  const char* q;  // (B, Hq, d) query rows of the step
  int64_t qsb, qsh;
  const float* mu;
  const float* var;
  int64_t B, Hq, Hkv, G, d, nbk, ncand, K, local, pos, block, W;
  float coef2;
  int nchunk, ngroups;
  unsigned int* arrive;  // (B*Hq) arrival counters
  unsigned int* ckth;    // (B*Hq, nchunk): entries the chunk kept (min(K, its candidates))
  unsigned int* ckey;    // (B*Hq, nchunk, kDTop): the chunk's kept keys, best first, then 0
  unsigned int* cidx;
  int32_t* kv_num;       // (B*Hq)
  int32_t* kv_idx;       // (B*Hq, W)
};

// One route workgroup's work: chunk `chunk` of the candidate blocks of key head bk.
// NW waves score (16 candidates each); all NWT >= NW waves take the rows' selections (one row
// per wave and round).
template <int DT, int DQ, int NW, int NWT = NW>
__device__ inline void route_chunk(const FusedStep& f, int64_t chunk, int64_t bk_) {
  static_assert(NWT >= NW, "selection waves include the scoring waves");
  constexpr int NT = NWT * 64, CH = NW * 16;  // threads, candidates per workgroup
  constexpr int NQ = kDMaxRows * kDMaxD / NT;  // query elements staged per thread
  __shared__ double qd[kDMaxRows][kDMaxD + 1];   // q as fp64 (rows padded: conflict-free reads)
  __shared__ double q2d[kDMaxRows][kDMaxD + 1];  // fl32(q*q) as fp64
  __shared__ unsigned int skey[kDMaxRows][CH];
  __shared__ unsigned int sbuf[NWT][2][64];      // per wave: a row's kept entries
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t bk = bk_, b = bk / f.Hkv, kvh = bk % f.Hkv;
  const int64_t c0 = chunk * CH;
  const int G = (int)f.G;
  constexpr int d = 4 * DQ;
  // the query element of this thread first (row tid / d, dim tid % d; 16 * d <= 2048 elements),
  // then the candidate operands, so that staging the query waits for the query load only
  float qx[NQ];
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    const int idx = tid + NT * u, r = idx / d, k = idx % d;
    qx[u] = idx < kDMaxRows * d && r < G ? load_elem<DT>(f.q, b * f.qsb + (kvh * G + r) * f.qsh + k)
                                          : 0.0f;
  }
  // Scores on v_mfma_f64_16x16x4_f64 (lane l supplies A[l%16][l/16] and B[l/16][l%16];
  // accumulator j of lane l is C[4j + l/16][l%16]): A = the G query rows (padded to 16), B = 16
  // candidates per wave, the 4-wide k of step s being head dims g*DQ + s of lane group g = l/16:
  // lane l holds dims [g*DQ, +DQ) of candidate l%16 in registers, loaded up front as 16-byte
  // vectors (a candidate past the last one reads the last one; its score is discarded).
  // E1 = <q, mu> and E2 = <q*q, var> accumulate in fp64 in two chains.
  const int g = lane >> 4, n16 = lane & 15;
  const int wsc = wv < NW ? wv : NW - 1;  // (waves past the scoring ones load wave NW-1's operands)
  const int64_t c = c0 + wsc * 16 + n16;
  const bool cv = c < f.ncand;
  const int64_t cl = cv ? c : (f.ncand > 0 ? f.ncand - 1 : 0);
  float mm[DQ], vv[DQ];
  {
    const float* pm = f.mu + (bk * f.nbk + cl) * d + g * DQ;
    const float* pv = f.var + (bk * f.nbk + cl) * d + g * DQ;
#pragma unroll
    for (int e = 0; e < DQ; e += 4) {
      const f32x4 m4 = *reinterpret_cast<const f32x4*>(pm + e);
      const f32x4 v4 = *reinterpret_cast<const f32x4*>(pv + e);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        mm[e + t] = m4[t];
        vv[e + t] = v4[t];
      }
    }
  }
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    const int idx = tid + NT * u, r = idx / d, k = idx % d;
    if (idx < kDMaxRows * d) {
      qd[r][k] = (double)qx[u];
      q2d[r][k] = (double)(qx[u] * qx[u]);  // rounded to fp32 like the reference's product
    }
  }
  __syncthreads();
  typedef double f64x4 __attribute__((ext_vector_type(4)));
  f64x4 a1 = {0.0, 0.0, 0.0, 0.0}, a2 = {0.0, 0.0, 0.0, 0.0};
  if (NWT == NW || wv < NW) {  // wave-uniform: the selection-only waves skip the scoring
#pragma unroll
    for (int s = 0; s < DQ; ++s) {
      a1 = __builtin_amdgcn_mfma_f64_16x16x4f64(qd[n16][g * DQ + s], (double)mm[s], a1, 0, 0, 0);
      a2 = __builtin_amdgcn_mfma_f64_16x16x4f64(q2d[n16][g * DQ + s], (double)vv[s], a2, 0, 0, 0);
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 4 * j + g;
    if (r < G && wv < NW)
      skey[r][wv * 16 + n16] =
          cv ? score_key(__fadd_rn((float)a1[j], __fmul_rn(f.coef2, (float)a2[j]))) : 0u;
  }
  __syncthreads();
  const int64_t nvalid = f.ncand - c0 < CH ? f.ncand - c0 : CH;
  const unsigned long long lt = (1ull << lane) - 1ull;
  constexpr int J = CH / 64;
  for (int r = wv; r < G; r += NWT) {
    const int64_t cb = (b * f.Hq + kvh * G + r) * f.nchunk + chunk;
    unsigned int key[J], cm = 0u;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      key[j] = skey[r][lane + 64 * j];
      cm |= (lane + 64 * j < nvalid ? 1u : 0u) << j;
    }
    const unsigned int selm = wave_select_top<J>(key, cm, f.K, nvalid);
    // the kept entries (at most K <= 64) to one lane each, sorted, then stored: entry j of a
    // chunk list is its (j+1)-th best, key 0 past its kept entries
    int at = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const bool take = (selm >> j) & 1u;
      const unsigned long long bt = __ballot(take);
      if (take) {
        const int slot = at + (int)__popcll(bt & lt);
        sbuf[wv][0][slot] = key[j];
        sbuf[wv][1][slot] = (unsigned int)(c0 + lane + 64 * j);
      }
      at += (int)__popcll(bt);
    }
    wave_lds_sync();
    unsigned int sk = lane < at ? sbuf[wv][0][lane] : 0u, sb = lane < at ? sbuf[wv][1][lane] : 0u;
    wave_lds_sync();
    wave_sort_desc(sk, sb);
    f.ckey[cb * kDTop + lane] = sk;
    f.cidx[cb * kDTop + lane] = sb;
    if (lane == 0) f.ckth[cb] = (unsigned int)at;  // entries kept
  }
}

template <int DT, int DQ, int NW, int NWT = NW>
__global__ __launch_bounds__(NWT * 64) void decode_route_kernel(FusedStep f) {
  if (blockIdx.x == 0 && blockIdx.y == 0)
    for (int64_t t = threadIdx.x; t < f.B * f.Hq; t += NWT * 64)
      __hip_atomic_store(&f.arrive[t], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  route_chunk<DT, DQ, NW, NWT>(f, blockIdx.x, blockIdx.y);
}

template <int NWA>
__device__ inline unsigned int block_sum_u32(unsigned int x, unsigned int* red) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += lane_xor(x, off);
  __syncthreads();
  if (lane == 0) red[wv] = x;
  __syncthreads();
  unsigned int t = 0u;
#pragma unroll
  for (int w = 0; w < NWA; ++w) t += red[w];
  return t;
}

// Bitonic sort of one value per lane across the wave, ascending: lane j ends with the (j+1)-th
// smallest.
__device__ inline unsigned int wave_sort_asc(unsigned int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
    for (int j = k >> 1; j >= 1; j >>= 1) {
      const unsigned int o = lane_xor(v, j);
      // the lower lane of an ascending pair keeps the smaller value, and so on
      const bool keep_min = ((lane & j) == 0) == ((lane & k) == 0);
      v = keep_min ? (o < v ? o : v) : (o > v ? o : v);
    }
  return v;
}

// One attend workgroup's work (NWA waves): group `group` of the selected slots of query row
// `row` (b*Hq + h), NWA / HALVES slots, each attended by HALVES waves (a wave per 1/HALVES of
// the block's keys, each storing a partial of its own).
template <int DT, int NWA, int HALVES>
__device__ inline void attend_group(const FusedStep& f, const DecodeParams& p, int64_t row,
                                    int64_t group) {
  constexpr int NT = NWA * 64, SPW = NWA / HALVES;
  __shared__ unsigned int skey[kDSurv], sidx[kDSurv];
  __shared__ unsigned int sel[kDBitWords], tie[kDBitWords];
  __shared__ int32_t list[kDMaxW];
  __shared__ __attribute__((aligned(16))) float qs[NWA][kDMaxD];
  __shared__ float ps[NWA][kDMaxBlock];
  __shared__ float wgt[kDMaxW];
  __shared__ float wpart[NWA][kDMaxD + 2];  // the waves' partials, combined into the group's
  __shared__ unsigned int red[NWA], rand_[4], hist[256];  // (hist: also reduction scratch)
  __shared__ unsigned int sh_n, sh_last, sh_ovf;
  __shared__ int wsum[NWA];
  __shared__ unsigned int rth[7][kDMaxChunks];  // r-th key of every chunk, r = 1, 2, 4, ..., 64
  __shared__ unsigned int rbound[8];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t b = row / f.Hq, h = row % f.Hq, kvh = h / f.G;
  const int64_t pos = f.pos;
  const int64_t own = pos / f.block;
  const int nwords = (int)((own + 32) / 32);  // bits of blocks 0..own
  const unsigned long long lt = (1ull << lane) - 1ull;

  // ---- merge the row's chunk lists ----
  // T_lb, a lower bound of the row's K-th key from the sorted chunk lists: for r = 1, 2, 4, ...,
  // the ceil(K / r)-th largest of the chunks' r-th keys (that many chunks hold r keys at or above
  // it: at least K entries reach it), the largest of these bounds. Real keys are nonzero; key 0
  // past a chunk's kept entries. A first pass loads the first P = 16 entries of every chunk list
  // (bound from r <= 16): when no chunk's 16th entry reaches that bound, every entry >= T_lb is
  // among them; otherwise a second pass loads the whole lists (bound from r <= 64). A pass's
  // thread (wave w, lane l) holds entry l % P of chunk (w + NWA u) 64/P + l / P in register u.
  for (int w = tid; w < nwords; w += NT) {
    sel[w] = 0u;
    tie[w] = 0u;
  }
  if (tid == 0) {
    sh_n = 0u;
    sh_ovf = 0u;
  }
  const int64_t K = f.K;
  const int nch = f.nchunk;
  const int ne = nch * kDTop;
  constexpr int SEG = kDSurv / NWA;
  auto merge_pass = [&](auto pc) -> bool {
    constexpr int P = decltype(pc)::value, CPR = 64 / P;
    constexpr int KR = (kDSurv / kDTop + NWA * CPR - 1) / (NWA * CPR);
    constexpr int LG = P == 64 ? 6 : P == 32 ? 5 : P == 16 ? 4 : P == 8 ? 3 : -1;
    static_assert(LG >= 0, "prefix length");
    const int pos = lane % P;
    unsigned int kk[KR], ci[KR];
#pragma unroll
    for (int u = 0; u < KR; ++u) {
      const int c = (wv + NWA * u) * CPR + lane / P;
      const int64_t i = row * ne + (c < nch ? c * kDTop + pos : 0);
      kk[u] = f.ckey[i];
      ci[u] = f.cidx[i];
      if (c >= nch) kk[u] = 0u;
    }
    // the r-th keys to LDS (chunks past the lists: 0)
    const int lgp = __popc(pos + 1) == 1 ? 31 - __clz(pos + 1) : -1;  // pos = r - 1, r = 2^lgp
#pragma unroll
    for (int u = 0; u < KR; ++u) {
      const int c = (wv + NWA * u) * CPR + lane / P;
      if (c < kDMaxChunks && lgp >= 0) rth[lgp][c] = kk[u];
    }
    __syncthreads();
    for (int lg = wv; lg <= LG; lg += NWA) {
      const unsigned int r = 1u << lg;
      const int64_t m = K > 0 ? (K + r - 1) / r : 0;  // chunks needed
      unsigned int v[kDMaxChunks / 64];
#pragma unroll
      for (int j = 0; j < kDMaxChunks / 64; ++j) v[j] = rth[lg][lane + 64 * j];
      unsigned int bnd = 0u;
      if (m > 0 && m <= kDMaxChunks)  // 0 when fewer than m chunks hold r keys
        bnd = wave_kth_key<kDMaxChunks / 64>(v, m);
      if (lane == 0) rbound[lg] = bnd;
    }
    __syncthreads();
    unsigned int tlb = 0u;
#pragma unroll
    for (int lg = 0; lg <= LG; ++lg) tlb = rbound[lg] > tlb ? rbound[lg] : tlb;
    const unsigned int floor_ = tlb > 1u ? tlb : 1u;
    if constexpr (P < kDTop) {  // a chunk whose P-th entry reaches the bound may hold more
      bool ovf = false;
#pragma unroll
      for (int u = 0; u < KR; ++u) ovf = ovf || (pos == P - 1 && kk[u] >= floor_);
      if (__ballot(ovf) != 0ull && lane == 0) sh_ovf = 1u;
      __syncthreads();
      if (sh_ovf) return true;  // uniform
    }
    // Survivors (keys >= T_lb) go to their wave's own LDS segment [SEG w, SEG w + n_w) in ballot
    // order -- no atomics; survivor i of the row is entry phys(i) of the concatenated segments.
    int at = 0;
#pragma unroll
    for (int u = 0; u < KR; ++u) {
      const bool take = kk[u] >= floor_;
      const unsigned long long bt = __ballot(take);
      if (take) {
        const int sl = wv * SEG + at + (int)__popcll(bt & lt);
        skey[sl] = kk[u];
        sidx[sl] = ci[u];
      }
      at += (int)__popcll(bt);
    }
    if (lane == 0) wsum[wv] = at;
    __syncthreads();
    return false;
  };
  if (merge_pass(std::integral_constant<int, 16>{})) merge_pass(std::integral_constant<int, 64>{});
  int pre[NWA];  // survivors of the waves before wave w
  int n = 0;
#pragma unroll
  for (int w = 0; w < NWA; ++w) {
    pre[w] = n;
    n += wsum[w];
  }
  auto phys = [&](int i) -> int {  // survivor i -> its LDS entry
    int w = 0;
#pragma unroll
    for (int v = 1; v < NWA; ++v) w += i >= pre[v] ? 1 : 0;
    int base = 0;
#pragma unroll
    for (int v = 0; v < NWA; ++v) base = v == w ? pre[v] : base;
    return w * SEG + (i - base);
  };
  // one wave (J survivors per lane): K-th key, ties by lowest block, then the ascending list of
  // the taken blocks, own block and local predecessors -- no workgroup barrier until the list is
  // done
  auto one_wave = [&](auto jc) {
    constexpr int J = decltype(jc)::value;
    if (wv == 0) {
      unsigned int key[J], blk[J];
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int i = lane + 64 * j;
        key[j] = i < n ? skey[phys(i)] : 0u;
        blk[j] = i < n ? sidx[phys(i)] : 0u;
      }
      unsigned int takem = 0u;
      if (K >= n) {
#pragma unroll
        for (int j = 0; j < J; ++j) takem |= (lane + 64 * j < n ? 1u : 0u) << j;
      } else if (K > 0) {
        const unsigned int T = wave_kth_key<J>(key, K);
        int above = 0, nt = 0;
#pragma unroll
        for (int j = 0; j < J; ++j) {
          above += (int)__popcll(__ballot(key[j] > T));
          nt += (int)__popcll(__ballot(key[j] == T));
        }
        const int need = (int)K - above;  // ties at T to take, lowest block first
        unsigned int tk[J];
#pragma unroll
        for (int j = 0; j < J; ++j) tk[j] = key[j] == T ? ~blk[j] : 0u;  // larger = lower block
        const unsigned int T2 = need < nt ? wave_kth_key<J>(tk, need) : 1u;
#pragma unroll
        for (int j = 0; j < J; ++j)
          takem |= (key[j] > T || (key[j] == T && tk[j] >= T2) ? 1u : 0u) << j;
      }
      // The list: the taken blocks below the local range [lo, hi] (at most K <= 64 of them,
      // distinct) sorted ascending in one register, then the local range (own block and its
      // predecessors, the largest block indices of the row)
      int64_t lo = own - f.local;
      if (lo < 0) lo = 0;
      const int64_t hi = own < f.nbk - 1 ? own : f.nbk - 1;
      int at = 0;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const bool t = ((takem >> j) & 1u) && (int64_t)blk[j] < lo;
        const unsigned long long bt = __ballot(t);
        if (t) hist[at + (int)__popcll(bt & lt)] = blk[j];
        at += (int)__popcll(bt);
      }
      wave_lds_sync();
      const unsigned int v = wave_sort_asc(lane < at ? hist[lane] : 0xffffffffu);
      if (lane < at && lane < f.W) list[lane] = (int32_t)v;
      for (int64_t c = lane; c <= hi - lo; c += 64)
        if (at + c < f.W) list[at + c] = (int32_t)(lo + c);
      if (lane == 0) sh_n = (unsigned int)(at + (hi - lo + 1));
    }
    __syncthreads();
  };
  if (n <= 128) {
    one_wave(std::integral_constant<int, 2>{});
  } else if (n <= 256) {
    one_wave(std::integral_constant<int, 4>{});
  } else if (n <= 512) {
    one_wave(std::integral_constant<int, 8>{});
  } else {
    // more survivors: workgroup-wide radix search for the K-th key and bitmaps
    unsigned int T = 0u;
    if (K > 0) {
      unsigned int prefix = 0u, pmask = 0u, kk_ = (unsigned int)K;
      for (int shift = 24; shift >= 0; shift -= 8) {
        if (tid < 256) hist[tid] = 0u;
        __syncthreads();
        for (int i = tid; i < n; i += NT) {
          const unsigned int k = skey[phys(i)];
          if ((k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid < 64) {
          unsigned int v[4], t = 0u;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            v[j] = hist[4 * tid + j];
            t += v[j];
          }
          unsigned int suf = t;  // inclusive suffix over lanes >= tid
#pragma unroll
          for (int off = 1; off < 64; off <<= 1) {
            const unsigned int o = __shfl_down(suf, off, 64);
            if (tid + off < 64) suf += o;
          }
          unsigned int above = suf - t;  // keys in the bins of higher lanes
#pragma unroll
          for (int j = 3; j >= 0; --j) {
            if (above < kk_ && kk_ <= above + v[j]) {
              rand_[0] = (unsigned int)(4 * tid + j);
              rand_[1] = above;
              rand_[2] = kk_ == above + v[j] ? 1u : 0u;
            }
            above += v[j];
          }
        }
        __syncthreads();
        prefix |= rand_[0] << shift;
        pmask |= 0xffu << shift;
        kk_ -= rand_[1];
        const bool whole = rand_[2] != 0u;
        __syncthreads();
        // the digit's whole bin is taken: exactly K keys are >= prefix (lower bits zero)
        if (whole) break;
      }
      T = prefix;
      unsigned int above = 0u;
      for (int i = tid; i < n; i += NT) {
        const unsigned int k = skey[phys(i)], c = sidx[phys(i)];
        if (k > T) {
          atomicOr(&sel[c >> 5], 1u << (c & 31));
          ++above;
        } else if (k == T) {
          atomicOr(&tie[c >> 5], 1u << (c & 31));
        }
      }
      above = block_sum_u32<NWA>(above, red);
      // ties at T: the lowest block indices, in order over the tie bitmap
      const int need = (int)K - (int)above;
      const int wpt = (nwords + NT - 1) / NT, w0 = tid * wpt;
      int tc = 0;
      for (int w = w0; w < w0 + wpt && w < nwords; ++w) tc += __popc(tie[w]);
      int tot;
      int tpre = block_exclusive_scan<NT>(tc, wsum, &tot);
      for (int w = w0; w < w0 + wpt && w < nwords; ++w) {
        unsigned int m = tie[w];
        while (m) {
          const int bit = __ffs(m) - 1;
          m &= m - 1;
          if (tpre < need) atomicOr(&sel[w], 1u << bit);
          ++tpre;
        }
      }
    }
    __syncthreads();
    // own block and its `local` predecessors
    {
      int64_t lo = own - f.local;
      if (lo < 0) lo = 0;
      const int64_t hi = own < f.nbk - 1 ? own : f.nbk - 1;
      for (int64_t c = lo + tid; c <= hi; c += NT) atomicOr(&sel[c >> 5], 1u << (c & 31));
    }
    __syncthreads();
    {
      const int wpt = (nwords + NT - 1) / NT, w0 = tid * wpt;
      int cnt = 0;
      for (int w = w0; w < w0 + wpt && w < nwords; ++w) cnt += __popc(sel[w]);
      int total;
      int at = block_exclusive_scan<NT>(cnt, wsum, &total);
      for (int w = w0; w < w0 + wpt && w < nwords; ++w) {
        unsigned int m = sel[w];
        while (m) {
          const int bit = __ffs(m) - 1;
          m &= m - 1;
          if (at < f.W) list[at] = w * 32 + bit;
          ++at;
        }
      }
      if (tid == 0) sh_n = (unsigned int)total;
    }
    __syncthreads();
  }
  const int num = (int)sh_n < f.W ? (int)sh_n : (int)f.W;

  // ---- attend slot SPW*group + w % SPW: keys [half kh, half kh + kh) of its block ----
  // Each wave's partial goes to LDS; the group's waves are combined into one partial (partial
  // `group` of the row), stored with agent-scope stores.
  const int64_t s = group * SPW + wv % SPW;
  const int half = wv / SPW;
  const int64_t stride = f.d + 2;
  float* prow = p.part + row * f.ngroups * stride;
  if (s < num) {
    const int64_t kh = (f.block + HALVES - 1) / HALVES;
    block_partial<DT, true, 16 / HALVES, false>(p, wpart[wv], qs[wv], ps[wv], b, h, kvh, 0, pos,
                                                list[s], half * kh, kh);
  } else {
    if (lane == 0) {
      wpart[wv][0] = -INFINITY;
      wpart[wv][1] = 0.0f;
    }
    for (int e = lane; e < f.d; e += 64) wpart[wv][2 + e] = 0.0f;
  }
  __syncthreads();
  {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWA; ++w) M = fmaxf(M, wpart[w][0]);
    float wt[NWA], L = 0.0f;
#pragma unroll
    for (int w = 0; w < NWA; ++w) {
      wt[w] = wpart[w][0] == -INFINITY ? 0.0f : exp2f(wpart[w][0] - M);  // empty: weight 0
      L += wpart[w][1] * wt[w];
    }
    float* gp = prow + group * stride;
    if (tid == 0) {
      put_part<true>(&gp[0], M);
      put_part<true>(&gp[1], L);
    }
    for (int e = tid; e < f.d; e += NT) {
      float o = 0.0f;
#pragma unroll
      for (int w = 0; w < NWA; ++w) o = fmaf(wpart[w][2 + e], wt[w], o);
      put_part<true>(&gp[2 + e], o);
    }
  }
  // folded append: workgroup 0 of the first query head of each key head writes the new token
  // into the caches (every read of that row in this launch comes from k_new / v_new)
  if (p.fused_append && group == 0 && h % f.G == 0 && wv == 0) {
    for (int e = lane; e < f.d; e += 64) {
      store_elem<DT>(const_cast<char*>(p.k), b * p.ksb + kvh * p.ksh + pos * p.ksn + e,
                     load_elem<DT>(p.k_new, b * p.knb + kvh * p.knh + e));
      store_elem<DT>(const_cast<char*>(p.v), b * p.vsb + kvh * p.vsh + pos * p.vsn + e,
                     load_elem<DT>(p.v_new, b * p.vnb + kvh * p.vnh + e));
    }
  }
  // The workgroup's partial stores happen before its arrival (the barrier), and the arrival
  // releases them at agent scope; the row's last workgroup acquires every other workgroup's
  // released stores with its own arrival (acq_rel: release and acquire edges of the HIP memory
  // model, not an ordering of this ISA's memory pipeline).
  __syncthreads();
  if (tid == 0) {
    const unsigned int old =
        __hip_atomic_fetch_add(&f.arrive[row], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    sh_last = old == (unsigned int)(f.ngroups - 1) ? 1u : 0u;
  }
  __syncthreads();
  if (!sh_last) return;  // uniform

  // ---- the row's last workgroup: combine the partials ----
  // (m_j, l_j) loaded by thread j together with the first batch of partials: partial j = w + NWA u
  // (u < kB) of wave w, lane e owning head dims e, e + 64; loads are unconditional (indices past
  // the partials / head dims read the last one and get weight 0 / are not stored)
  constexpr int kDE = kDMaxD / 64, kB = (kDMaxW / SPW + NWA - 1) / NWA;
  const int nump = (int)f.ngroups;  // partials of the row (one per group)
  const int jc = tid < nump ? tid : nump - 1;
  const float mj0 = __hip_atomic_load(&prow[jc * stride], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const float lj0 = __hip_atomic_load(&prow[jc * stride + 1], __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
  const int nb = (nump - wv + NWA - 1) / NWA;  // partials of this wave
  float acc[kDE];
#pragma unroll
  for (int t = 0; t < kDE; ++t) acc[t] = 0.0f;
  float M = 0.0f, L = 0.0f;
  for (int u0 = 0; u0 < nb || u0 == 0; u0 += kB) {
    float x[kB][kDE];
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const int jw = wv + NWA * (u0 + u), j = jw < nump ? jw : nump - 1;  // nump >= 1 (own block)
#pragma unroll
      for (int t = 0; t < kDE; ++t) {
        const int e = lane + 64 * t < f.d ? lane + 64 * t : (int)f.d - 1;
        x[u][t] = __hip_atomic_load(&prow[j * stride + 2 + e], __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (u0 == 0) {  // the weights, once the first batch is in flight
      const float mj = tid < nump ? mj0 : -INFINITY, lj = tid < nump ? lj0 : 0.0f;
      M = wave_max(mj);
      if (lane == 0) ps[0][wv] = M;
      __syncthreads();
      M = ps[0][0];
#pragma unroll
      for (int w = 1; w < NWA; ++w) M = fmaxf(M, ps[0][w]);
      const float wj = mj == -INFINITY ? 0.0f : exp2f(mj - M);  // empty partials: weight 0
      if (tid < nump) wgt[tid] = wj;
      L = wave_sum(lj * wj);
      if (lane == 0) ps[1][wv] = L;
      __syncthreads();
      L = 0.0f;
#pragma unroll
      for (int w = 0; w < NWA; ++w) L += ps[1][w];
    }
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const float w = u0 + u < nb ? wgt[wv + NWA * (u0 + u)] : 0.0f;
#pragma unroll
      for (int t = 0; t < kDE; ++t) acc[t] = fmaf(x[u][t], w, acc[t]);
    }
  }
#pragma unroll
  for (int t = 0; t < kDE; ++t)
    if (lane + 64 * t < f.d) qs[wv][lane + 64 * t] = acc[t];
  __syncthreads();
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  for (int e = tid; e < f.d; e += NT) {
    float o = 0.0f;
#pragma unroll
    for (int w = 0; w < NWA; ++w) o += qs[w][e];
    store_elem<DT>(p.o, b * p.osb + h * p.osh + e, o * inv);
  }
  int32_t* out = f.kv_idx + row * f.W;
  for (int j = tid; j < f.W; j += NT) out[j] = j < num ? list[j] : 0;
  if (tid == 0) {
    f.kv_num[row] = num;
    __hip_atomic_store(&f.arrive[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// 8 waves: 4 slots, each attended by 2 waves (half of the block's keys each)
template <int DT>
__global__ __launch_bounds__(512) void decode_attend_fused_kernel(FusedStep f, DecodeParams p) {
  attend_group<DT, 8, 2>(f, p, blockIdx.y, blockIdx.x);
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

namespace ssa {
namespace {
// The router keys of the general step (B*Hq*nbk u32), large enough to also hold the fused step's
// counters and chunk lists at 64-candidate chunks (with the query region before it).
size_t step_key_bytes(int64_t B, int64_t Hq, int64_t nbk) {
  const auto r256 = [](size_t x) { return (x + 255) / 256 * 256; };
  const size_t rows = (size_t)B * (size_t)Hq, nch = (size_t)(nbk + 63) / 64;
  const size_t keys = r256(rows * (size_t)nbk * 4u);
  const size_t lists = r256(rows * 4u) + r256(rows * nch * 4u) + 2 * r256(rows * nch * kDTop * 4u);
  return keys > lists ? keys : lists;
}
}  // namespace
}  // namespace ssa

extern "C" size_t ssa_decode_step_workspace_size(int64_t B, int64_t Hq, int64_t cap, int64_t d,
                                                 int64_t block, int64_t W) {
  const int64_t nbk = block > 0 ? (cap + block - 1) / block : 0;
  size_t qf = (size_t)B * Hq * d * 4u;
  qf = (qf + 255) / 256 * 256;
  const size_t keys = ssa::step_key_bytes(B, Hq, nbk);
  // partials: two per selected block (the one-launch step attends a block with two waves)
  return qf + keys + ssa_decode_attend_workspace_size(B, Hq, 2, W, d);
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
  const size_t key_bytes = step_key_bytes(B, Hq, nbk);
  float* qf = reinterpret_cast<float*>(ws);
  void* keys = ws + qf_bytes;
  float* part = reinterpret_cast<float*>(ws + qf_bytes + key_bytes);

  const bool completes = (pos + 1) % block == 0;
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

  // The fused two-launch step (decode_route_kernel + decode_attend_fused_kernel) serves the
  // common shapes; its workspace lives inside the regions of the general step's.
  const int64_t ncand = (pos + 1) / block < nbk ? (pos + 1) / block : nbk;  // complete blocks
  int64_t keep = top_c;
  if (top_c < 0) {
    keep = (int64_t)ceilf(budget_frac * (float)ncand);
    if (keep < 1) keep = 1;
  }
  const int64_t Kf = keep < ncand ? keep : ncand;
  const int64_t own = pos / block;
  const auto r256 = [](size_t x) { return (x + 255) / 256 * 256; };
  const size_t rows = (size_t)(B * Hq);
  // the smallest chunk (64, 128 or 256 candidates) whose lists the merge can hold: it loads
  // kDTop entries per chunk (whatever K is) and bounds from at most kDMaxChunks chunks
  auto fused_fits = [&](int64_t chunk, int64_t* nch_out) {
    const int64_t nch = ncand > 0 ? (ncand + chunk - 1) / chunk : 1;
    const size_t fa = r256(rows * 4u), fk = r256(rows * nch * 4u), fl = r256(rows * nch * kDTop * 4u);
    *nch_out = nch;
    return nch * kDTop <= kDSurv && nch <= kDMaxChunks && fa + fk + 2 * fl <= qf_bytes + key_bytes;
  };
  int64_t nchunk = 1, chunk = kDChunk / 4;
  bool fits = fused_fits(chunk, &nchunk);
  while (!fits && chunk < kDChunk) {
    chunk *= 2;
    fits = fused_fits(chunk, &nchunk);
  }
  const size_t f_arrive = r256(rows * 4u), f_kth = r256(rows * nchunk * 4u);
  const size_t f_list = r256(rows * nchunk * kDTop * 4u);
  const bool fused = fits && G <= kDMaxRows && (d == 32 || d == 64 || d == 128) &&
                     block <= kDMaxBlock && Kf <= kDTop && own < (int64_t)kDBitWords * 32 &&
                     W <= kDMaxW && aligned16(mu) && aligned16(var) && B * Hkv < 65536 &&
                     B * Hq < 65536;

  // 1. append the new token (and convert the query rows for the general router) in a launch of
  //    its own when the step completes a block (its summary needs the token in the cache) or the
  //    general step's router cannot read the query rows as they are; otherwise the append rides
  //    in the attend launch
  const bool fold = !completes && (fused || (strides[1] == d && strides[0] == Hq * d));
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
  if (completes) {
    const int64_t c = pos / block;
    const char* blk = kc + c * block * as.kcn * es;
    SSA_TRY(launch_block_summary(blk, dtype, B, Hkv, block, d, as.kcb, as.kch, as.kcn, block, block,
                                 SSA_STATS_POP, mu, var, nullptr, nbk, c, st));
  }

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

  if (fused) {
    // 3+4. route (exact scores, chunk top-K) -> merge, attend, combine
    FusedStep f;
    f.q = qc;
    f.qsb = strides[0];
    f.qsh = strides[1];
    f.mu = mu;
    f.var = var;
    f.B = B; f.Hq = Hq; f.Hkv = Hkv; f.G = G; f.d = d; f.nbk = nbk; f.ncand = ncand; f.K = Kf;
    f.local = local; f.pos = pos; f.block = block; f.W = W;
    f.coef2 = coef2;
    f.nchunk = (int)nchunk;
    f.ngroups = (int)((W + 3) / 4);
    f.arrive = reinterpret_cast<unsigned int*>(ws);
    f.ckth = reinterpret_cast<unsigned int*>(ws + f_arrive);
    f.ckey = reinterpret_cast<unsigned int*>(ws + f_arrive + f_kth);
    f.cidx = reinterpret_cast<unsigned int*>(ws + f_arrive + f_kth + f_list);
    f.kv_num = kv_num;
    f.kv_idx = kv_idx;
    const dim3 g1((unsigned)nchunk, (unsigned)(B * Hkv)), g2((unsigned)f.ngroups, (unsigned)(B * Hq));
#define SSA_FUSED_ROUTE(DT, NW, NWT)                                                              \
  do {                                                                                            \
    if (d == 32) decode_route_kernel<DT, 8, NW, NWT><<<g1, NWT * 64, 0, st>>>(f);                 \
    else if (d == 64) decode_route_kernel<DT, 16, NW, NWT><<<g1, NWT * 64, 0, st>>>(f);           \
    else decode_route_kernel<DT, 32, NW, NWT><<<g1, NWT * 64, 0, st>>>(f);                        \
  } while (0)
#define SSA_FUSED_STEP(DT)                                                                        \
  do {                                                                                            \
    if (chunk == kDChunk) SSA_FUSED_ROUTE(DT, 16, 16);                                            \
    else if (chunk == kDChunk / 4) SSA_FUSED_ROUTE(DT, 4, 8);                                     \
    else SSA_FUSED_ROUTE(DT, 8, 8);                                                               \
    decode_attend_fused_kernel<DT><<<g2, 512, 0, st>>>(f, p);                                     \
  } while (0)
    switch (dtype) {
      case SSA_F32: SSA_FUSED_STEP(SSA_F32); break;
      case SSA_F16: SSA_FUSED_STEP(SSA_F16); break;
      default: SSA_FUSED_STEP(SSA_BF16); break;
    }
#undef SSA_FUSED_STEP
#undef SSA_FUSED_ROUTE
    return launch_status("decode_attend_fused_kernel");
  }

  // 3. route the queries over the complete blocks
  SSA_TRY(route_impl(fold ? static_cast<const void*>(qc) : qf, fold ? dtype : SSA_F32, mu, var,
                     nullptr, B, Hq, Hkv, 1, nbk, d, SSA_ROUTE_QUERY, top_c, budget_frac, local,
                     coef2, 0.0f, pos, block, 1, kv_num, kv_idx, W, keys, key_bytes, st));

  // 4. attend
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
