// Shared helpers for the gfx950 kernels of libssa_hip.so: status/error plumbing, dtype traits,
// and the order-preserving float key used by the router.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ssa_hip.h"

namespace ssa {

// Records a printf-style message as this thread's last error (read via ssa_last_error()).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// Maps a hipError_t to SSA_ERR_HIP with a message naming `what`; SSA_OK on success.
int hip_status(hipError_t e, const char* what);

// Checks for a failed launch of the kernel named `what`.
inline int launch_status(const char* what) { return hip_status(hipGetLastError(), what); }

#define SSA_REQUIRE(cond, code, ...)   \
  do {                                 \
    if (!(cond)) {                     \
      ::ssa::set_error(__VA_ARGS__);   \
      return (code);                   \
    }                                  \
  } while (0)

#define SSA_TRY(expr)            \
  do {                           \
    int ssa_rc_ = (expr);        \
    if (ssa_rc_ != SSA_OK)       \
      return ssa_rc_;            \
  } while (0)

inline int dtype_size(int dtype) {
  switch (dtype) {
    case SSA_F32: return 4;
    case SSA_F16: return 2;
    case SSA_BF16: return 2;
    default: return 0;
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- device-side helpers -----------------------------------------------------------------------

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Converts 8 packed 16-bit values (one 16-byte load) to fp32.
__device__ inline void unpack8(const u32x4& w, float* out, bool is_bf16) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    unsigned int x = w[i];
    if (is_bf16) {
      out[2 * i] = __uint_as_float(x << 16);
      out[2 * i + 1] = __uint_as_float(x & 0xffff0000u);
    } else {
      _Float16 lo = __builtin_bit_cast(_Float16, (unsigned short)(x & 0xffffu));
      _Float16 hi = __builtin_bit_cast(_Float16, (unsigned short)(x >> 16));
      out[2 * i] = (float)lo;
      out[2 * i + 1] = (float)hi;
    }
  }
}

// The value of lane (lane ^ j) of the wave, for j = 1, 2, 4, 8, 16, 32: DPP quad permutes and
// row rotations within 16-lane rows, the gfx950 permlane swaps across rows and halves -- VALU
// operations of a few cycles, where __shfl_xor goes through the LDS unit (ds_bpermute, ~100+
// cycles of latency per step of a dependent chain). j must be a compile-time constant after
// unrolling (the switch folds). Lane mapping checked against lane ^ j on the GPU.
__device__ inline unsigned int lane_xor(unsigned int x, int j) {
  const int lane = threadIdx.x & 63;
  switch (j) {
    case 1: return __builtin_amdgcn_update_dpp(0u, x, 0xB1, 0xf, 0xf, false);  // quad_perm 1,0,3,2
    case 2: return __builtin_amdgcn_update_dpp(0u, x, 0x4E, 0xf, 0xf, false);  // quad_perm 2,3,0,1
    case 4: {
      const unsigned int up = __builtin_amdgcn_update_dpp(0u, x, 0x12C, 0xf, 0xf, false);  // ror 12
      const unsigned int dn = __builtin_amdgcn_update_dpp(0u, x, 0x124, 0xf, 0xf, false);  // ror 4
      return (lane & 4) ? dn : up;
    }
    case 8: return __builtin_amdgcn_update_dpp(0u, x, 0x128, 0xf, 0xf, false);  // row_ror 8
    case 16: {
      const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
      return (lane & 16) ? r[0] : r[1];
    }
    default: {
      const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
      return (lane & 32) ? r[0] : r[1];
    }
  }
}
__device__ inline float lane_xor(float x, int j) {
  return __uint_as_float(lane_xor(__float_as_uint(x), j));
}
__device__ inline int lane_xor(int x, int j) { return (int)lane_xor((unsigned int)x, j); }
__device__ inline double lane_xor(double x, int j) {
  const unsigned long long u = __double_as_longlong(x);
  const unsigned int lo = lane_xor((unsigned int)(u & 0xffffffffu), j);
  const unsigned int hi = lane_xor((unsigned int)(u >> 32), j);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// Orders one wave's LDS writes before its later LDS reads (other lanes' data).
__device__ inline void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Order-preserving map of an fp32 score to uint32 (larger score -> larger key). -0 is folded
// onto +0 so the two compare equal, as they do for torch.topk; NaN maps above +inf (torch.topk
// treats NaN as the largest value).
__device__ inline unsigned int score_key(float r) {
  unsigned int u = __float_as_uint(r);
  u = u == 0x80000000u ? 0u : u;  // -0 -> +0
  // negative: all bits flipped; otherwise the sign bit set
  const unsigned int k = u ^ ((unsigned int)((int)u >> 31) | 0x80000000u);
  return r != r ? 0xffffffffu : k;
}

}  // namespace ssa
