// Shared device helpers for the gfx950 kernels: vector types, wave64
// reductions built on DPP / ds_swizzle, and host-side launch checking.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "aar_hip.h"

namespace aar {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// ---------------------------------------------------------------- wave64 reductions
// Butterfly over the 64 lanes of a wave.  Quad steps use DPP quad_perm, the
// 8- and 16-lane steps use DPP row_half_mirror / row_mirror (after the quad
// step every lane of a quad holds the same value, so mirroring pairs each lane
// with the other half), the 32-lane step uses ds_swizzle (xor 0x10 within 32
// lanes) and the final step combines the two 32-lane halves with readlane.
// Every lane returns the full reduction.

__device__ __forceinline__ float dpp_quad_xor1(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_quad_xor2(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_half_mirror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_row_mirror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
}
__device__ __forceinline__ float swizzle_xor16(float v) {
  // bitmask mode: and_mask=0x1f, or_mask=0, xor_mask=0x10
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}
__device__ __forceinline__ float lane_xor32(float v) {
  return __shfl_xor(v, 32, 64);
}

// v (op) v[lane ^ 32] in one VALU op pair: v_permlane32_swap (gfx950) hands
// every lane both halves' values, so no LDS round trip is needed.  Both
// halves compute the same commutative op and end with identical bits.  The
// builtin exists only for the device target; the host pass never runs this.
__device__ __forceinline__ float half_swap_sum(float v) {
#if defined(__HIP_DEVICE_COMPILE__)
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
#else
  return v;
#endif
}
__device__ __forceinline__ float half_swap_max(float v) {
#if defined(__HIP_DEVICE_COMPILE__)
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
#else
  return v;
#endif
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_quad_xor1(v);
  v += dpp_quad_xor2(v);
  v += dpp_half_mirror(v);
  v += dpp_row_mirror(v);
  v += swizzle_xor16(v);
  const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  return lo + hi;
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_quad_xor1(v));
  v = fmaxf(v, dpp_quad_xor2(v));
  v = fmaxf(v, dpp_half_mirror(v));
  v = fmaxf(v, dpp_row_mirror(v));
  v = fmaxf(v, swizzle_xor16(v));
  const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  return fmaxf(lo, hi);
}

// ---------------------------------------------------------------- host helpers

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? AAR_OK : static_cast<int>(e);
}

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Multiprocessor count of the current device, cached per device.
int device_cu_count();

}  // namespace aar
