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

// ---------------------------------------------------------------- HBM -> LDS DMA
typedef __attribute__((address_space(3))) void lds_void_t;

// One 16-byte-per-lane HBM -> LDS DMA (global_load_lds_dwordx4): lane i
// writes the 16 bytes at g into LDS at lds + 16 * i; `lds` must be
// wave-uniform.  The builtin only exists for the device target; the host
// pass, which never runs this code, sees an empty body so kernel host stubs
// are still emitted.
__device__ __forceinline__ void dma16(const void* g, lds_void_t* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
#endif
}

// The same with 4 bytes per lane (lane i writes lds + 4 * i).
__device__ __forceinline__ void dma4(const void* g, lds_void_t* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(g, lds, 4, 0, 0);
#endif
}

// The same two DMAs issued as inline assembly, which the compiler's wait
// insertion does not see.  For the builtins it assumes an LDS read may alias
// any DMA in flight unless it can tell their buffers apart, and waits for all
// of them (vmcnt(0)) before the read; with a double-buffered stage indexed at
// run time it cannot, so the next tile's DMA latency lands on every
// iteration.  Callers of these forms order the DMAs themselves: an explicit
// wait_vm_lgkm0 and barrier before any wave reads the staged buffer, and none
// of their own vector-memory operations between the DMAs and that wait that
// the wait's count does not allow for.  M0 (the LDS base) is an asm operand,
// so the compiler writes it.
__device__ __forceinline__ void dma16_untracked(const void* g, lds_void_t* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds);
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(m0) : "memory");
#endif
}

__device__ __forceinline__ void dma4_untracked(const void* g, lds_void_t* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds);
  asm volatile("global_load_lds_dword %0, off" ::"v"(g), "{m0}"(m0) : "memory");
#endif
}

// The untracked DMAs with a wave-uniform 64-bit base in SGPRs and a 32-bit
// per-lane byte offset (the global "saddr" form): a loop that walks tiles
// moves only the scalar base, so issuing costs no vector arithmetic.
__device__ __forceinline__ void dma16_untracked_s(uint32_t lane_off, const void* base, lds_void_t* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds);
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(lane_off), "s"(base), "{m0}"(m0) : "memory");
#endif
}

__device__ __forceinline__ void dma4_untracked_s(uint32_t lane_off, const void* base, lds_void_t* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds);
  asm volatile("global_load_lds_dword %0, %1" ::"v"(lane_off), "s"(base), "{m0}"(m0) : "memory");
#endif
}

// s_waitcnt vmcnt(N) lgkmcnt(0) (expcnt untouched): this wave's DMAs and
// loads but the last N are done, and its LDS accesses are complete.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

// Workgroup barrier without a memory fence (DMA buffers are ordered by the
// explicit waits); the empty asm statements keep the compiler from moving
// LDS accesses across it.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------- host helpers

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? AAR_OK : static_cast<int>(e);
}

__host__ __device__ inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Multiprocessor count of the current device, cached per device.
int device_cu_count();

}  // namespace aar
