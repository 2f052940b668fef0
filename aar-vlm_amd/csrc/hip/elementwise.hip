// Elementwise fp32 kernels.  aar_add_f32 is the device leg of add_grads
// (reference add_kernel, cppsrc/ops/elementwise.cu:11-14, launched from
// add_cuda at cppsrc/ops/elementwise.cu:107-118): c = a + b.
// 128-bit loads/stores, grid-stride over a grid sized to the chip.
#include <hip/hip_runtime.h>

#include "common.hpp"

namespace aar {
namespace {

__global__ void __launch_bounds__(256)
add_vec_kernel(const f32x4* __restrict__ a, const f32x4* __restrict__ b, f32x4* __restrict__ c,
               int64_t n4) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) c[i] = a[i] + b[i];
}

__global__ void __launch_bounds__(256)
add_scalar_kernel(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ c,
                  int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) c[i] = a[i] + b[i];
}

struct StridedDesc {
  int ndim;
  int64_t shape[8];
  int64_t src[8];
  int64_t dst[8];
};

// dst[off_dst(idx)] = src[off_src(idx)] for the row-major linear index i of
// `shape`; the index is decomposed from the last dim (fastest) outward.
__global__ void __launch_bounds__(256)
strided_copy_kernel(const float* __restrict__ src, float* __restrict__ dst, StridedDesc desc,
                    int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    int64_t rem = i, so = 0, dof = 0;
    for (int dim = desc.ndim - 1; dim >= 0; --dim) {
      const int64_t ext = desc.shape[dim];
      const int64_t idx = rem % ext;
      rem /= ext;
      so += idx * desc.src[dim];
      dof += idx * desc.dst[dim];
    }
    dst[dof] = src[so];
  }
}

// Fast path: the innermost dim is contiguous in both views, so each row of
// `inner` floats is copied with 128-bit accesses; the outer index is
// decomposed once per row (32-bit math: outer extents < 2^31).
struct RowDesc {
  int ndim;  // outer dims (all but the last)
  int shape[7];
  int64_t src[7];
  int64_t dst[7];
};

template <bool VEC>
__global__ void __launch_bounds__(256)
strided_rows_kernel(const float* __restrict__ src, float* __restrict__ dst, RowDesc desc, int64_t rows,
                    int inner) {
  const int per_row = VEC ? inner / 4 : inner;
  const int64_t total = rows * per_row;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
    const int64_t row = e / per_row;
    const int c = (int)(e - row * per_row);
    int64_t so = 0, dof = 0;
    uint32_t rem = (uint32_t)row;
    for (int dim = desc.ndim - 1; dim >= 0; --dim) {
      const uint32_t ext = (uint32_t)desc.shape[dim];
      const uint32_t idx = rem % ext;
      rem /= ext;
      so += (int64_t)idx * desc.src[dim];
      dof += (int64_t)idx * desc.dst[dim];
    }
    if (VEC) {
      *reinterpret_cast<f32x4*>(dst + dof + 4 * c) = *reinterpret_cast<const f32x4*>(src + so + 4 * c);
    } else {
      dst[dof + c] = src[so + c];
    }
  }
}

// One thread per work item over a grid that covers the data once (faster HBM
// streaming on MI355X than a persistent grid-stride loop); past 2^20 blocks
// the kernels' grid-stride loops take over.
unsigned grid_for(int64_t work) {
  constexpr int64_t kCap = int64_t(1) << 20;
  int64_t g = (work + 255) / 256;
  if (g > kCap) g = kCap;
  return (unsigned)(g > 0 ? g : 1);
}

}  // namespace
}  // namespace aar

using namespace aar;

extern "C" int aar_add_f32(const float* a, const float* b, float* c, int64_t n, void* stream) {
  if (n < 0) return AAR_EINVAL;
  if (n == 0) return AAR_OK;
  if (!a || !b || !c) return AAR_EINVAL;
  hipStream_t st = as_stream(stream);
  if (aligned16(a) && aligned16(b) && aligned16(c)) {
    const int64_t n4 = n / 4;
    if (n4 > 0) {
      add_vec_kernel<<<dim3(grid_for(n4)), dim3(256), 0, st>>>(reinterpret_cast<const f32x4*>(a),
                                                              reinterpret_cast<const f32x4*>(b),
                                                              reinterpret_cast<f32x4*>(c), n4);
      const int rc = launch_status();
      if (rc != AAR_OK) return rc;
    }
    const int64_t done = n4 * 4;
    if (done < n) {
      add_scalar_kernel<<<dim3(1), dim3(256), 0, st>>>(a + done, b + done, c + done, n - done);
    }
  } else {
    add_scalar_kernel<<<dim3(grid_for(n)), dim3(256), 0, st>>>(a, b, c, n);
  }
  return launch_status();
}

extern "C" int aar_strided_copy_f32(const float* src, float* dst, int ndim, const int64_t* shape,
                                    const int64_t* src_strides, const int64_t* dst_strides,
                                    void* stream) {
  if (ndim < 0 || ndim > 8) return AAR_EINVAL;
  int64_t n = 1;
  StridedDesc desc;
  desc.ndim = ndim;
  for (int i = 0; i < ndim; ++i) {
    if (!shape || !src_strides || !dst_strides || shape[i] < 0) return AAR_EINVAL;
    desc.shape[i] = shape[i];
    desc.src[i] = src_strides[i];
    desc.dst[i] = dst_strides[i];
    n *= shape[i];
  }
  if (n == 0) return AAR_OK;
  if (!src || !dst) return AAR_EINVAL;
  hipStream_t st = as_stream(stream);
  const int64_t inner = ndim > 0 ? shape[ndim - 1] : 1;
  const int64_t rows = ndim > 0 ? n / inner : 1;
  if (ndim >= 1 && src_strides[ndim - 1] == 1 && dst_strides[ndim - 1] == 1 && rows < INT32_MAX &&
      inner < INT32_MAX) {
    RowDesc rd;
    rd.ndim = ndim - 1;
    for (int i = 0; i < ndim - 1; ++i) {
      rd.shape[i] = (int)shape[i];
      rd.src[i] = src_strides[i];
      rd.dst[i] = dst_strides[i];
    }
    bool vec = inner % 4 == 0 && aligned16(src) && aligned16(dst);
    for (int i = 0; i < ndim - 1 && vec; ++i) vec = (src_strides[i] % 4 == 0) && (dst_strides[i] % 4 == 0);
    if (vec) {
      strided_rows_kernel<true><<<dim3(grid_for(n / 4)), dim3(256), 0, st>>>(src, dst, rd, rows, (int)inner);
    } else {
      strided_rows_kernel<false><<<dim3(grid_for(n)), dim3(256), 0, st>>>(src, dst, rd, rows, (int)inner);
    }
    return launch_status();
  }
  strided_copy_kernel<<<dim3(grid_for(n)), dim3(256), 0, st>>>(src, dst, desc, n);
  return launch_status();
}
