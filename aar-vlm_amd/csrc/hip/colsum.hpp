// Column sums (nn_ops.hip) as other kernels' epilogues produce them: the GEMM
// relu-mask epilogue (gemm_f32.hip) writes aar_colsum_f32's stage-1 partials
// and finishes with its stage 2, so the sums are bit for bit aar_colsum_f32's.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aar {

// Whether aar_colsum_f32 over `rows` rows sums the 64-row chunks
// p = row / 64 in its stage 1 (rows a positive multiple of 64, at most 256
// chunks).
bool colsum_chunks_of_64(int64_t rows);

// aar_colsum_f32's stage 2: out[c] = sum over p of part[p * cols + c], in its
// fixed order.
int colsum_finish(const float* part, float* out, int nparts, int64_t cols, hipStream_t st);

// That order, for a workgroup of kColsumSlices * COLS threads owning columns
// c0 .. c0 + COLS - 1: slice j sums its contiguous run of the parts in order,
// then a fixed pairwise tree over the slices in LDS finishes each column.
// The result does not depend on COLS, so launches of any width agree bit for
// bit.
constexpr int kColsumSlices = 64;
template <int COLS>
__device__ __forceinline__ void colsum_stage2_block(const float* __restrict__ part, float* __restrict__ out,
                                                    int nparts, int64_t cols, int64_t c0,
                                                    float (&acc)[kColsumSlices][COLS]) {
  const int cl = threadIdx.x % COLS, slice = threadIdx.x / COLS;
  const int64_t c = c0 + cl;
  const int per = (nparts + kColsumSlices - 1) / kColsumSlices;
  const int p0 = slice * per;
  const int p1 = nparts < p0 + per ? nparts : p0 + per;
  float s = 0.f;
  if (c < cols) {
    for (int p = p0; p < p1; ++p) s += part[(int64_t)p * cols + c];
  }
  acc[slice][cl] = s;
  __syncthreads();
#pragma unroll
  for (int h = kColsumSlices / 2; h >= 1; h /= 2) {
    if (slice < h) acc[slice][cl] += acc[slice + h][cl];
    __syncthreads();
  }
  if (slice == 0 && c < cols) out[c] = acc[0][cl];
}

}  // namespace aar
