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

}  // namespace aar
