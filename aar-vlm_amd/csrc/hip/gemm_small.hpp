// Short-operand GEMM kernels (gemm_small.hip), called by the GEMM planner in
// gemm_f32.hip and by the embedding backward in nn_ops.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace aar {

// TN with a short output height: C[M, N] = A[K, M]^T . B[K, N], A and B
// contiguous (lda = M, ldb = N), M <= kShortMMax.  With ids != nullptr, A is
// the one-hot matrix A[k][m] = (ids[k] == m) (ids out of [0, M) give a zero
// row) and the A pointer is ignored.  Split over K into `splits` partial
// products summed in split order by a second launch (deterministic); needs
// splits*M*N floats of workspace when splits > 1.
constexpr int64_t kShortMMax = 260;
bool shortm_shape_ok(int64_t M, int64_t N, int64_t K);
// The split count the planner uses, limited to what `ws_bytes` holds.
int shortm_splits(int64_t M, int64_t N, int64_t K, size_t ws_bytes);
// Workspace for `splits` (the one-hot form caps a split's K chunk, so it may
// need more partial products).
size_t shortm_workspace_bytes(int64_t M, int64_t N, int64_t K, int splits, bool onehot = false);
int run_shortm(const float* A, const int64_t* ids, const float* B, float* C, int64_t M, int64_t N, int64_t K,
               int splits, void* workspace, size_t ws_bytes, hipStream_t st);

// NN with a short contraction: C[M, N] = A[M, K] . B[K, N], contiguous
// operands, K <= kShortKMax.
constexpr int64_t kShortKMax = 128;
bool shortk_shape_ok(int64_t M, int64_t N, int64_t K);
int run_shortk(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K, hipStream_t st);

}  // namespace aar
