/*
 * aar_hip.h — C ABI of the MI355X (gfx950) device backend for aargrad.
 *
 * Plain C: pointers, sizes, an opaque stream handle (hipStream_t passed as
 * void*; NULL is the null stream) and an int status.  No C++ or torch types.
 *
 * Contract for every entry point:
 *   - Returns AAR_OK (0) on success.  A positive value is a hipError_t code;
 *     a negative value is one of the AAR_E* codes below.
 *     aar_error_string() turns either into text.
 *   - Never allocates an output.  Inputs are borrowed and outputs are written
 *     in place; the caller owns all memory.  Entry points that need scratch
 *     memory take an explicit workspace and expose its size through a
 *     *_workspace_bytes() query (the one *_noalloc_* entry point uses a
 *     static per-GPU buffer instead).
 *   - All work is enqueued on `stream` and returns without waiting; results are
 *     visible to the host after aar_stream_synchronize()/aar_synchronize() or a
 *     device-to-host copy.
 *   - fp32 tensors are dense row-major (C-contiguous).
 *
 * Each declaration names the reference (AARONKANG04/aar-vlm) interface it
 * replaces, as file:line under the reference tree.
 */
#ifndef AAR_HIP_H
#define AAR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AAR_OK 0
#define AAR_EINVAL (-1)        /* bad shape / argument (maps to std::invalid_argument) */
#define AAR_EWORKSPACE (-2)    /* workspace pointer NULL or too small */
#define AAR_EUNSUPPORTED (-3)  /* shape outside what the kernels implement */
#define AAR_ENOMEM (-4)        /* device allocation failed (maps to std::bad_alloc) */
#define AAR_ESCRATCH (-5)      /* needs more than a no-allocation entry point's static scratch */

/* ---------------------------------------------------------------- runtime */

/* Text for a status returned by any aar_* call (static storage). */
const char* aar_error_string(int status);

/* Number of visible GPUs.  Replaces the implicit lazy CUDA init that the
 * reference probes with Tensor::zeros(..., CUDA) (tests/python/test_flash_attention.py:8-13). */
int aar_device_count(int* count);

/* Device properties used by launch heuristics and roofline reporting. */
int aar_device_info(int* cu_count, int* clock_khz, int* lds_bytes_per_cu,
                    char* arch_name, int arch_name_len);

/* Device allocation (AAR_ENOMEM when the device is out of memory).  Replaces
 * CUDAAllocator::alloc/free (cppsrc/core/cuda_allocator.cpp:8-22). */
int aar_malloc(void** ptr, size_t bytes);
int aar_free(void* ptr);

/* Copies.  Replaces copy_bytes (cppsrc/core/cuda_copy.hpp:8-10).
 * kind: 1 = host->device, 2 = device->host, 3 = device->device.
 * Host<->device copies are synchronous with respect to the host;
 * device->device copies are ordered on `stream`. */
int aar_memcpy(void* dst, const void* src, size_t bytes, int kind, void* stream);

/* Zero `bytes` of device memory with a fill kernel (capturable into a HIP graph).
 * Replaces zero_bytes (cppsrc/core/cuda_copy.hpp:12). */
int aar_memset_zero(void* ptr, size_t bytes, void* stream);

/* Replaces cuda_synchronize (cppsrc/python/binding.cpp:62-69). */
int aar_synchronize(void);
int aar_stream_synchronize(void* stream);

/* Timing events (bench harness; the reference uses cudaEvent in
 * bench/bench_matmul.cu:66-89). */
int aar_event_create(void** event);
int aar_event_destroy(void* event);
int aar_event_record(void* event, void* stream);
int aar_event_elapsed_ms(float* ms, void* start, void* stop);

/* ------------------------------------------------------------------- GEMM */

#define AAR_GEMM_NN 0  /* C[M,N] = A[M,K]   . B[K,N]    matmul       */
#define AAR_GEMM_NT 1  /* C[M,N] = A[M,K]   . B[N,K]^T  matmul_a_bt  */
#define AAR_GEMM_TN 2  /* C[M,N] = A[K,M]^T . B[K,N]    matmul_at_b  */

/* Scratch needed by aar_gemm_f32 for a split-K launch of this shape (0 when
 * the shape runs without split-K). */
size_t aar_gemm_f32_workspace_bytes(int op, int64_t M, int64_t N, int64_t K);

/* fp32 GEMM on v_mfma_f32_32x32x2f32.  Replaces matmul_cuda /
 * matmul_a_bt_cuda / matmul_at_b_cuda (cppsrc/ops/matmul.cpp:10-12) and the
 * raw-pointer launchers matmul_v4_launch / matmul_a_bt_v4_launch /
 * matmul_at_b_v4_launch (cppsrc/ops/matmul.cu:648-650).
 * `workspace` may be NULL when aar_gemm_f32_workspace_bytes() returned 0;
 * with a smaller workspace the call runs without split-K (same result up to
 * summation order).  K == 0 writes zeros. */
int aar_gemm_f32(int op, int64_t M, int64_t N, int64_t K,
                 const float* A, const float* B, float* C,
                 void* workspace, size_t workspace_bytes, void* stream);

/* C[M,N] = op(A, B) + bias, bias[N] added to every row: the GEMM with the bias
 * in its epilogue (or after the split-K reduction).  Bit-identical to
 * aar_gemm_f32 followed by aar_add_bias_f32 (one fp32 addition per element).
 * K == 0 returns AAR_EUNSUPPORTED.  Replaces the matmul_a_bt_cuda + add_bias_cuda
 * pair of nn.Linear with bias (aargrad/nn.py:101-105, cppsrc/ops/matmul.cpp:11,
 * elementwise.cpp:24). */
int aar_gemm_f32_bias(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B,
                      const float* bias, float* C, void* workspace, size_t workspace_bytes, void* stream);

/* C = max(0, A W^T + bias[col]): the linear layer followed by relu, with both
 * in the GEMM epilogue; bit-identical to aar_gemm_f32_bias then relu.  op must
 * be AAR_GEMM_NT (else AAR_EUNSUPPORTED, as is K == 0).  Replaces
 * matmul_a_bt_cuda + add_bias_cuda + relu_cuda of the MLP's first layer
 * (cppsrc/ops/matmul.cpp:11, elementwise.cpp:24 and :15). */
int aar_gemm_f32_bias_relu(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B,
                           const float* bias, float* C, void* workspace, size_t workspace_bytes,
                           void* stream);
/* C = A W^T + R (R [M, N] contiguous): a linear layer without bias followed
 * by a residual add, the add in the GEMM epilogue.  Bit-identical to
 * aar_gemm_f32 then aar_add_f32 (the same product plan, one fp32 addition per
 * element).  op must be AAR_GEMM_NT (else AAR_EUNSUPPORTED, as is K == 0).
 * Replaces matmul_a_bt_cuda + add_cuda of a pre-norm block's attention
 * output projection and residual, x + proj(attn) (cppsrc/ops/matmul.cpp:11,
 * elementwise.cpp:13; python/shakespeare/scripts/model.py:19-23). */
int aar_gemm_f32_add(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B,
                     const float* R, float* C, void* workspace, size_t workspace_bytes, void* stream);
/* C = (A W^T + bias[col]) + R: the same after a linear layer with a bias;
 * bit-identical to aar_gemm_f32_bias then aar_add_f32.  NT only.  Replaces
 * matmul_a_bt_cuda + add_bias_cuda + add_cuda of the MLP's output layer and
 * its residual (cppsrc/ops/matmul.cpp:11, elementwise.cpp:24 and :13). */
int aar_gemm_f32_bias_add(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B,
                          const float* bias, const float* R, float* C, void* workspace,
                          size_t workspace_bytes, void* stream);
/* C = mask > 0 ? A B : 0 elementwise (mask [M, N] contiguous, the relu's
 * output): the relu backward applied in the GEMM epilogue of the next layer's
 * input gradient dY W; bit-identical to aar_gemm_f32 then relu_backward.  op
 * must be AAR_GEMM_NN (else AAR_EUNSUPPORTED).  Replaces matmul_cuda +
 * relu_backward_cuda (cppsrc/ops/matmul.cpp:10, elementwise.cpp:17).  On
 * MI355X at the GPT step's 16384x1536x384 it runs slower than the GEMM plus
 * the separate mask pass, so the host MLP op uses those. */
int aar_gemm_f32_relu_mask(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B,
                           const float* mask, float* C, void* workspace, size_t workspace_bytes,
                           void* stream);
/* The MLP's relu carried as a bit mask from its forward product to its
 * backward one, so the backward reads 1 bit per element instead of the relu's
 * output.  aar_gemm_f32_bias_relu_bits: C as aar_gemm_f32_bias_relu (same
 * plan, bit-identical) and bits[(r / 32) * N + c] bit (r % 32) = (C[r][c] > 0):
 * one uint32_t word per column of each 32-row block, (M + 31) / 32 * N words,
 * bits past row M zero.  NT only.
 * aar_gemm_f32_mask_bits_colsum: C = bit(r, c) ? A B : 0 (NN) and colsum[c] =
 * sum over rows of C, bit-identical to aar_gemm_f32 (given the workspace
 * aar_gemm_f32_workspace_bytes asks for), the relu backward and
 * aar_colsum_f32; its workspace (aar_gemm_f32_mask_bits_colsum_workspace_bytes)
 * holds colsum's per-64-row partials, which the GEMM epilogue writes.  With
 * colsum NULL it applies the mask only (no workspace).  Both return
 * AAR_EUNSUPPORTED, launching nothing, where the product's plan splits K or
 * has no such epilogue (register staging, K-group tiles, wave tiles of other
 * than 64 rows for the mask) or, for the column sums, where M is not a
 * multiple of 64 up to 16384 (colsum's partials are not 64-row chunks
 * there); the caller then runs the separate passes.  Replace
 * matmul_a_bt_cuda + add_bias_cuda + relu_cuda and matmul_cuda +
 * relu_backward_cuda + the bias gradient's column sum of the MLP
 * (cppsrc/ops/matmul.cpp:10-11, elementwise.cpp:15-24). */
int aar_gemm_f32_bias_relu_bits(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B,
                                const float* bias, float* C, uint32_t* bits, void* workspace,
                                size_t workspace_bytes, void* stream);
size_t aar_gemm_f32_mask_bits_colsum_workspace_bytes(int64_t M, int64_t N);
int aar_gemm_f32_mask_bits_colsum(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B,
                                  const uint32_t* bits, float* C, float* colsum, void* workspace,
                                  size_t workspace_bytes, void* stream);
/* A linear layer's weight and bias gradients from one pass over its output
 * gradient G: C = A^T B (TN; A = G [K, M], B = the layer input [K, N]) and
 * colsum[m] = sum over k of A[k][m].  C is bit-identical to aar_gemm_f32 given
 * the workspace aar_gemm_f32_workspace_bytes asks for (the same plan), colsum
 * to aar_colsum_f32 over A: the GEMM's main loop sums the A tiles it stages
 * into colsum's per-64-row partials.  The workspace
 * (aar_gemm_f32_colsum_a_workspace_bytes) holds the split-K partials and those.
 * Returns AAR_EUNSUPPORTED, launching nothing, for op other than TN, K not a
 * multiple of 64 up to 16384 (colsum's partials are not 64-row chunks there),
 * or a plan without the path (unaligned operands, the thin or short kernels,
 * K-group tiles, K splits not on 64-row chunks); the caller then runs the two
 * passes.  Replaces matmul_at_b_cuda + bias_grad_cuda of nn.Linear's backward
 * (cppsrc/ops/matmul.cpp:12, elementwise.cpp:25). */
size_t aar_gemm_f32_colsum_a_workspace_bytes(int op, int64_t M, int64_t N, int64_t K);
int aar_gemm_f32_colsum_a(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B, float* C,
                          float* colsum, void* workspace, size_t workspace_bytes, void* stream);

/* Batched GEMM with explicit leading dimensions: for b in [0, batch),
 * C_b = op(A_b, B_b) with A_b = A + b*strideA (and so on), op as in
 * aar_gemm_f32 but rows of A/B/C at lda/ldb/ldc elements (lda >= K for NN/NT,
 * >= M for TN; ldb >= N for NN/TN, >= K for NT; ldc >= N).  No split-K, so no
 * workspace.  Any batch count: batches go in launches of at most 65535.
 * K == 0 needs a contiguous C (ldc == N, strideC == M*N).
 * Replaces bmm_cuda / bmm_a_bt_cuda / bmm_at_b_cuda (cppsrc/ops/bmm.cpp:10-12). */
int aar_gemm_f32_batched(int op, int64_t batch, int64_t M, int64_t N, int64_t K,
                         const float* A, int64_t lda, int64_t strideA,
                         const float* B, int64_t ldb, int64_t strideB,
                         float* C, int64_t ldc, int64_t strideC, void* stream);

/* Tuning and test access to the GEMM tile configurations (no counterpart in
 * the reference, whose launchers pick a tile size internally,
 * cppsrc/ops/matmul.cu:792-832).  Tile configurations are numbered 0..n-1;
 * aar_gemm_f32_tile_config returns AAR_EINVAL past the last one.  Id n is
 * the thin-output kernel: N <= 128, 16 <= K <= 512 with K % 16 == 0, B
 * padded to 16-column blocks in LDS (at most 128 KB), a 16-byte aligned A
 * for NN/NT and B for NT, no split (splits must be 1); outside those limits
 * it returns AAR_EUNSUPPORTED.  Id n+1 is the short-operand kernels: TN with
 * M <= 260 (split over K: `splits` partial products summed in order; a
 * 16-byte aligned B, N % 4 == 0; up to 6 32-row blocks of M, 2 when A is not
 * 16-byte aligned) and NN with K <= 128 (unsplit); aar_gemm_f32 plans them
 * for plain products whose rows the tiled kernels cannot stage (not 16-byte
 * aligned: a vocabulary of 65).
 * aar_gemm_f32_plan reports the configuration and split count aar_gemm_f32
 * would use with `workspace_bytes` of scratch (id n for thin outputs such as
 * a vocabulary head; aar_gemm_f32 takes it only when the operands' alignment
 * allows).  aar_gemm_f32_with_config runs a given configuration and split-K
 * count (needs splits*M*N*4 bytes of workspace when splits > 1, else
 * AAR_EWORKSPACE); results agree with aar_gemm_f32 up to summation order. */
int aar_gemm_f32_tile_config(int config, int* tile_m, int* tile_n, int* tile_k);
int aar_gemm_f32_plan(int op, int64_t M, int64_t N, int64_t K, size_t workspace_bytes,
                      int* config, int* splits);
int aar_gemm_f32_with_config(int op, int64_t M, int64_t N, int64_t K,
                             const float* A, const float* B, float* C,
                             void* workspace, size_t workspace_bytes,
                             int config, int splits, void* stream);

/* ------------------------------------------------------- row-wise kernels */

/* y = softmax(x) over the last dim; x,y [rows, cols].
 * Replaces softmax_cuda (cppsrc/ops/softmax.cpp:11). */
int aar_softmax_fwd_f32(const float* x, float* y, int64_t rows, int64_t cols,
                        void* stream);

/* dx = y * (g - sum(g*y)) per row.  Replaces softmax_backward_cuda
 * (cppsrc/ops/softmax.cpp:12). */
int aar_softmax_bwd_f32(const float* g, const float* y, float* dx,
                        int64_t rows, int64_t cols, void* stream);

/* y = (x - mean) * rstd * w + b per row; mean/rstd [rows] are written when both
 * are non-NULL.  Replaces layernorm_cuda and layernorm_with_stats_cuda
 * (cppsrc/ops/layernorm.cpp:12-14). */
int aar_layernorm_fwd_f32(const float* x, const float* w, const float* b,
                          float* y, float* mean, float* rstd,
                          int64_t rows, int64_t cols, float eps, void* stream);

/* Workspace for aar_layernorm_bwd_f32: the dgamma/dbeta partial rows of its
 * persistent workgroups (parts x 2 x cols floats; covers both load paths). */
size_t aar_layernorm_bwd_workspace_bytes(int64_t rows, int64_t cols);

/* dx [rows,cols], dw and db [cols] (fully overwritten; deterministic two-stage
 * column reduction through `workspace`).  Replaces layernorm_backward_cuda
 * (cppsrc/ops/layernorm.cpp:15-17). */
int aar_layernorm_bwd_f32(const float* gy, const float* x, const float* w,
                          const float* mean, const float* rstd,
                          float* dx, float* dw, float* db,
                          int64_t rows, int64_t cols,
                          void* workspace, size_t workspace_bytes, void* stream);

/* aar_layernorm_bwd_f32 with the input gradient added onto `dx_addend`
 * ([rows, cols] contiguous; may be dx itself): dx = dx_addend + the layernorm
 * input gradient, bit-identical to aar_layernorm_bwd_f32 followed by
 * aar_add_f32(dx_addend, dx).  dw and db as there.  Replaces the
 * layernorm_backward_cuda + add_cuda pair of a gradient fan-in: the autograd
 * sum of a layernorm input that also feeds a residual connection
 * (cppsrc/ops/layernorm.cpp:15-17, cppsrc/autograd/backward.cpp:17-36). */
int aar_layernorm_bwd_acc_f32(const float* gy, const float* x, const float* w,
                              const float* mean, const float* rstd, const float* dx_addend,
                              float* dx, float* dw, float* db,
                              int64_t rows, int64_t cols,
                              void* workspace, size_t workspace_bytes, void* stream);

/* No counterpart in the reference: aar_layernorm_bwd_f32 for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The dgamma/dbeta partial rows go
 * to a static per-GPU device buffer of aar_layernorm_bwd_noalloc_max_bytes()
 * (16 MiB, held by each GPU the library runs on until the process ends)
 * instead of a caller workspace; the call allocates nothing (no hipMalloc,
 * no allocating library routine).  Same kernels and results as
 * aar_layernorm_bwd_f32, bit for bit.  A shape whose partial rows exceed
 * the buffer returns AAR_ESCRATCH before any launch.  The partial rows number
 * CUs x resident workgroups, so the limits scale with the device: on
 * MI355X's 256 CUs, with 16-byte aligned operands and a column count
 * divisible by 4, any number of rows fits up to 4096 columns; unaligned
 * operands or other column counts take the element-wise plan, which fits up
 * to 2048 columns (a device with more CUs fits proportionally fewer).  Every
 * call on one GPU shares that GPU's buffer: calls that overlap on one GPU
 * (several streams or host threads at once) race and must be serialised by
 * the caller; calls ordered on one stream are safe. */
size_t aar_layernorm_bwd_noalloc_max_bytes(void);
int aar_layernorm_bwd_noalloc_f32(const float* gy, const float* x, const float* w,
                                  const float* mean, const float* rstd,
                                  float* dx, float* dw, float* db,
                                  int64_t rows, int64_t cols, void* stream);

/* ------------------------------------------------------- flash attention */

/* O = softmax(scale * Q K^T [+ causal mask]) V and lse = m + ln(l) per query
 * row; q,k,v,o [bh, T, d], lse [bh, T].  d <= 128 (d % 4 == 0 for the MFMA
 * path).  Replaces flash_attention_forward_cuda
 * (cppsrc/ops/flash_attention.cpp:15-16). */
int aar_flash_fwd_f32(const float* q, const float* k, const float* v,
                      float* o, float* lse, int64_t bh, int64_t T, int64_t d,
                      int causal, float scale, void* stream);

/* Minimum workspace for aar_flash_bwd_f32 / _strided_f32: the D = rowsum(dO*O)
 * rows, bh x T floats (the recompute path). */
size_t aar_flash_bwd_workspace_bytes(int64_t bh, int64_t T, int64_t d);
/* Workspace that also holds every dS tile of the dK/dV pass (a 32x32 float
 * tile per query/key tile pair with work: bh * n(n+1)/2 tiles causal, bh * n^2
 * otherwise, n = ceil(T/32); 3.2 GB for causal bh=96, T=4096).  Given at
 * least this much, aar_flash_bwd_f32 / _strided_f32 compute dQ from the stored
 * tiles instead of recomputing P and dP; with less (but at least
 * aar_flash_bwd_workspace_bytes) they recompute.  No counterpart in the
 * reference, whose backward keeps no workspace. */
size_t aar_flash_bwd_fast_workspace_bytes(int64_t bh, int64_t T, int64_t d, int causal);

/* dq, dk, dv [bh, T, d] (fully overwritten; no float atomics).  Replaces
 * flash_attention_backward_cuda (cppsrc/ops/flash_attention.cpp:18-22). */
int aar_flash_bwd_f32(const float* q, const float* k, const float* v,
                      const float* o, const float* lse, const float* dout,
                      float* dq, float* dk, float* dv,
                      int64_t bh, int64_t T, int64_t d, int causal, float scale,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Strided forms of the two calls above, for q/k/v views of a packed
 * [B, T, 3, H, d] projection and outputs in [B, T, H, d] order (the
 * MultiHeadAttention views of aargrad/nn.py:177-189, which the reference
 * copies to contiguous tensors first, cppsrc/ops/shape.cpp:244-274).  Every
 * [B, H, T, d] operand X has element (b, h, t, c) at
 *   X[b*sb + h*sh + t*st + c]      (element strides, head dim contiguous)
 * and `strides` lists (sb, sh, st) per operand: 12 values for the forward
 * (q, k, v, o), 24 for the backward (q, k, v, o, dout, dq, dk, dv).  lse and
 * the workspace are contiguous [B*H, T].  128-bit paths need 16-byte aligned
 * pointers and d and all strides multiples of 4; other layouts take the
 * element-wise path.  The unstrided calls are these with contiguous strides
 * (the forward with no workspace). */
int aar_flash_fwd_strided_f32(const float* q, const float* k, const float* v,
                              float* o, float* lse, int64_t B, int64_t H,
                              int64_t T, int64_t d, const int64_t* strides,
                              int causal, float scale,
                              void* workspace, size_t workspace_bytes, void* stream);
/* Workspace for the causal strided forward's key-range split (0 when the shape
 * never splits; shape-only, no device needed).  With at least this much
 * (16-byte aligned) and a grid of at most one round of resident workgroups,
 * the longest half of the query blocks each run as two workgroups over the two
 * halves of their key range, merged by a combine pass; with less, or a null
 * workspace, every block is one workgroup.  Same results up to rounding.  No
 * counterpart in the reference, whose forward keeps no workspace. */
size_t aar_flash_fwd_workspace_bytes(int64_t bh, int64_t T, int64_t d, int causal);
int aar_flash_bwd_strided_f32(const float* q, const float* k, const float* v,
                              const float* o, const float* lse, const float* dout,
                              float* dq, float* dk, float* dv,
                              int64_t B, int64_t H, int64_t T, int64_t d,
                              const int64_t* strides, int causal, float scale,
                              void* workspace, size_t workspace_bytes, void* stream);

/* Plans the flash calls would take on the current device (tuning and tests;
 * no counterpart in the reference, whose kernels have one launch shape,
 * cppsrc/ops/flash_attention.cu:227-280).  vec: 1 when the operands take the
 * 128-bit path (16-byte aligned, d and all strides multiples of 4).
 * aar_flash_fwd_plan: query blocks per head that the causal strided forward
 * splits over two workgroups given `workspace_bytes` of workspace (0: none).
 * aar_flash_bwd_plan: keys per dK/dV workgroup, 64 (the paired kernel: two
 * query phases per key tile, for grids of about one round) or 128.
 * aar_flash_fwd_query_block: queries per forward workgroup, 64 (the paired
 * kernel: two key phases per query tile, for causal grids of up to two
 * rounds of resident 128-query workgroups, four when T <= 1024) or 128; when
 * it is 64 the forward does not split and aar_flash_fwd_plan's count does not
 * apply.  The library keeps no plan state: these are pure functions of the
 * shape and the device. */
int aar_flash_fwd_plan(int64_t bh, int64_t T, int64_t d, int causal, int vec, size_t workspace_bytes,
                       int* split_blocks);
int aar_flash_bwd_plan(int64_t bh, int64_t T, int64_t d, int causal, int vec, int* key_block);
int aar_flash_fwd_query_block(int64_t bh, int64_t T, int64_t d, int causal, int vec, int* query_block);

/* The strided calls with the plan forced for this call only (tuning and
 * tests; no counterpart in the reference).  query_block / key_block: 64 or
 * 128 forces the forward's queries per workgroup / the backward's keys per
 * dK/dV workgroup, 0 takes the planner's choice (the plain strided calls pass
 * 0); other values are AAR_EINVAL.  Only shapes that can take either plan are
 * forced (causal d = 64 with 128-bit operands for the forward, d = 64 with
 * 128-bit operands for the backward); others keep 128.  Calls on other
 * threads are unaffected. */
int aar_flash_fwd_strided_plan_f32(const float* q, const float* k, const float* v,
                                   float* o, float* lse, int64_t B, int64_t H,
                                   int64_t T, int64_t d, const int64_t* strides,
                                   int causal, float scale, int query_block,
                                   void* workspace, size_t workspace_bytes, void* stream);
int aar_flash_bwd_strided_plan_f32(const float* q, const float* k, const float* v,
                                   const float* o, const float* lse, const float* dout,
                                   float* dq, float* dk, float* dv,
                                   int64_t B, int64_t H, int64_t T, int64_t d,
                                   const int64_t* strides, int causal, float scale, int key_block,
                                   void* workspace, size_t workspace_bytes, void* stream);

/* Strided fp32 copy of an ndim <= 8 view: dst[idx] = src[idx] for every index
 * of `shape`, element offsets given by the two stride arrays (host arrays, read
 * during the call).  Replaces contiguous_cuda / copy_contiguous_into_strided_cuda
 * (cppsrc/ops/shape.cpp:11-12); no per-call device allocation. */
int aar_strided_copy_f32(const float* src, float* dst, int ndim, const int64_t* shape,
                         const int64_t* src_strides, const int64_t* dst_strides, void* stream);

/* ------------------------------------------------------------ elementwise */

/* c = a + b over n floats: the device leg of add_grads.  Replaces add_cuda
 * (cppsrc/autograd/backward.cpp:14, cppsrc/ops/elementwise.cu:107-118). */
int aar_add_f32(const float* a, const float* b, float* c, int64_t n, void* stream);

/* ------------------------------------------- GPT-step ops around the path */
/* Elementwise over n floats; outputs may alias inputs.  Replace the reference
 * device legs sub_cuda / mul_cuda / scale_cuda / neg_cuda / relu_cuda /
 * relu_backward_cuda / gelu_cuda / gelu_backward_cuda / fill_cuda /
 * scaled_add_inplace_cuda (cppsrc/ops/elementwise.cpp:13-26, kernels
 * cppsrc/ops/elementwise.cu:16-72). */
int aar_sub_f32(const float* a, const float* b, float* c, int64_t n, void* stream);      /* c = a - b */
int aar_mul_f32(const float* a, const float* b, float* c, int64_t n, void* stream);      /* c = a * b */
int aar_scale_f32(const float* x, float* y, float alpha, int64_t n, void* stream);       /* y = alpha * x */
int aar_neg_f32(const float* x, float* y, int64_t n, void* stream);                      /* y = -x */
int aar_relu_f32(const float* x, float* y, int64_t n, void* stream);                     /* y = max(0, x) */
int aar_relu_bwd_f32(const float* g, const float* x, float* dx, int64_t n, void* stream);/* dx = x > 0 ? g : 0 */
int aar_gelu_f32(const float* x, float* y, int64_t n, void* stream);                     /* exact (erf) GELU */
int aar_gelu_bwd_f32(const float* g, const float* x, float* dx, int64_t n, void* stream);
int aar_fill_f32(float* y, float value, int64_t n, void* stream);
int aar_scaled_add_f32(float* dst, const float* src, float alpha, int64_t n, void* stream); /* dst += alpha*src (SGD) */

/* y[r][c] = x[r][c] + bias[c].  Replaces add_bias_cuda (cppsrc/ops/elementwise.cpp:24). */
int aar_add_bias_f32(const float* x, const float* bias, float* y, int64_t rows, int64_t cols, void* stream);

/* out[c] = sum_r g[r][c], deterministic two-stage tree.  Replaces bias_grad_cuda
 * (cppsrc/ops/elementwise.cpp:25, atomicAdd kernel elementwise.cu:79-82). */
size_t aar_colsum_workspace_bytes(int64_t rows, int64_t cols);
int aar_colsum_f32(const float* g, float* out, int64_t rows, int64_t cols,
                   void* workspace, size_t workspace_bytes, void* stream);
/* dx = x > 0 ? g : 0 over [rows, cols] and colsum[c] = sum over rows of
 * dx[r][c] in one pass over g, x and dx: the relu backward followed by the
 * bias-gradient column sum of the layer below it, bit-identical to
 * aar_relu_bwd_f32 then aar_colsum_f32 (the same row chunks summed in the same
 * order; workspace as aar_colsum_workspace_bytes).  Replaces
 * relu_backward_cuda + bias_grad_cuda of the MLP's first layer
 * (cppsrc/ops/elementwise.cpp:17, :25). */
int aar_relu_bwd_colsum_f32(const float* g, const float* x, float* dx, float* colsum, int64_t rows,
                            int64_t cols, void* workspace, size_t workspace_bytes, void* stream);

/* out[0] = sum of n floats, deterministic two-stage tree.  Replaces sum_all_cuda
 * (cppsrc/ops/elementwise.cpp:16, single-block kernel elementwise.cu:84-100). */
size_t aar_sum_workspace_bytes(int64_t n);
int aar_sum_f32(const float* x, float* out, int64_t n, void* workspace, size_t workspace_bytes, void* stream);

/* out[i][:] = w[ids[i]][:], w [vocab, dim], ids int64 [n].  An id outside
 * [0, vocab) yields a zero row and sets *err = 1 (err may be NULL).
 * Replaces embedding_cuda (cppsrc/ops/embedding.cpp:9). */
int aar_embedding_fwd_f32(const float* w, const int64_t* ids, float* out, int64_t n, int64_t vocab,
                          int64_t dim, int* err, void* stream);
/* out[i][:] = w1[ids1[i]][:] + w2[ids2[i]][:] (both tables [vocab_k, dim]): two
 * lookups and their sum in one pass, bit-identical to two
 * aar_embedding_fwd_f32 calls then aar_add_f32 (an id out of range gives a
 * zero row and sets *err = 1).  Replaces embedding_cuda x2 + add_cuda of the
 * GPT's token + position embeddings (cppsrc/ops/embedding.cpp:9,
 * elementwise.cpp:13; python/shakespeare/scripts/model.py:53). */
int aar_embedding_add_fwd_f32(const float* w1, const int64_t* ids1, int64_t vocab1, const float* w2,
                              const int64_t* ids2, int64_t vocab2, float* out, int64_t n, int64_t dim, int* err,
                              void* stream);

/* dw[vocab, dim] = onehot(ids)^T . g[n, dim] on matrix cores (deterministic;
 * AAR_EUNSUPPORTED when n*vocab > 2^30).  Up to 260 rows (dim % 4 == 0, g
 * 16-byte aligned) the one-hot values are made from the ids in registers by
 * the short-M GEMM kernel; larger vocabularies build the one-hot matrix in
 * the workspace and run the tiled GEMM.  Replaces embedding_backward_cuda
 * (cppsrc/ops/embedding.cpp:10-11, atomicAdd kernel embedding.cu:19-26). */
size_t aar_embedding_bwd_workspace_bytes(int64_t n, int64_t vocab, int64_t dim);
int aar_embedding_bwd_f32(const float* g, const int64_t* ids, float* dw, int64_t n, int64_t vocab,
                          int64_t dim, void* workspace, size_t workspace_bytes, void* stream);

/* Token-window batch from an int64 token stream on the device:
 * x[b][t] = tokens[starts[b] + t], y[b][t] = tokens[starts[b] + t + 1] for
 * b < batch, t < seq_len.  A start outside [0, n_tokens - seq_len - 1] yields
 * zero rows and sets *err = 1 (err may be NULL).  Replaces the host-side
 * window gather, collate and batch copy of TokenWindowDataset.__getitem__ /
 * default_collate / to_device_batch (python/shakespeare/scripts/data.py:38-53,
 * train.py:99-102). */
int aar_token_windows_i64(const int64_t* tokens, int64_t n_tokens, const int64_t* starts, int64_t batch,
                          int64_t seq_len, int64_t* x, int64_t* y, int* err, void* stream);

/* Mean cross entropy over rows whose target != ignore_index; logits [n, vocab],
 * targets int64 [n], loss a device scalar.  A target outside [0, vocab) (and not
 * ignore_index) sets *err = 1 and the row is skipped.  Replaces
 * cross_entropy_cuda / cross_entropy_backward_cuda (cppsrc/ops/cross_entropy.cpp:8-14). */
size_t aar_cross_entropy_workspace_bytes(int64_t n);
int aar_cross_entropy_fwd_f32(const float* logits, const int64_t* targets, float* loss, int64_t n,
                              int64_t vocab, int64_t ignore_index, int* err,
                              void* workspace, size_t workspace_bytes, void* stream);
/* dlogits = (softmax(logits) - onehot(target)) * grad[0] / active, zero rows for
 * ignored targets; grad is a device scalar (no host round trip). */
int aar_cross_entropy_bwd_f32(const float* grad, const float* logits, const int64_t* targets,
                              float* dlogits, int64_t n, int64_t vocab, int64_t ignore_index,
                              void* workspace, size_t workspace_bytes, void* stream);

/* Fused AdamW step over n floats (param, m, v updated in place).  Replaces
 * adamw_step_cuda (cppsrc/ops/adamw.cpp:6-10, kernel adamw.cu:11-27). */
int aar_adamw_f32(float* param, const float* grad, float* m, float* v, int64_t n, float lr,
                  float beta1, float beta2, float eps, float weight_decay,
                  float bias_correction1, float bias_correction2, void* stream);

/* Multi-tensor optimizer updates: tensor i has n[i] floats at dst[i]/src[i]
 * (param[i], grad[i], m[i], v[i]); up to 48 tensors go in one launch, their
 * pointers passed by value in the kernel arguments.  Element for element the
 * same arithmetic as aar_scaled_add_f32 / aar_adamw_f32, so results are
 * bit-identical to calling those per tensor.  They replace the per-parameter
 * loops of the reference optimizers: SGD.step calling scaled_add_inplace
 * (aargrad/optim.py:13-18) and AdamW.step calling adamw_step
 * (aargrad/optim.py:36-54), one launch per parameter there. */
int aar_scaled_add_multi_f32(int count, float* const* dst, const float* const* src, const int64_t* n,
                             float alpha, void* stream);
int aar_adamw_multi_f32(int count, float* const* param, const float* const* grad, float* const* m,
                        float* const* v, const int64_t* n, float lr, float beta1, float beta2, float eps,
                        float weight_decay, float bias_correction1, float bias_correction2, void* stream);

/* Dropout over n floats with the reference's counter-based stream: element i
 * keeps iff philox_uniform(seed, i) >= p (Philox-4x32-10, word 0 / 2^32);
 * mask[i] = keep ? 1/(1-p) : 0, out[i] = x[i] * mask[i].  Bit-identical to the
 * reference CPU path for the same seed.  0 <= p < 1.  Replaces dropout_cuda
 * (cppsrc/ops/dropout.cpp:14-15, kernel dropout.cu:8-18). */
int aar_dropout_f32(const float* x, float* out, float* mask, int64_t n, float p, uint64_t seed,
                    void* stream);

/* y[m][i][j] = (j <= i) ? x[m][i][j] : fill over `mats` contiguous [T, T]
 * matrices; fill = -inf is apply_causal_mask, fill = 0 its backward.
 * Replaces apply_causal_mask_cuda / causal_mask_backward_cuda
 * (cppsrc/ops/attention.cpp:10-11). */
int aar_causal_mask_f32(const float* x, float* y, int64_t mats, int64_t T, float fill,
                        void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif /* AAR_HIP_H */
