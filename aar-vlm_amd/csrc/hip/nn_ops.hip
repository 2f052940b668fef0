// Device ops of the GPT training step around the hot path (elementwise
// family, bias add/grad, reductions, embedding, cross entropy).  Reference
// semantics:
//   sub/mul/scale/neg/relu/gelu/add_bias/bias_grad/sum_all/fill/scaled_add
//                              cppsrc/ops/elementwise.cpp:44-474, elementwise.cu:11-276
//   embedding fwd/bwd          cppsrc/ops/embedding.cpp:9-104
//   cross_entropy fwd/bwd      cppsrc/ops/cross_entropy.cpp:15-152
// Design:
//  * Streaming elementwise kernels: 128-bit loads/stores, one thread per
//    4-float unit over a grid that covers the data once, one templated body
//    per op.
//  * Every reduction is a fixed-order two-stage tree (bias_grad = column sums,
//    sum_all, cross-entropy mean), so results are bit-reproducible; the
//    reference uses float atomicAdd for bias_grad and embedding backward.
//  * Embedding backward is dW = onehot(ids)^T . dY on matrix cores:
//    deterministic, and at the vocabularies of the GPT step (65, 256) far
//    cheaper than atomics into a few hot rows.  Up to 260 rows it runs the
//    short-M TN kernel (gemm_small.hip), which makes the one-hot values from
//    the ids in registers and skips row blocks absent from a tile; larger
//    vocabularies build the one-hot matrix and run the tiled GEMM.
//  * Out-of-range ids/targets cannot throw on the device: the kernels write
//    zeros for such rows (never reading out of bounds) and raise a flag in a
//    caller-provided int that the host checks at its next synchronisation.
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

#include "colsum.hpp"
#include "common.hpp"
#include "gemm_small.hpp"

namespace aar {
namespace {

// One thread per work item (a 4-float unit for the vector kernels): a grid
// that covers the data once streams HBM measurably faster on MI355X than a
// persistent grid-stride loop (the dispatcher walks the blocks in address
// order, so the in-flight accesses form one compact window).  Past 2^20
// blocks the kernels' grid-stride loops take over.
unsigned stream_grid(int64_t work) {
  constexpr int64_t kCap = int64_t(1) << 20;
  int64_t g = (work + 255) / 256;
  if (g > kCap) g = kCap;
  return (unsigned)(g > 0 ? g : 1);
}

// ---------------------------------------------------------------- elementwise

enum class Ew { Sub, Mul, Scale, Neg, Relu, ReluBwd, Gelu, GeluBwd, Fill, ScaledAdd };

constexpr float kInvSqrt2 = 0.70710678118654752440f;
constexpr float kInvSqrt2Pi = 0.39894228040143267794f;

template <Ew OP>
__device__ __forceinline__ float ew(float a, float b, float alpha) {
  switch (OP) {
    case Ew::Sub: return a - b;
    case Ew::Mul: return a * b;
    case Ew::Scale: return alpha * a;
    case Ew::Neg: return -a;
    case Ew::Relu: return fmaxf(0.0f, a);
    case Ew::ReluBwd: return b > 0.0f ? a : 0.0f;  // a = grad, b = x
    case Ew::Gelu: return 0.5f * a * (1.0f + erff(a * kInvSqrt2));
    case Ew::GeluBwd: {  // a = grad, b = x
      const float cdf = 0.5f * (1.0f + erff(b * kInvSqrt2));
      const float pdf = kInvSqrt2Pi * expf(-0.5f * b * b);
      return a * (cdf + b * pdf);
    }
    case Ew::Fill: return alpha;
    case Ew::ScaledAdd: return a + alpha * b;  // a = dst, b = src
  }
  return 0.f;
}

template <Ew OP>
__global__ void __launch_bounds__(256)
ew_vec_kernel(const f32x4* __restrict__ a, const f32x4* __restrict__ b, f32x4* __restrict__ c, float alpha,
              int64_t n4) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    f32x4 x = {0.f, 0.f, 0.f, 0.f}, y = {0.f, 0.f, 0.f, 0.f};
    if (OP != Ew::Fill) x = a[i];
    if (OP == Ew::Sub || OP == Ew::Mul || OP == Ew::ReluBwd || OP == Ew::GeluBwd || OP == Ew::ScaledAdd) y = b[i];
    f32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = ew<OP>(x[e], y[e], alpha);
    c[i] = r;
  }
}

template <Ew OP>
__global__ void __launch_bounds__(256)
ew_scalar_kernel(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ c, float alpha,
                 int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float x = OP != Ew::Fill ? a[i] : 0.f;
    const float y = (OP == Ew::Sub || OP == Ew::Mul || OP == Ew::ReluBwd || OP == Ew::GeluBwd ||
                     OP == Ew::ScaledAdd)
                        ? b[i]
                        : 0.f;
    c[i] = ew<OP>(x, y, alpha);
  }
}

template <Ew OP>
int launch_ew(const float* a, const float* b, float* c, float alpha, int64_t n, void* stream) {
  if (n < 0) return AAR_EINVAL;
  if (n == 0) return AAR_OK;
  const bool needs_a = OP != Ew::Fill;
  const bool needs_b = OP == Ew::Sub || OP == Ew::Mul || OP == Ew::ReluBwd || OP == Ew::GeluBwd ||
                       OP == Ew::ScaledAdd;
  if (!c || (needs_a && !a) || (needs_b && !b)) return AAR_EINVAL;
  hipStream_t st = as_stream(stream);
  const bool vec = aligned16(c) && (!needs_a || aligned16(a)) && (!needs_b || aligned16(b));
  if (vec) {
    const int64_t n4 = n / 4;
    if (n4 > 0) {
      ew_vec_kernel<OP><<<dim3(stream_grid(n4)), dim3(256), 0, st>>>(
          reinterpret_cast<const f32x4*>(a), reinterpret_cast<const f32x4*>(b), reinterpret_cast<f32x4*>(c),
          alpha, n4);
      const int rc = launch_status();
      if (rc != AAR_OK) return rc;
    }
    const int64_t done = n4 * 4;
    if (done < n)
      ew_scalar_kernel<OP><<<dim3(1), dim3(256), 0, st>>>(needs_a ? a + done : nullptr,
                                                           needs_b ? b + done : nullptr, c + done, alpha,
                                                           n - done);
  } else {
    ew_scalar_kernel<OP><<<dim3(stream_grid(n)), dim3(256), 0, st>>>(a, b, c, alpha, n);
  }
  return launch_status();
}

// ---------------------------------------------------------------- bias

// y[r][c] = x[r][c] + bias[c]
__global__ void __launch_bounds__(256)
add_bias_kernel(const float* __restrict__ x, const float* __restrict__ bias, float* __restrict__ y, int64_t n,
                int64_t cols) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) y[i] = x[i] + bias[i % cols];
}

__global__ void __launch_bounds__(256)
add_bias_vec_kernel(const f32x4* __restrict__ x, const f32x4* __restrict__ bias, f32x4* __restrict__ y,
                    int64_t n4, int64_t cols4) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) y[i] = x[i] + bias[i % cols4];
}

// Column sums, stage 1: part[p][c] = sum of g[r][c] for rows r in chunk p
// (rows r0 = p*chunk .. r0+chunk-1) as two running sums from 0.f, in row
// order: s0 over the rows with (r - r0) & 4 == 0, s1 over the others, then
// s0 + s1.  The two sets are the row sets of the two lane halves of a 32x32
// MFMA accumulator block (and of the A fragments of a TN product's K tile),
// so the GEMM paths holding 64-row chunks (kEpiMaskBits, kEpiColsumA,
// gemm_f32.hip) form the same partials with one exchange between the halves.
__global__ void __launch_bounds__(256)
colsum_stage1_kernel(const float* __restrict__ g, float* __restrict__ part, int64_t rows, int64_t cols,
                     int64_t chunk) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  const int64_t r0 = (int64_t)blockIdx.y * chunk;
  const int64_t r1 = min(rows, r0 + chunk);
  float s0 = 0.f, s1 = 0.f;
#pragma unroll 8
  for (int64_t r = r0; r < r1; ++r) {
    const float v = g[r * cols + c];
    if ((r - r0) & 4) {
      s1 += v;
    } else {
      s0 += v;
    }
  }
  part[(int64_t)blockIdx.y * cols + c] = s0 + s1;
}

// Stage 1 fused with the relu backward that produces g: dx = x > 0 ? g : 0
// is stored and summed in the same order as colsum_stage1_kernel sums dx, so
// the partials are bit for bit those of the two kernels in sequence.  Each
// thread owns 4 consecutive columns (128-bit accesses; cols % 4 == 0 and
// 16-byte aligned rows), a workgroup 1024 columns of one row chunk.
__global__ void __launch_bounds__(256)
relu_bwd_colsum_stage1_kernel(const f32x4* __restrict__ g, const f32x4* __restrict__ x, f32x4* __restrict__ dx,
                              float* __restrict__ part, int64_t rows, int64_t cols4, int64_t chunk) {
  const int64_t c4 = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c4 >= cols4) return;
  const int64_t r0 = (int64_t)blockIdx.y * chunk;
  const int64_t r1 = min(rows, r0 + chunk);
  f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
  for (int64_t r = r0; r < r1; ++r) {
    const f32x4 gv = __builtin_nontemporal_load(g + r * cols4 + c4);
    const f32x4 xv = __builtin_nontemporal_load(x + r * cols4 + c4);
    f32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = xv[e] > 0.0f ? gv[e] : 0.0f;
    __builtin_nontemporal_store(v, dx + r * cols4 + c4);
    if ((r - r0) & 4) {
      s1 += v;
    } else {
      s0 += v;
    }
  }
  *reinterpret_cast<f32x4*>(part + (int64_t)blockIdx.y * cols4 * 4 + c4 * 4) = s0 + s1;
}

// Stage 2: out[c] = sum over p of part[p][c] (colsum_stage2_block: a
// workgroup owns kCsCols columns and kColsumSlices slices of the parts, a
// slice sums its run of parts in order, a fixed tree finishes each column).
// Deterministic; one thread per column and part run instead of one per
// column keeps the few-column case off the latency floor.
constexpr int kCsCols = 16;
constexpr int kCsThreads = kColsumSlices * kCsCols;

__global__ void __launch_bounds__(kCsThreads)
colsum_stage2_kernel(const float* __restrict__ part, float* __restrict__ out, int nparts, int64_t cols) {
  __shared__ float acc[kColsumSlices][kCsCols];
  colsum_stage2_block<kCsCols>(part, out, nparts, cols, (int64_t)blockIdx.x * kCsCols, acc);
}

int colsum_parts(int64_t rows) {
  const int64_t p = ceil_div(rows, 64);
  return (int)(p < 256 ? (p > 0 ? p : 1) : 256);
}

// ---------------------------------------------------------------- sum_all

constexpr int kSumBlocks = 256;

// Stage 1: block b sums elements [b*chunk, (b+1)*chunk) (thread-strided,
// then a fixed-shape block tree); stage 2 sums the block partials in order.
__global__ void __launch_bounds__(256)
sum_stage1_kernel(const float* __restrict__ x, float* __restrict__ part, int64_t n, int64_t chunk) {
  __shared__ float red[4];
  const int64_t b0 = (int64_t)blockIdx.x * chunk;
  const int64_t b1 = min(n, b0 + chunk);
  float s = 0.f;
  for (int64_t i = b0 + threadIdx.x; i < b1; i += 256) s += x[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = ((red[0] + red[1]) + red[2]) + red[3];
}

__global__ void __launch_bounds__(256)
sum_stage2_kernel(const float* __restrict__ part, float* __restrict__ out, int nparts) {
  __shared__ float red[4];
  float s = threadIdx.x < nparts ? part[threadIdx.x] : 0.f;
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) out[0] = ((red[0] + red[1]) + red[2]) + red[3];
}

// ---------------------------------------------------------------- embedding

// out[i][:] = w[ids[i]][:]; an out-of-range id writes a zero row and sets *err.
__global__ void __launch_bounds__(256)
embedding_fwd_kernel(const float* __restrict__ w, const int64_t* __restrict__ ids, float* __restrict__ out,
                     int64_t n, int64_t vocab, int64_t dim, int* __restrict__ err) {
  const int64_t total = n * dim;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
    const int64_t i = e / dim, k = e - i * dim;
    const int64_t id = ids[i];
    float v = 0.f;
    if (id >= 0 && id < vocab) {
      v = w[id * dim + k];
    } else if (k == 0 && err) {
      *err = 1;
    }
    out[e] = v;
  }
}

// The same with one wave per row and 128-bit accesses (dim % 4 == 0,
// 16-byte aligned w and out): the row's id is read once, lanes stride over
// the row's float4 columns.
__global__ void __launch_bounds__(256)
embedding_fwd_vec_kernel(const f32x4* __restrict__ w, const int64_t* __restrict__ ids, f32x4* __restrict__ out,
                         int64_t n, int64_t vocab, int64_t dim4, int* __restrict__ err) {
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (i >= n) return;
  const int64_t id = ids[i];
  const bool ok = id >= 0 && id < vocab;
  if (!ok && lane == 0 && err) *err = 1;
  const f32x4* src = w + (ok ? id : 0) * dim4;
  f32x4* dst = out + i * dim4;
  for (int64_t k = lane; k < dim4; k += 64) {
    const f32x4 v = ok ? src[k] : f32x4{0.f, 0.f, 0.f, 0.f};
    __builtin_nontemporal_store(v, dst + k);
  }
}

// Two lookups and their sum, out[i] = w1[ids1[i]] + w2[ids2[i]] (the token +
// position embeddings of a GPT): each table row as embedding_fwd reads it (a
// zero row for an id out of range, which sets *err), then one fp32 add, so
// the result is bit for bit the two lookups followed by an add, with one
// write of the sum instead of two rows written and read back.
__global__ void __launch_bounds__(256)
embedding_add_fwd_vec_kernel(const f32x4* __restrict__ w1, const int64_t* __restrict__ ids1, int64_t vocab1,
                             const f32x4* __restrict__ w2, const int64_t* __restrict__ ids2, int64_t vocab2,
                             f32x4* __restrict__ out, int64_t n, int64_t dim4, int* __restrict__ err) {
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (i >= n) return;
  const int64_t id1 = ids1[i], id2 = ids2[i];
  const bool ok1 = id1 >= 0 && id1 < vocab1, ok2 = id2 >= 0 && id2 < vocab2;
  if ((!ok1 || !ok2) && lane == 0 && err) *err = 1;
  const f32x4* s1 = w1 + (ok1 ? id1 : 0) * dim4;
  const f32x4* s2 = w2 + (ok2 ? id2 : 0) * dim4;
  f32x4* dst = out + i * dim4;
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  for (int64_t k = lane; k < dim4; k += 64) {
    const f32x4 a = ok1 ? s1[k] : z, b = ok2 ? s2[k] : z;
    __builtin_nontemporal_store(a + b, dst + k);
  }
}

__global__ void __launch_bounds__(256)
embedding_add_fwd_kernel(const float* __restrict__ w1, const int64_t* __restrict__ ids1, int64_t vocab1,
                         const float* __restrict__ w2, const int64_t* __restrict__ ids2, int64_t vocab2,
                         float* __restrict__ out, int64_t n, int64_t dim, int* __restrict__ err) {
  const int64_t total = n * dim;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
    const int64_t i = e / dim, k = e - i * dim;
    const int64_t id1 = ids1[i], id2 = ids2[i];
    const bool ok1 = id1 >= 0 && id1 < vocab1, ok2 = id2 >= 0 && id2 < vocab2;
    if ((!ok1 || !ok2) && k == 0 && err) *err = 1;
    const float a = ok1 ? w1[id1 * dim + k] : 0.f, b = ok2 ? w2[id2 * dim + k] : 0.f;
    out[e] = a + b;
  }
}

// onehot[i][v] = (ids[i] == v)  (row-major [n, vocab])
__global__ void __launch_bounds__(256)
onehot_kernel(const int64_t* __restrict__ ids, float* __restrict__ oh, int64_t n, int64_t vocab) {
  const int64_t total = n * vocab;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
    const int64_t i = e / vocab, v = e - i * vocab;
    oh[e] = ids[i] == v ? 1.0f : 0.0f;
  }
}

// --------------------------------------------------------------- cross entropy

// Row loss: lse(row) - row[t] (0 for ignored rows), active flag 1/0; one wave
// per row, lanes strided over the vocabulary.  Mirrors cross_entropy_cpu's
// float arithmetic (max, sum of exp(x - max), m + log(s)).
__global__ void __launch_bounds__(256)
ce_row_kernel(const float* __restrict__ L, const int64_t* __restrict__ T, float* __restrict__ row_loss,
              int* __restrict__ active, int64_t n, int64_t V, int64_t ignore_index, int* __restrict__ err) {
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (i >= n) return;
  const int64_t t = T[i];
  if (t == ignore_index) {
    if (lane == 0) {
      row_loss[i] = 0.f;
      active[i] = 0;
    }
    return;
  }
  if (t < 0 || t >= V) {
    if (lane == 0) {
      row_loss[i] = 0.f;
      active[i] = 0;
      if (err) *err = 1;
    }
    return;
  }
  const float* row = L + i * V;
  float m = -INFINITY;
  for (int64_t v = lane; v < V; v += 64) m = fmaxf(m, row[v]);
  m = wave_max(m);
  float s = 0.f;
  for (int64_t v = lane; v < V; v += 64) s += expf(row[v] - m);
  s = wave_sum(s);
  if (lane == 0) {
    row_loss[i] = (m + logf(s)) - row[t];
    active[i] = 1;
  }
}

// Mean over active rows and the active count: one workgroup of 1024 threads.
// Thread t sums rows t, t + 1024, ... in order (loss in double, count in
// int64), issuing a chunk's 16 loads before its first add; a wave butterfly
// and the 16 waves in order finish.  The order is fixed, so the result is
// deterministic.  Writes the float mean (0 when no row is active) and the
// count.
constexpr int kCeThreads = 1024;
constexpr int kCeChunk = 16;  // rows per thread whose loads are in flight together

template <typename T>
__device__ __forceinline__ T wave_sum_any(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__global__ void __launch_bounds__(kCeThreads)
ce_mean_kernel(const float* __restrict__ row_loss, const int* __restrict__ active, int64_t n,
               float* __restrict__ out, long long* __restrict__ count_out) {
  __shared__ double dsum[kCeThreads / 64];
  __shared__ long long csum[kCeThreads / 64];
  double s = 0.0;
  long long c = 0;
  for (int64_t base = 0; base < n; base += (int64_t)kCeThreads * kCeChunk) {
    float l[kCeChunk];
    int a[kCeChunk];
#pragma unroll
    for (int k = 0; k < kCeChunk; ++k) {
      const int64_t i = base + (int64_t)k * kCeThreads + threadIdx.x;
      l[k] = i < n ? row_loss[i] : 0.f;
      a[k] = i < n ? active[i] : 0;
    }
#pragma unroll
    for (int k = 0; k < kCeChunk; ++k) {
      s += (double)l[k];
      c += a[k];
    }
  }
  s = wave_sum_any(s);
  c = wave_sum_any(c);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    dsum[wave] = s;
    csum[wave] = c;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double ts = dsum[0];
    long long tc = csum[0];
    for (int w = 1; w < kCeThreads / 64; ++w) {
      ts += dsum[w];
      tc += csum[w];
    }
    out[0] = tc > 0 ? (float)(ts / (double)tc) : 0.0f;
    if (count_out) count_out[0] = tc;
  }
}

__global__ void __launch_bounds__(kCeThreads)
ce_count_kernel(const int64_t* __restrict__ T, int64_t n, int64_t ignore_index, long long* __restrict__ count) {
  __shared__ long long csum[kCeThreads / 64];
  long long c = 0;
  for (int64_t base = 0; base < n; base += (int64_t)kCeThreads * kCeChunk) {
    int64_t t[kCeChunk];
#pragma unroll
    for (int k = 0; k < kCeChunk; ++k) {
      const int64_t i = base + (int64_t)k * kCeThreads + threadIdx.x;
      t[k] = i < n ? T[i] : ignore_index;
    }
#pragma unroll
    for (int k = 0; k < kCeChunk; ++k) c += (t[k] != ignore_index) ? 1 : 0;
  }
  c = wave_sum_any(c);
  if ((threadIdx.x & 63) == 0) csum[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    long long tc = csum[0];
    for (int w = 1; w < kCeThreads / 64; ++w) tc += csum[w];
    count[0] = tc;
  }
}

// dL[i][v] = (softmax(row)[v] - [v == t]) * go / active, zeros for ignored
// (or out-of-range) rows.  Same float order as cross_entropy_backward_cpu.
__global__ void __launch_bounds__(256)
ce_bwd_kernel(const float* __restrict__ L, const int64_t* __restrict__ T, const float* __restrict__ grad,
              const long long* __restrict__ count, float* __restrict__ dL, int64_t n, int64_t V,
              int64_t ignore_index) {
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (i >= n) return;
  const int64_t t = T[i];
  float* drow = dL + i * V;
  const long long active = count[0];
  if (t == ignore_index || t < 0 || t >= V || active == 0) {
    for (int64_t v = lane; v < V; v += 64) drow[v] = 0.f;
    return;
  }
  const float scale = grad[0] / (float)active;
  const float* row = L + i * V;
  float m = -INFINITY;
  for (int64_t v = lane; v < V; v += 64) m = fmaxf(m, row[v]);
  m = wave_max(m);
  float s = 0.f;
  for (int64_t v = lane; v < V; v += 64) s += expf(row[v] - m);
  s = wave_sum(s);
  const float inv_s = 1.0f / s;
  for (int64_t v = lane; v < V; v += 64) {
    float d = (expf(row[v] - m) * inv_s) * scale;
    if (v == t) d -= scale;
    drow[v] = d;
  }
}

// ------------------------------------------------------------------- AdamW

// Same per-element arithmetic as adamw_step_cpu (cppsrc/ops/adamw.cpp:22-44).
// One AdamW element update (adamw.cu:11-50 arithmetic): m, v moments, bias
// corrections as divisors, decoupled weight decay as a factor on p.
__device__ __forceinline__ void adamw_elem(float& p, float g, float& m, float& v, float lr, float beta1, float beta2,
                                           float eps, float wd_factor, float bc1, float bc2) {
  const float mi = beta1 * m + (1.0f - beta1) * g;
  const float vi = beta2 * v + (1.0f - beta2) * g * g;
  m = mi;
  v = vi;
  const float m_hat = mi / bc1;
  const float v_hat = vi / bc2;
  p = p * wd_factor - lr * m_hat / (sqrtf(v_hat) + eps);
}

__global__ void __launch_bounds__(256)
adamw_kernel(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m, float* __restrict__ v,
             int64_t n, float lr, float beta1, float beta2, float eps, float wd_factor, float bc1, float bc2) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    adamw_elem(p[i], g[i], m[i], v[i], lr, beta1, beta2, eps, wd_factor, bc1, bc2);
}

// ------------------------------------------------------ multi-tensor update

// One launch updates up to kMultiMax tensors (an optimizer step over a
// model's parameters is otherwise one small launch per parameter).  Pointers
// and sizes travel by value in the kernel arguments; workgroup b works on
// tensor t with start[t] <= b < start[t + 1], elements
// [(b - start[t]) * kMultiChunk, +kMultiChunk).  The per-element arithmetic is
// that of the single-tensor kernels, so results are bit-identical to them.
constexpr int kMultiMax = 48;
constexpr int kMultiChunk = 4096;
struct MultiArgs {
  float* a[kMultiMax];        // dst / param
  const float* b[kMultiMax];  // src / grad
  float* m[kMultiMax];
  float* v[kMultiMax];
  int64_t n[kMultiMax];
  int start[kMultiMax + 1];
  int count;
};
static_assert(sizeof(MultiArgs) < 4096, "kernel arguments");

__device__ __forceinline__ int multi_tensor_of(const MultiArgs& A, int blk) {
  int t = 0;
  while (t + 1 < A.count && A.start[t + 1] <= blk) ++t;
  return t;
}

template <bool ADAMW>
__global__ void __launch_bounds__(256)
multi_update_kernel(MultiArgs A, float alpha, float lr, float beta1, float beta2, float eps, float wd_factor,
                    float bc1, float bc2) {
  const int t = multi_tensor_of(A, blockIdx.x);
  const int64_t i0 = (int64_t)(blockIdx.x - A.start[t]) * kMultiChunk;
  const int64_t i1 = min(A.n[t], i0 + kMultiChunk);
  float* a = A.a[t];  // may alias b (dst += alpha * dst)
  const float* b = A.b[t];
  int64_t tail = i0;  // first element left to the scalar loop
  if (!ADAMW && aligned16(a) && aligned16(b)) {
    // 128-bit accesses: thread x takes float4s x, x + 256, ... of the chunk,
    // every load issued before the first store (each element is read and
    // written by this thread only, so an aliased b still reads old values).
    // (AdamW keeps the scalar loop: in this form the compiler contracted its
    // update into FMAs differently from the single-tensor kernel, 1 ulp off.)
    constexpr int kU = kMultiChunk / (4 * 256);
    const int64_t q0 = i0 / 4, q1 = i1 / 4;  // whole float4s
    f32x4 pa[kU], pb[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t q = q0 + threadIdx.x + 256 * u;
      if (q < q1) {
        pa[u] = reinterpret_cast<const f32x4*>(a)[q];
        pb[u] = reinterpret_cast<const f32x4*>(b)[q];
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t q = q0 + threadIdx.x + 256 * u;
      if (q < q1) {
#pragma unroll
        for (int e = 0; e < 4; ++e) pa[u][e] = ew<Ew::ScaledAdd>(pa[u][e], pb[u][e], alpha);
        reinterpret_cast<f32x4*>(a)[q] = pa[u];
      }
    }
    tail = q1 * 4;
  }
  for (int64_t i = tail + threadIdx.x; i < i1; i += 256) {
    if (ADAMW)
      adamw_elem(a[i], b[i], A.m[t][i], A.v[t][i], lr, beta1, beta2, eps, wd_factor, bc1, bc2);
    else
      a[i] = ew<Ew::ScaledAdd>(a[i], b[i], alpha);
  }
}

// Byte ranges [p, p + n floats) overlap.
inline bool spans_overlap(const void* p, const void* q, int64_t n_p, int64_t n_q) {
  if (!p || !q) return false;
  const uintptr_t a0 = reinterpret_cast<uintptr_t>(p), b0 = reinterpret_cast<uintptr_t>(q);
  const uintptr_t a1 = a0 + (uintptr_t)n_p * sizeof(float), b1 = b0 + (uintptr_t)n_q * sizeof(float);
  return a0 < b1 && b0 < a1;
}

// Tensor `i` may join the group only if nothing it writes (a, m, v) overlaps
// anything a member reads or writes, and nothing it reads (b) overlaps what a
// member writes.  Workgroups of one launch run in no fixed order, so a
// parameter listed twice (a shared module, a tied weight) must be updated in
// two launches, one after the other, as the per-parameter loop does.
inline bool conflicts_with_group(const MultiArgs& A, bool adamw, float* a, const float* b, float* m, float* v,
                                 int64_t n) {
  for (int k = 0; k < A.count; ++k) {
    const int64_t nk = A.n[k];
    const void* written_k[3] = {A.a[k], adamw ? A.m[k] : nullptr, adamw ? A.v[k] : nullptr};
    const void* written_i[3] = {a, adamw ? m : nullptr, adamw ? v : nullptr};
    for (const void* wi : written_i) {
      if (spans_overlap(wi, A.b[k], n, nk)) return true;
      for (const void* wk : written_k)
        if (spans_overlap(wi, wk, n, nk)) return true;
    }
    for (const void* wk : written_k)
      if (spans_overlap(b, wk, n, nk)) return true;
  }
  return false;
}

// Launch groups of up to kMultiMax non-empty tensors whose written ranges are
// disjoint from every other member's ranges.
int launch_multi(bool adamw, int count, float* const* a, const float* const* b, float* const* m, float* const* v,
                 const int64_t* n, float alpha, float lr, float beta1, float beta2, float eps, float wd_factor,
                 float bc1, float bc2, hipStream_t st) {
  MultiArgs A{};
  int64_t blocks = 0;
  auto flush = [&]() -> int {
    if (A.count == 0) return AAR_OK;
    A.start[A.count] = (int)blocks;
    if (adamw)
      multi_update_kernel<true><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(A, alpha, lr, beta1, beta2, eps,
                                                                              wd_factor, bc1, bc2);
    else
      multi_update_kernel<false><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(A, alpha, lr, beta1, beta2, eps,
                                                                               wd_factor, bc1, bc2);
    const int rc = launch_status();
    A = MultiArgs{};
    blocks = 0;
    return rc;
  };
  for (int i = 0; i < count; ++i) {
    if (n[i] == 0) continue;
    const int64_t nb = ceil_div(n[i], (int64_t)kMultiChunk);
    if (A.count == kMultiMax || blocks + nb > INT32_MAX / 2 ||
        conflicts_with_group(A, adamw, a[i], b[i], adamw ? m[i] : nullptr, adamw ? v[i] : nullptr, n[i])) {
      const int rc = flush();
      if (rc != AAR_OK) return rc;
    }
    const int k = A.count++;
    A.a[k] = a[i];
    A.b[k] = b[i];
    A.m[k] = adamw ? m[i] : nullptr;
    A.v[k] = adamw ? v[i] : nullptr;
    A.n[k] = n[i];
    A.start[k] = (int)blocks;
    blocks += nb;
  }
  return flush();
}

// ---------------------------------------------------------------- dropout

// Philox-4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel Random Numbers: As
// Easy as 1, 2, 3", SC'11): counter (idx lo, idx hi, 0, 0), key (seed lo,
// seed hi), ten rounds with the Weyl key bump between rounds; the uniform is
// word 0 scaled by 2^-32 in float arithmetic, which is the stream the
// reference's dropout draws (cppsrc/core/rng.hpp:13-46).
__device__ __forceinline__ float philox_uniform(uint64_t seed, uint64_t idx) {
  uint32_t c0 = (uint32_t)idx, c1 = (uint32_t)(idx >> 32), c2 = 0u, c3 = 0u;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t lo0 = c0 * 0xD2511F53u, hi0 = __umulhi(c0, 0xD2511F53u);
    const uint32_t lo1 = c2 * 0xCD9E8D57u, hi1 = __umulhi(c2, 0xCD9E8D57u);
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return (float)c0 * (1.0f / 4294967296.0f);
}

// out = x * m, m = (u >= p ? 1/(1-p) : 0) with u the Philox uniform of the
// element's flat index (cppsrc/ops/dropout.cpp:30-42).  Four consecutive
// elements per thread with 128-bit accesses; the Philox rounds (10 per
// element, the reference keeps word 0 only) are the cost, not the bytes.
__global__ void __launch_bounds__(256)
dropout_vec_kernel(const f32x4* __restrict__ x, f32x4* __restrict__ out, f32x4* __restrict__ mask, int64_t n4,
                   float p, float scale, uint64_t seed) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < n4; u += stride) {
    const f32x4 v = x[u];
    f32x4 m;
#pragma unroll
    for (int k = 0; k < 4; ++k) m[k] = philox_uniform(seed, (uint64_t)(4 * u + k)) >= p ? scale : 0.0f;
    mask[u] = m;
    out[u] = v * m;
  }
}

// Elements [begin, n) one per thread: unaligned operands, or the n % 4 tail.
__global__ void __launch_bounds__(256)
dropout_kernel(const float* __restrict__ x, float* __restrict__ out, float* __restrict__ mask, int64_t begin,
               int64_t n, float p, float scale, uint64_t seed) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = begin + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float keep = philox_uniform(seed, (uint64_t)i) >= p ? scale : 0.0f;
    mask[i] = keep;
    out[i] = x[i] * keep;
  }
}

// ---------------------------------------------------------------- causal mask

// y[m][i][j] = j <= i ? x[m][i][j] : fill over [mats, T, T] (forward fill is
// -inf, backward 0; cppsrc/ops/attention.cpp:24-73).  Four columns per
// thread when T % 4 == 0 and the pointers are 16-byte aligned.
__global__ void __launch_bounds__(256)
causal_mask_vec_kernel(const f32x4* __restrict__ x, f32x4* __restrict__ y, int64_t n4, int64_t T, float fill) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < n4; u += stride) {
    const int64_t e = u * 4;
    const int64_t j = e % T, i = (e / T) % T;
    f32x4 v = x[u];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (j + k > i) v[k] = fill;
    y[u] = v;
  }
}

__global__ void __launch_bounds__(256)
causal_mask_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n, int64_t T, float fill) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += stride) {
    const int64_t j = e % T, i = (e / T) % T;
    y[e] = j <= i ? x[e] : fill;
  }
}

}  // namespace

bool colsum_chunks_of_64(int64_t rows) {
  return rows > 0 && rows % 64 == 0 && colsum_parts(rows) == rows / 64 && ceil_div(rows, colsum_parts(rows)) == 64;
}

int colsum_finish(const float* part, float* out, int nparts, int64_t cols, hipStream_t st) {
  colsum_stage2_kernel<<<dim3((unsigned)ceil_div(cols, (int64_t)kCsCols)), dim3(kCsThreads), 0, st>>>(part, out, nparts,
                                                                                                   cols);
  return launch_status();
}

}  // namespace aar

using namespace aar;

extern "C" {

int aar_sub_f32(const float* a, const float* b, float* c, int64_t n, void* s) {
  return launch_ew<Ew::Sub>(a, b, c, 0.f, n, s);
}
int aar_mul_f32(const float* a, const float* b, float* c, int64_t n, void* s) {
  return launch_ew<Ew::Mul>(a, b, c, 0.f, n, s);
}
int aar_scale_f32(const float* x, float* y, float alpha, int64_t n, void* s) {
  return launch_ew<Ew::Scale>(x, nullptr, y, alpha, n, s);
}
int aar_neg_f32(const float* x, float* y, int64_t n, void* s) { return launch_ew<Ew::Neg>(x, nullptr, y, 0.f, n, s); }
int aar_relu_f32(const float* x, float* y, int64_t n, void* s) {
  return launch_ew<Ew::Relu>(x, nullptr, y, 0.f, n, s);
}
int aar_relu_bwd_f32(const float* g, const float* x, float* dx, int64_t n, void* s) {
  return launch_ew<Ew::ReluBwd>(g, x, dx, 0.f, n, s);
}
int aar_gelu_f32(const float* x, float* y, int64_t n, void* s) {
  return launch_ew<Ew::Gelu>(x, nullptr, y, 0.f, n, s);
}
int aar_gelu_bwd_f32(const float* g, const float* x, float* dx, int64_t n, void* s) {
  return launch_ew<Ew::GeluBwd>(g, x, dx, 0.f, n, s);
}
int aar_fill_f32(float* y, float value, int64_t n, void* s) {
  return launch_ew<Ew::Fill>(nullptr, nullptr, y, value, n, s);
}
int aar_scaled_add_f32(float* dst, const float* src, float alpha, int64_t n, void* s) {
  return launch_ew<Ew::ScaledAdd>(dst, src, dst, alpha, n, s);
}

int aar_add_bias_f32(const float* x, const float* bias, float* y, int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols <= 0) return AAR_EINVAL;
  const int64_t n = rows * cols;
  if (n == 0) return AAR_OK;
  if (!x || !bias || !y) return AAR_EINVAL;
  hipStream_t st = as_stream(stream);
  if (cols % 4 == 0 && aligned16(x) && aligned16(bias) && aligned16(y)) {
    add_bias_vec_kernel<<<dim3(stream_grid(n / 4)), dim3(256), 0, st>>>(
        reinterpret_cast<const f32x4*>(x), reinterpret_cast<const f32x4*>(bias), reinterpret_cast<f32x4*>(y),
        n / 4, cols / 4);
  } else {
    add_bias_kernel<<<dim3(stream_grid(n)), dim3(256), 0, st>>>(x, bias, y, n, cols);
  }
  return launch_status();
}

size_t aar_colsum_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return (size_t)colsum_parts(rows) * (size_t)cols * sizeof(float);
}

int aar_colsum_f32(const float* g, float* out, int64_t rows, int64_t cols, void* workspace, size_t workspace_bytes,
                   void* stream) {
  if (rows < 0 || cols <= 0) return AAR_EINVAL;
  if (!out) return AAR_EINVAL;
  if (rows == 0) return aar_memset_zero(out, (size_t)cols * sizeof(float), stream);
  if (!g) return AAR_EINVAL;
  const int parts = colsum_parts(rows);
  if (!workspace || workspace_bytes < aar_colsum_workspace_bytes(rows, cols)) return AAR_EWORKSPACE;
  hipStream_t st = as_stream(stream);
  const int64_t chunk = ceil_div(rows, parts);
  float* part = static_cast<float*>(workspace);
  colsum_stage1_kernel<<<dim3((unsigned)ceil_div(cols, 256), (unsigned)parts), dim3(256), 0, st>>>(g, part, rows,
                                                                                                  cols, chunk);
  int rc = launch_status();
  if (rc != AAR_OK) return rc;
  colsum_stage2_kernel<<<dim3((unsigned)ceil_div(cols, (int64_t)kCsCols)), dim3(kCsThreads), 0, st>>>(part, out, parts,
                                                                                                   cols);
  return launch_status();
}

int aar_relu_bwd_colsum_f32(const float* g, const float* x, float* dx, float* colsum, int64_t rows, int64_t cols,
                            void* workspace, size_t workspace_bytes, void* stream) {
  if (rows < 0 || cols <= 0) return AAR_EINVAL;
  if (!colsum) return AAR_EINVAL;
  if (rows == 0) return aar_memset_zero(colsum, (size_t)cols * sizeof(float), stream);
  if (!g || !x || !dx) return AAR_EINVAL;
  if (!workspace || workspace_bytes < aar_colsum_workspace_bytes(rows, cols)) return AAR_EWORKSPACE;
  if (cols % 4 != 0 || !aligned16(g) || !aligned16(x) || !aligned16(dx) || !aligned16(workspace)) {
    const int rc = aar_relu_bwd_f32(g, x, dx, rows * cols, stream);
    return rc != AAR_OK ? rc : aar_colsum_f32(dx, colsum, rows, cols, workspace, workspace_bytes, stream);
  }
  hipStream_t st = as_stream(stream);
  const int parts = colsum_parts(rows);
  const int64_t chunk = ceil_div(rows, parts);
  float* part = static_cast<float*>(workspace);
  relu_bwd_colsum_stage1_kernel<<<dim3((unsigned)ceil_div(cols / 4, 256), (unsigned)parts), dim3(256), 0, st>>>(
      reinterpret_cast<const f32x4*>(g), reinterpret_cast<const f32x4*>(x), reinterpret_cast<f32x4*>(dx), part,
      rows, cols / 4, chunk);
  int rc = launch_status();
  if (rc != AAR_OK) return rc;
  colsum_stage2_kernel<<<dim3((unsigned)ceil_div(cols, (int64_t)kCsCols)), dim3(kCsThreads), 0, st>>>(part, colsum,
                                                                                                    parts, cols);
  return launch_status();
}

size_t aar_sum_workspace_bytes(int64_t n) {
  (void)n;
  return (size_t)kSumBlocks * sizeof(float);
}

int aar_sum_f32(const float* x, float* out, int64_t n, void* workspace, size_t workspace_bytes, void* stream) {
  if (n < 0 || !out) return AAR_EINVAL;
  if (n > 0 && !x) return AAR_EINVAL;
  if (!workspace || workspace_bytes < aar_sum_workspace_bytes(n)) return AAR_EWORKSPACE;
  hipStream_t st = as_stream(stream);
  const int64_t chunk = n > 0 ? ceil_div(n, kSumBlocks) : 1;
  float* part = static_cast<float*>(workspace);
  sum_stage1_kernel<<<dim3(kSumBlocks), dim3(256), 0, st>>>(x, part, n, chunk);
  int rc = launch_status();
  if (rc != AAR_OK) return rc;
  sum_stage2_kernel<<<dim3(1), dim3(256), 0, st>>>(part, out, kSumBlocks);
  return launch_status();
}

int aar_embedding_fwd_f32(const float* w, const int64_t* ids, float* out, int64_t n, int64_t vocab, int64_t dim,
                          int* err, void* stream) {
  if (n < 0 || vocab < 0 || dim < 0) return AAR_EINVAL;
  if (n == 0 || dim == 0) return AAR_OK;
  if (!ids || !out || (vocab > 0 && !w)) return AAR_EINVAL;
  if (dim % 4 == 0 && (vocab == 0 || aligned16(w)) && aligned16(out) && ceil_div(n, 4) <= (int64_t)UINT32_MAX) {
    embedding_fwd_vec_kernel<<<dim3((unsigned)ceil_div(n, 4)), dim3(256), 0, as_stream(stream)>>>(
        reinterpret_cast<const f32x4*>(w), ids, reinterpret_cast<f32x4*>(out), n, vocab, dim / 4, err);
    return launch_status();
  }
  embedding_fwd_kernel<<<dim3(stream_grid(n * dim)), dim3(256), 0, as_stream(stream)>>>(w, ids, out, n, vocab, dim,
                                                                                         err);
  return launch_status();
}

int aar_embedding_add_fwd_f32(const float* w1, const int64_t* ids1, int64_t vocab1, const float* w2,
                              const int64_t* ids2, int64_t vocab2, float* out, int64_t n, int64_t dim, int* err,
                              void* stream) {
  if (n < 0 || vocab1 < 0 || vocab2 < 0 || dim < 0) return AAR_EINVAL;
  if (n == 0 || dim == 0) return AAR_OK;
  if (!ids1 || !ids2 || !out || (vocab1 > 0 && !w1) || (vocab2 > 0 && !w2)) return AAR_EINVAL;
  hipStream_t st = as_stream(stream);
  if (dim % 4 == 0 && (vocab1 == 0 || aligned16(w1)) && (vocab2 == 0 || aligned16(w2)) && aligned16(out) &&
      ceil_div(n, 4) <= (int64_t)UINT32_MAX) {
    embedding_add_fwd_vec_kernel<<<dim3((unsigned)ceil_div(n, 4)), dim3(256), 0, st>>>(
        reinterpret_cast<const f32x4*>(w1), ids1, vocab1, reinterpret_cast<const f32x4*>(w2), ids2, vocab2,
        reinterpret_cast<f32x4*>(out), n, dim / 4, err);
    return launch_status();
  }
  embedding_add_fwd_kernel<<<dim3(stream_grid(n * dim)), dim3(256), 0, st>>>(w1, ids1, vocab1, w2, ids2, vocab2, out,
                                                                              n, dim, err);
  return launch_status();
}

// The one-hot GEMM path: one-hot [n, vocab] followed by the GEMM's own
// workspace.  Vocabularies up to 260 (with dim % 4 == 0) take the short-M
// kernel with the one-hot values made from the ids in registers; its split
// partial products need their own workspace.  The larger of the two is
// reported, so either path runs with it.
size_t aar_embedding_bwd_workspace_bytes(int64_t n, int64_t vocab, int64_t dim) {
  if (n <= 0 || vocab <= 0 || dim <= 0) return 0;
  const size_t oh = ((size_t)n * (size_t)vocab * sizeof(float) + 255) / 256 * 256;
  size_t bytes = oh + aar_gemm_f32_workspace_bytes(AAR_GEMM_TN, vocab, dim, n);
  if (shortm_shape_ok(vocab, dim, n)) {
    const int s = shortm_splits(vocab, dim, n, (size_t)-1);
    bytes = std::max(bytes, shortm_workspace_bytes(vocab, dim, n, s, true));
  }
  return bytes;
}

int aar_embedding_bwd_f32(const float* g, const int64_t* ids, float* dw, int64_t n, int64_t vocab, int64_t dim,
                          void* workspace, size_t workspace_bytes, void* stream) {
  if (n < 0 || vocab < 0 || dim < 0) return AAR_EINVAL;
  if (vocab == 0 || dim == 0) return AAR_OK;
  if (!dw) return AAR_EINVAL;
  if (n == 0) return aar_memset_zero(dw, (size_t)vocab * dim * sizeof(float), stream);
  if (!g || !ids) return AAR_EINVAL;
  if ((double)n * (double)vocab > (double)(1ll << 30)) return AAR_EUNSUPPORTED;
  if (!workspace || workspace_bytes < aar_embedding_bwd_workspace_bytes(n, vocab, dim)) return AAR_EWORKSPACE;
  if (shortm_shape_ok(vocab, dim, n) && aligned16(g) && aligned16(workspace)) {
    // dW = onehot(ids)^T . g with the one-hot rows made from the ids in registers
    const int s = shortm_splits(vocab, dim, n, workspace_bytes);
    if (shortm_workspace_bytes(vocab, dim, n, s, true) <= workspace_bytes)
      return run_shortm(nullptr, ids, g, dw, vocab, dim, n, s, workspace, workspace_bytes, as_stream(stream));
  }
  float* oh = static_cast<float*>(workspace);
  const size_t oh_bytes = ((size_t)n * (size_t)vocab * sizeof(float) + 255) / 256 * 256;
  onehot_kernel<<<dim3(stream_grid(n * vocab)), dim3(256), 0, as_stream(stream)>>>(ids, oh, n, vocab);
  int rc = launch_status();
  if (rc != AAR_OK) return rc;
  // dW[vocab, dim] = onehot[n, vocab]^T . g[n, dim]
  return aar_gemm_f32(AAR_GEMM_TN, vocab, dim, n, oh, g, dw, static_cast<char*>(workspace) + oh_bytes,
                      workspace_bytes - oh_bytes, stream);
}

// row_loss [n] floats, active [n] ints, count (int64)
size_t aar_cross_entropy_workspace_bytes(int64_t n) {
  if (n < 0) return 0;
  return (size_t)n * (sizeof(float) + sizeof(int)) + 16;
}

int aar_cross_entropy_fwd_f32(const float* logits, const int64_t* targets, float* loss, int64_t n, int64_t vocab,
                              int64_t ignore_index, int* err, void* workspace, size_t workspace_bytes,
                              void* stream) {
  if (n < 0 || vocab <= 0 || !loss) return AAR_EINVAL;
  if (n > 0 && (!logits || !targets)) return AAR_EINVAL;
  if (!workspace || workspace_bytes < aar_cross_entropy_workspace_bytes(n)) return AAR_EWORKSPACE;
  hipStream_t st = as_stream(stream);
  long long* count = static_cast<long long*>(workspace);
  float* row_loss = reinterpret_cast<float*>(static_cast<char*>(workspace) + 16);
  int* active = reinterpret_cast<int*>(row_loss + n);
  if (n > 0) {
    ce_row_kernel<<<dim3((unsigned)ceil_div(n, 4)), dim3(256), 0, st>>>(logits, targets, row_loss, active, n, vocab,
                                                                          ignore_index, err);
    const int rc = launch_status();
    if (rc != AAR_OK) return rc;
  }
  ce_mean_kernel<<<dim3(1), dim3(kCeThreads), 0, st>>>(row_loss, active, n, loss, count);
  return launch_status();
}

int aar_cross_entropy_bwd_f32(const float* grad, const float* logits, const int64_t* targets, float* dlogits,
                              int64_t n, int64_t vocab, int64_t ignore_index, void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (n < 0 || vocab <= 0) return AAR_EINVAL;
  if (n == 0) return AAR_OK;
  if (!grad || !logits || !targets || !dlogits) return AAR_EINVAL;
  if (!workspace || workspace_bytes < 16) return AAR_EWORKSPACE;
  hipStream_t st = as_stream(stream);
  long long* count = static_cast<long long*>(workspace);
  ce_count_kernel<<<dim3(1), dim3(kCeThreads), 0, st>>>(targets, n, ignore_index, count);
  int rc = launch_status();
  if (rc != AAR_OK) return rc;
  ce_bwd_kernel<<<dim3((unsigned)ceil_div(n, 4)), dim3(256), 0, st>>>(logits, targets, grad, count, dlogits, n,
                                                                        vocab, ignore_index);
  return launch_status();
}

int aar_adamw_f32(float* param, const float* grad, float* m, float* v, int64_t n, float lr, float beta1,
                  float beta2, float eps, float weight_decay, float bias_correction1, float bias_correction2,
                  void* stream) {
  if (n < 0) return AAR_EINVAL;
  if (n == 0) return AAR_OK;
  if (!param || !grad || !m || !v) return AAR_EINVAL;
  adamw_kernel<<<dim3(stream_grid(n)), dim3(256), 0, as_stream(stream)>>>(
      param, grad, m, v, n, lr, beta1, beta2, eps, 1.0f - lr * weight_decay, bias_correction1, bias_correction2);
  return launch_status();
}

int aar_scaled_add_multi_f32(int count, float* const* dst, const float* const* src, const int64_t* n, float alpha,
                             void* stream) {
  if (count < 0) return AAR_EINVAL;
  if (count == 0) return AAR_OK;
  if (!dst || !src || !n) return AAR_EINVAL;
  for (int i = 0; i < count; ++i)
    if (n[i] < 0 || (n[i] > 0 && (!dst[i] || !src[i]))) return AAR_EINVAL;
  return launch_multi(false, count, dst, src, nullptr, nullptr, n, alpha, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f,
                      as_stream(stream));
}

int aar_adamw_multi_f32(int count, float* const* param, const float* const* grad, float* const* m, float* const* v,
                        const int64_t* n, float lr, float beta1, float beta2, float eps, float weight_decay,
                        float bias_correction1, float bias_correction2, void* stream) {
  if (count < 0) return AAR_EINVAL;
  if (count == 0) return AAR_OK;
  if (!param || !grad || !m || !v || !n) return AAR_EINVAL;
  for (int i = 0; i < count; ++i)
    if (n[i] < 0 || (n[i] > 0 && (!param[i] || !grad[i] || !m[i] || !v[i]))) return AAR_EINVAL;
  return launch_multi(true, count, param, grad, m, v, n, 0.f, lr, beta1, beta2, eps, 1.0f - lr * weight_decay,
                      bias_correction1, bias_correction2, as_stream(stream));
}

int aar_dropout_f32(const float* x, float* out, float* mask, int64_t n, float p, uint64_t seed, void* stream) {
  if (n < 0 || !(p >= 0.0f && p < 1.0f)) return AAR_EINVAL;
  if (n == 0) return AAR_OK;
  if (!x || !out || !mask) return AAR_EINVAL;
  hipStream_t st = as_stream(stream);
  const float scale = 1.0f / (1.0f - p);
  int64_t begin = 0;
  if (aligned16(x) && aligned16(out) && aligned16(mask)) {
    const int64_t n4 = n / 4;
    if (n4 > 0) {
      dropout_vec_kernel<<<dim3(stream_grid(n4)), dim3(256), 0, st>>>(
          reinterpret_cast<const f32x4*>(x), reinterpret_cast<f32x4*>(out), reinterpret_cast<f32x4*>(mask), n4, p,
          scale, seed);
    }
    begin = 4 * n4;
  }
  if (begin < n) {
    dropout_kernel<<<dim3(stream_grid(n - begin)), dim3(256), 0, st>>>(x, out, mask, begin, n, p, scale, seed);
  }
  return launch_status();
}

int aar_causal_mask_f32(const float* x, float* y, int64_t mats, int64_t T, float fill, void* stream) {
  if (mats < 0 || T < 0) return AAR_EINVAL;
  if (mats == 0 || T == 0) return AAR_OK;
  if (!x || !y) return AAR_EINVAL;
  const int64_t n = mats * T * T;
  hipStream_t st = as_stream(stream);
  if (T % 4 == 0 && aligned16(x) && aligned16(y)) {
    causal_mask_vec_kernel<<<dim3(stream_grid(n / 4)), dim3(256), 0, st>>>(
        reinterpret_cast<const f32x4*>(x), reinterpret_cast<f32x4*>(y), n / 4, T, fill);
  } else {
    causal_mask_kernel<<<dim3(stream_grid(n)), dim3(256), 0, st>>>(x, y, n, T, fill);
  }
  return launch_status();
}

}  // extern "C"
