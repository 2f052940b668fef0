// fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x2f32), three layouts:
//   NN  C[M,N] = A[M,K]   . B[K,N]     (reference matmul,      cppsrc/ops/matmul.cu:345-444)
//   NT  C[M,N] = A[M,K]   . B[N,K]^T   (reference matmul_a_bt, cppsrc/ops/matmul.cu:446-547)
//   TN  C[M,N] = A[K,M]^T . B[K,N]     (reference matmul_at_b, cppsrc/ops/matmul.cu:549-645)
//
// Design (not a translation of the reference's FFMA kernels):
//  * One workgroup computes a BM x BN tile; each wave64 owns a WM x WN sub-tile
//    held as (WM/32) x (WN/32) MFMA 32x32 accumulators.
//  * K is consumed in chunks of 8.  In chunk step s (0..3) lane half h = lane/32
//    supplies k = kc + 4h + s, so the four k-steps of a lane are 4 consecutive
//    k values.  An operand that is K-contiguous in HBM is therefore staged in
//    LDS as [row][k] and read with one ds_read_b128 per chunk; an operand that
//    is M/N-contiguous in HBM is staged as [k][row] and read with four
//    conflict-free ds_read_b32.  The transposed variants differ only in these
//    load patterns: no transpose kernels and no transposing LDS stores.
//  * A/B tiles are double-buffered in LDS; the next tile's global loads are
//    issued into registers before the current tile's MFMAs, so one barrier per
//    K tile suffices.  LDS rows are padded so the 128-bit fragment reads are
//    bank-conflict free.
//  * Workgroup ids are remapped so that the tiles resident on one XCD (the
//    hardware deals workgroups round-robin over the 8 XCDs) form a compact
//    GROUP_M-row band and share A/B panels in that XCD's L2.
//  * Thin outputs with a long contraction (weight gradients) use a split-K
//    launch into a workspace followed by a fixed-order reduction, so results
//    are deterministic (no float atomics).
#include <hip/hip_runtime.h>

#include "common.hpp"

namespace aar {
namespace {

constexpr int kGroupM = 4;

__device__ __forceinline__ void map_tile(int tiles_m, int tiles_n, int& tm, int& tn) {
  int w = blockIdx.x;
  const int nb = gridDim.x;
  if ((nb & 7) == 0) w = (w & 7) * (nb >> 3) + (w >> 3);  // XCD-contiguous ranges
  const int group_size = kGroupM * tiles_n;
  const int group = w / group_size;
  const int first_m = group * kGroupM;
  const int rows = min(tiles_m - first_m, kGroupM);
  const int in_group = w - group * group_size;
  tm = first_m + in_group % rows;
  tn = in_group / rows;
}

// Global -> register staging for one operand tile.
//   KC: operand is K-contiguous in HBM (element (r,k) at P[r*ld + k]); LDS [r][k].
//   else: operand is R-contiguous (element (r,k) at P[k*ld + r]); LDS [k][r].
// R is the operand's M or N extent (BR rows of the tile).
template <int BR, int BK, int NT, bool KC, bool VEC>
struct TileLoader {
  static constexpr int kUnits = BR * BK / 4;  // float4 units per tile
  static_assert(kUnits % NT == 0, "tile must divide evenly over the workgroup");
  static constexpr int kPer = kUnits / NT;
  static constexpr int kLd = KC ? (BK + 4) : (BR + 8);  // padded LDS row (floats)
  static constexpr int kSize = KC ? BR * kLd : BK * kLd;

  f32x4 reg[kPer];

  __device__ __forceinline__ void load(const float* __restrict__ P, int64_t ld, int64_t r0,
                                       int64_t R, int64_t k0, int64_t kend, int tid) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int u = tid + i * NT;
      int rr, kk;
      if (KC) {
        rr = u / (BK / 4);
        kk = (u % (BK / 4)) * 4;
      } else {
        kk = u / (BR / 4);
        rr = (u % (BR / 4)) * 4;
      }
      const int64_t gr = r0 + rr;
      const int64_t gk = k0 + kk;
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (KC) {
        if (gr < R) {
          const float* p = P + gr * ld + gk;
          if (VEC) {
            if (gk < kend) v = *reinterpret_cast<const f32x4*>(p);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (gk + e < kend) v[e] = p[e];
          }
        }
      } else {
        if (gk < kend) {
          const float* p = P + gk * ld + gr;
          if (VEC) {
            if (gr < R) v = *reinterpret_cast<const f32x4*>(p);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (gr + e < R) v[e] = p[e];
          }
        }
      }
      reg[i] = v;
    }
  }

  __device__ __forceinline__ void store(float* __restrict__ S, int tid) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int u = tid + i * NT;
      int off;
      if (KC) {
        off = (u / (BK / 4)) * kLd + (u % (BK / 4)) * 4;
      } else {
        off = (u / (BR / 4)) * kLd + (u % (BR / 4)) * 4;
      }
      *reinterpret_cast<f32x4*>(S + off) = reg[i];
    }
  }

  // MFMA operand fragment: lane (r = lane%32, h = lane/32) gets the 4 values
  // for k = kc + 4h + {0,1,2,3} of tile row `row`.
  __device__ __forceinline__ static f32x4 frag(const float* __restrict__ S, int row, int kc, int h) {
    if (KC) {
      return *reinterpret_cast<const f32x4*>(S + row * kLd + kc + 4 * h);
    } else {
      f32x4 v;
      const float* p = S + (kc + 4 * h) * kLd + row;
      v[0] = p[0];
      v[1] = p[kLd];
      v[2] = p[2 * kLd];
      v[3] = p[3 * kLd];
      return v;
    }
  }
};

template <int BM, int BN, int BK, int WM, int WN, bool A_KC, bool B_KC, bool VEC>
__global__ void __launch_bounds__((BM / WM) * (BN / WN) * 64)
gemm_f32_kernel(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C,
                int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                int64_t k_per_split, int64_t split_stride, int tiles_m, int tiles_n) {
  constexpr int NWM = BM / WM;
  constexpr int NT = NWM * (BN / WN) * 64;
  constexpr int TM = WM / 32;
  constexpr int TN = WN / 32;
  static_assert(BK % 8 == 0, "BK must be a multiple of 8");
  using LA = TileLoader<BM, BK, NT, A_KC, VEC>;
  using LB = TileLoader<BN, BK, NT, B_KC, VEC>;

  __shared__ __attribute__((aligned(16))) float smem[2 * (LA::kSize + LB::kSize)];
  constexpr int kStage = LA::kSize + LB::kSize;  // floats per pipeline stage

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lr = lane & 31;
  const int h = lane >> 5;
  const int wm0 = (wave % NWM) * WM;
  const int wn0 = (wave / NWM) * WN;

  int tm, tn;
  map_tile(tiles_m, tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * BM;
  const int64_t n0 = (int64_t)tn * BN;

  const int64_t kbeg = (int64_t)blockIdx.y * k_per_split;
  const int64_t kend = min(K, kbeg + k_per_split);
  C += (int64_t)blockIdx.y * split_stride;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  LA la;
  LB lb;
  if (kbeg < kend) {
    la.load(A, lda, m0, M, kbeg, kend, tid);
    lb.load(B, ldb, n0, N, kbeg, kend, tid);
    la.store(smem, tid);
    lb.store(smem + LA::kSize, tid);
  }
  __syncthreads();

  int cur = 0;
  for (int64_t kt = kbeg; kt < kend; kt += BK) {
    const bool has_next = kt + BK < kend;
    if (has_next) {
      la.load(A, lda, m0, M, kt + BK, kend, tid);
      lb.load(B, ldb, n0, N, kt + BK, kend, tid);
    }
    const float* as = smem + cur * kStage;
    const float* bs = as + LA::kSize;
#pragma unroll
    for (int kc = 0; kc < BK; kc += 8) {
      f32x4 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = LA::frag(as, wm0 + 32 * i + lr, kc, h);
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = LB::frag(bs, wn0 + 32 * j + lr, kc, h);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s], bf[j][s], acc[i][j], 0, 0, 0);
    }
    if (has_next) {
      float* nxt = smem + (cur ^ 1) * kStage;
      la.store(nxt, tid);
      lb.store(nxt + LA::kSize, tid);
    }
    __syncthreads();
    cur ^= 1;
  }

  // Accumulator layout of a 32x32 block: lane (lr, h), register r holds
  // row 8*(r/4) + 4*h + (r%4), column lr.
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t col = n0 + wn0 + 32 * j + lr;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm0 + 32 * i + 8 * (r / 4) + 4 * h + (r % 4);
        if (row < M && col < N) C[row * ldc + col] = acc[i][j][r];
      }
    }
  }
}

// C[i] = sum_s W[s*stride + i], s in order 0..splits-1 (deterministic), four
// consecutive outputs per thread with 128-bit loads (stride % 4 == 0 and
// 16-byte aligned W/C); the split loop is unrolled so its loads overlap.
__global__ void __launch_bounds__(256)
splitk_reduce_vec_kernel(const f32x4* __restrict__ W, f32x4* __restrict__ C, int64_t n4, int64_t stride4,
                         int splits) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  f32x4 s = W[i];
#pragma unroll 8
  for (int p = 1; p < splits; ++p) s += W[p * stride4 + i];
  C[i] = s;
}

__global__ void __launch_bounds__(256)
splitk_reduce_kernel(const float* __restrict__ W, float* __restrict__ C, int64_t n, int64_t stride,
                     int splits) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float s = W[i];
#pragma unroll 8
  for (int p = 1; p < splits; ++p) s += W[p * stride + i];
  C[i] = s;
}

struct Cfg {
  int bm, bn, resident;  // resident workgroups per CU
  float eff;             // rough relative MFMA efficiency of the tile shape
};
constexpr Cfg kCfgs[] = {
    {256, 256, 1, 1.00f},
    {128, 128, 2, 0.85f},
    {64, 64, 4, 0.55f},
};

struct Plan {
  int cfg;
  int splits;
  int64_t k_per_split;
};

constexpr int kBK = 16;

Plan plan_gemm(int64_t M, int64_t N, int64_t K, size_t ws_bytes, bool allow_split) {
  const int cus = device_cu_count();
  Plan best{2, 1, K};
  double best_t = 1e300;
  for (int c = 0; c < 3; ++c) {
    const Cfg& cf = kCfgs[c];
    const int64_t tiles = ceil_div(M, cf.bm) * ceil_div(N, cf.bn);
    for (int splits = 1; splits <= 64; splits *= 2) {
      if (splits > 1) {
        if (!allow_split) break;
        if (K / splits < 256) break;
        if ((size_t)splits * M * N * sizeof(float) > ws_bytes) break;
      }
      int64_t kps = ceil_div(ceil_div(K, splits), kBK) * kBK;
      const int64_t real_splits = ceil_div(K, kps);
      const int64_t blocks = tiles * real_splits;
      const int64_t slots = (int64_t)cus * cf.resident;
      const int64_t waves = ceil_div(blocks, slots);
      double t = (double)waves * cf.resident * 2.0 * cf.bm * cf.bn * (double)kps / (cf.eff * 614e9);
      if (splits > 1) t += (double)(real_splits + 1) * M * N * 4.0 / 4e12 + 4e-6;
      if (t < best_t) {
        best_t = t;
        best = Plan{c, (int)real_splits, kps};
      }
    }
  }
  return best;
}

template <int BM, int BN, int WM, int WN, bool A_KC, bool B_KC>
int launch_cfg(bool vec, const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
               int64_t lda, int64_t ldb, int64_t ldc, int splits, int64_t kps, int64_t split_stride,
               hipStream_t st) {
  const int tiles_m = (int)ceil_div(M, BM);
  const int tiles_n = (int)ceil_div(N, BN);
  dim3 grid((unsigned)(tiles_m * tiles_n), (unsigned)splits);
  dim3 block((BM / WM) * (BN / WN) * 64);
  if (vec)
    gemm_f32_kernel<BM, BN, kBK, WM, WN, A_KC, B_KC, true><<<grid, block, 0, st>>>(
        A, B, C, M, N, K, lda, ldb, ldc, kps, split_stride, tiles_m, tiles_n);
  else
    gemm_f32_kernel<BM, BN, kBK, WM, WN, A_KC, B_KC, false><<<grid, block, 0, st>>>(
        A, B, C, M, N, K, lda, ldb, ldc, kps, split_stride, tiles_m, tiles_n);
  return launch_status();
}

template <bool A_KC, bool B_KC>
int launch_op(int cfg, bool vec, const float* A, const float* B, float* C, int64_t M, int64_t N,
              int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int splits, int64_t kps,
              int64_t split_stride, hipStream_t st) {
  switch (cfg) {
    case 0:
      return launch_cfg<256, 256, 128, 128, A_KC, B_KC>(vec, A, B, C, M, N, K, lda, ldb, ldc, splits,
                                                       kps, split_stride, st);
    case 1:
      return launch_cfg<128, 128, 64, 64, A_KC, B_KC>(vec, A, B, C, M, N, K, lda, ldb, ldc, splits,
                                                     kps, split_stride, st);
    default:
      return launch_cfg<64, 64, 32, 32, A_KC, B_KC>(vec, A, B, C, M, N, K, lda, ldb, ldc, splits, kps,
                                                   split_stride, st);
  }
}

bool gemm_vec_ok(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B) {
  if (!aligned16(A) || !aligned16(B)) return false;
  switch (op) {
    case AAR_GEMM_NN: return (K % 4 == 0) && (N % 4 == 0);
    case AAR_GEMM_NT: return (K % 4 == 0);
    default: return (M % 4 == 0) && (N % 4 == 0);
  }
}

}  // namespace
}  // namespace aar

using namespace aar;

extern "C" size_t aar_gemm_f32_workspace_bytes(int op, int64_t M, int64_t N, int64_t K) {
  if (op < 0 || op > 2 || M <= 0 || N <= 0 || K <= 0) return 0;
  const Plan p = plan_gemm(M, N, K, (size_t)-1, true);
  if (p.splits <= 1) return 0;
  return (size_t)p.splits * (size_t)M * (size_t)N * sizeof(float);
}

extern "C" int aar_gemm_f32(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B,
                            float* C, void* workspace, size_t workspace_bytes, void* stream) {
  if (op < 0 || op > 2 || M < 0 || N < 0 || K < 0) return AAR_EINVAL;
  if (M == 0 || N == 0) return AAR_OK;
  if (!C) return AAR_EINVAL;
  hipStream_t st = as_stream(stream);
  if (K == 0) return aar_memset_zero(C, (size_t)M * N * sizeof(float), stream);
  if (!A || !B) return AAR_EINVAL;
  if (M > INT32_MAX / 2 || N > INT32_MAX / 2) return AAR_EUNSUPPORTED;

  const bool vec = gemm_vec_ok(op, M, N, K, A, B);
  const Plan p = plan_gemm(M, N, K, workspace ? workspace_bytes : 0, workspace != nullptr);
  int64_t lda, ldb;
  switch (op) {
    case AAR_GEMM_NN: lda = K; ldb = N; break;
    case AAR_GEMM_NT: lda = K; ldb = K; break;
    default: lda = M; ldb = N; break;
  }
  float* out = p.splits > 1 ? static_cast<float*>(workspace) : C;
  const int64_t split_stride = p.splits > 1 ? M * N : 0;
  int rc;
  switch (op) {
    case AAR_GEMM_NN:
      rc = launch_op<true, false>(p.cfg, vec, A, B, out, M, N, K, lda, ldb, N, p.splits, p.k_per_split,
                                  split_stride, st);
      break;
    case AAR_GEMM_NT:
      rc = launch_op<true, true>(p.cfg, vec, A, B, out, M, N, K, lda, ldb, N, p.splits, p.k_per_split,
                                 split_stride, st);
      break;
    default:
      rc = launch_op<false, false>(p.cfg, vec, A, B, out, M, N, K, lda, ldb, N, p.splits,
                                   p.k_per_split, split_stride, st);
      break;
  }
  if (rc != AAR_OK || p.splits <= 1) return rc;
  const int64_t n = M * N;
  if (n % 4 == 0 && aligned16(out) && aligned16(C)) {
    splitk_reduce_vec_kernel<<<dim3((unsigned)ceil_div(n / 4, 256)), dim3(256), 0, st>>>(
        reinterpret_cast<const f32x4*>(out), reinterpret_cast<f32x4*>(C), n / 4, split_stride / 4, p.splits);
  } else {
    splitk_reduce_kernel<<<dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, st>>>(out, C, n, split_stride,
                                                                                p.splits);
  }
  return launch_status();
}
