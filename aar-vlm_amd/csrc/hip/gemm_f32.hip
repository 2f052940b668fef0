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
//  * 16-byte aligned operands (the common case) are streamed HBM -> LDS with
//    global_load_lds_dwordx4 into a 2-4 stage ring: no register staging, and
//    the loads of the next S-2 tiles are in flight while a tile is computed
//    (one s_waitcnt + one barrier per K tile).  LDS layouts are XOR-swizzled
//    so the fragment reads are bank-conflict free without padding.  Tile rows
//    beyond the matrix are clamped onto its last row (they feed only
//    accumulator rows or columns the epilogue never stores), so interior K
//    tiles load without per-lane predicates; a ragged last K tile goes
//    through registers with K predicates.  Within a tile the fragments of
//    chunk c+1 are read from LDS while chunk c's MFMAs run.
//  * Other operands use predicated register loads into a padded,
//    double-buffered LDS tile.
//  * Workgroup ids are remapped so that the tiles resident on one XCD (the
//    hardware deals workgroups round-robin over the 8 XCDs) form a compact
//    GROUP_M-row band and share A/B panels in that XCD's L2.
//  * Thin outputs with a long contraction (weight gradients) use a split-K
//    launch into a workspace followed by a fixed-order reduction, so results
//    are deterministic (no float atomics).
#include <hip/hip_runtime.h>

#include <algorithm>

#include <type_traits>

#include "colsum.hpp"
#include "common.hpp"
#include "gemm_small.hpp"

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

// Epilogues (a template argument, because every one but the plain store
// needs the accumulators in VGPRs: the kernels without one store straight
// from the accumulators and keep their occupancy).  Each is the same fp32
// operation as the separate op applied to the stored product:
//   kEpiBias      C = acc + bias[col]            (linear layer: add_bias)
//   kEpiBiasRelu  C = max(0, acc + bias[col])    (linear layer, then relu)
//   kEpiMask      C = aux[row][col] > 0 ? acc : 0  (relu backward, aux = the
//                 relu's output, which is positive exactly where its input is;
//                 aux has C's layout)
//   kEpiAdd       C = acc + aux[row][col]          (a residual add after the
//                 product: x + y W^T)
//   kEpiBiasAdd   C = (acc + bias[col]) + aux[row][col]  (the same after a
//                 linear layer with a bias)
// and two that carry a relu's mask as bits from the forward product to the
// backward one (store_tile_bits), so the backward reads 1 bit per element
// where kEpiMask reads the relu's whole output:
//   kEpiBiasReluBits  C = max(0, acc + bias[col]) as kEpiBiasRelu, and bit
//                     row % 32 of word bits[(row / 32) * N + col] set where
//                     C > 0: a word holds one column of a 32-row block, the
//                     rows of one accumulator block
//   kEpiMaskBits      C = bit(row, col) ? acc : 0 (the relu backward), and
//                     part[row / 64][col] = the sum of C over the 64 rows of
//                     that chunk, in aar_colsum_f32's stage-1 order (two
//                     running sums, see colsum_stage1_kernel): its partials
//                     (a wave owns one chunk)
enum : int {
  kEpiNone = 0,
  kEpiBias = 1,
  kEpiBiasRelu = 2,
  kEpiMask = 3,
  kEpiAdd = 4,
  kEpiBiasAdd = 5,
  kEpiBiasReluBits = 6,
  kEpiMaskBits = 7,
  kEpiColsumA = 8
};
// kEpiColsumA is not an epilogue but work in the main loop (TN only): C is
// stored plainly, and the waves of the first column of waves also sum the
// staged A tile's columns: part[k / 64][m] = the sum of A[k][m] over the
// 64-row chunk of k, in aar_colsum_f32's stage-1 order.  A lane holds the
// k's with k & 4 == 4h of its column in order, i.e. one of that order's two
// running sums; the halves add them at the chunk's end.  Chunk q is summed by
// the workgroups with tn == q % tiles_n, so the work spreads over the grid.
struct GemmEpi {
  const float* bias;
  const float* aux;
  uint32_t* bits = nullptr;  // [ceil(M / 32)][N]: kEpiBiasReluBits writes, kEpiMaskBits reads
  float* part = nullptr;     // kEpiMaskBits: [M / 64][N] column partials; kEpiColsumA: [K / 64][M]
};
constexpr bool epi_bits(int epi) { return epi == kEpiBiasReluBits || epi == kEpiMaskBits; }
constexpr bool epi_dma_only(int epi) { return epi_bits(epi) || epi == kEpiColsumA; }

// Epilogue: a wave's (32*TM) x (32*TN) accumulators to C.  Accumulator
// layout of a 32x32 block: lane (lr, h), register r holds row
// 8*(r/4) + 4*h + (r%4), column lr.
// A wave tile wholly inside C (the common case) stores without bounds tests;
// element offsets from the lane's first element are a constant row count
// times ldc, which the compiler forms once in scalar registers.
// NQ < 4: only register quads q0 .. q0 + NQ - 1 of each accumulator are
// stored, their values held in quads 0 .. NQ - 1 of acc (a K group's share).
constexpr bool epi_has_bias(int epi) {
  return epi == kEpiBias || epi == kEpiBiasRelu || epi == kEpiBiasAdd || epi == kEpiBiasReluBits;
}

// The bias values a lane's accumulator columns need (column c0 + 32 j + lr),
// read before the main loop so their latency is hidden under it: read at
// the epilogue, they cost a memory round trip per workgroup round (measured
// +10 us on a 16384 x 1536 x 384 product with the bias epilogue).
template <int TN, int EPI>
__device__ __forceinline__ void load_bias(const GemmEpi& ep, int64_t N, int64_t c0, int lr, float (&bias)[TN]) {
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t col = c0 + 32 * j + lr;
    bias[j] = 0.f;
    if constexpr (epi_has_bias(EPI)) bias[j] = col < N ? ep.bias[col] : 0.f;
  }
}

// Mask words the kEpiMaskBits epilogue needs, read before the main loop like
// the bias: lane (lr, h) holds, for block (i, j), the word of column
// c0 + 32 j + lr over rows r0 + 32 i .. + 31 (both halves read the same word,
// 128 contiguous bytes per half-wave).
template <int TM, int TN, int EPI>
__device__ __forceinline__ void load_bits(const GemmEpi& ep, int64_t M, int64_t N, int64_t r0, int64_t c0, int lr,
                                          uint32_t (&words)[TM][TN]) {
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      words[i][j] = 0u;
      if constexpr (EPI == kEpiMaskBits) {
        const int64_t col = c0 + 32 * j + lr;
        if (r0 + 32 * i < M && col < N) words[i][j] = ep.bits[((r0 + 32 * i) >> 5) * N + col];
      }
    }
}

// The two mask-bit epilogues (see kEpiBiasReluBits / kEpiMaskBits).  Wave
// tiles start at multiples of 32 rows, so accumulator block (i, j) covers
// whole mask words: lane (lr, h) holds the bits 8 (r / 4) + 4 h + r % 4 of the
// word of its column c0 + 32 j + lr, its half's 16 rows.
//   kEpiBiasReluBits: each lane sets its 16 bits, the two halves OR their
//   words (v_permlane32_swap) and half 0 stores the word.
//   kEpiMaskBits (WM = 64: the wave's rows are one 64-row chunk): each lane
//   tests its 16 bits of the prefetched word and sums its 32 rows of the
//   chunk in order, the row set (row & 4 == 4h) of one of colsum's two
//   running sums; half 0 adds its partner's (v_permlane32_swap) and stores
//   the chunk partial s0 + s1.
// The swap hands each lane its own value and its partner's, one in each
// result; where the two are equal either is the partner's.
__device__ __forceinline__ uint32_t partner_u32(uint32_t u) {
#if defined(__HIP_DEVICE_COMPILE__)
  const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return sw[0] == u ? sw[1] : sw[0];
#else
  return u;
#endif
}

template <int TM, int TN, int EPI>
__device__ __forceinline__ void store_tile_bits(const f32x16 (&acc)[TM][TN], float* __restrict__ C,
                                                const GemmEpi& ep, const float (&bias)[TN],
                                                const uint32_t (&words)[TM][TN], int64_t M, int64_t N, int64_t ldc,
                                                int64_t r0, int64_t c0, int lr, int h) {
  static_assert(epi_bits(EPI), "mask-bit epilogues only");
  static_assert(EPI != kEpiMaskBits || TM == 2, "a kEpiMaskBits wave owns one 64-row chunk");
  // addressing as store_tile: a lane base and row offsets dr * ldc that the
  // compiler forms in scalar registers, bounds tests only off the interior
  const bool interior = r0 + 32 * TM <= M && c0 + 32 * TN <= N;
  float* const Cl = C + (r0 + 4 * h) * ldc + c0 + lr;
  wait_vm_lgkm0<0>();  // bias / mask words (see store_tile)
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t col = c0 + 32 * j + lr;
    float vals[TM][16];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      uint32_t w = 0u;                           // this half's bits, at 8 (r / 4) + r % 4
      const uint32_t mine = words[i][j] >> (4 * h);  // kEpiMaskBits: the same positions
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dr = 32 * i + 8 * (r >> 2) + (r & 3);  // row - r0 - 4h
        const int bit = 8 * (r >> 2) + (r & 3);
        const bool ok = interior || (r0 + 4 * h + dr < M && col < N);
        float v;
        // (the bit tests stay free of the bounds test: with it, the compiler
        // kept every element's lane mask live and spilled them to VGPR lanes)
        if constexpr (EPI == kEpiBiasReluBits) {
          v = fmaxf(0.0f, acc[i][j][r] + bias[j]);
          w |= v > 0.0f ? (1u << bit) : 0u;
        } else {
          // all ones where the bit is set: acc, else +0.0f
#if defined(__HIP_DEVICE_COMPILE__)
          const uint32_t keep = (uint32_t)__builtin_amdgcn_sbfe((int)mine, bit, 1);
#else
          const uint32_t keep = ((mine >> bit) & 1u) ? ~0u : 0u;
#endif
          v = __uint_as_float(__float_as_uint(acc[i][j][r]) & keep);
          vals[i][r] = v;
        }
        if (ok) Cl[(int64_t)dr * ldc + 32 * j] = v;
      }
      if constexpr (EPI == kEpiBiasReluBits) {
        w <<= 4 * h;
        w |= partner_u32(w);
        const int64_t rows = M - (r0 + 32 * i);  // rows of this word inside C
        if (rows < 32) w &= (1u << (rows > 0 ? rows : 0)) - 1u;
        if (h == 0 && rows > 0 && col < N) ep.bits[((r0 + 32 * i) >> 5) * N + col] = w;
      }
    }
    if constexpr (EPI == kEpiMaskBits) {
      if (!ep.part) continue;  // the mask only
      // colsum's chunk partial: half h's running sum over its rows (row & 4
      // == 4h) in row order, i.e. its registers in order, then s0 + s1
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += vals[i][r];
      s += __uint_as_float(partner_u32(__float_as_uint(s)));
      if (h == 0 && col < N && r0 < M) ep.part[(r0 >> 6) * N + col] = s;
    }
  }
}

template <int TM, int TN, int EPI, int NQ = 4, bool BATCH = false>
__device__ __forceinline__ void store_tile(const f32x16 (&acc)[TM][TN], float* __restrict__ C, const GemmEpi& ep,
                                           const float (&bias)[TN], int64_t M, int64_t N, int64_t ldc, int64_t r0,
                                           int64_t c0, int lr, int h, int q0 = 0) {
  const bool interior = r0 + 32 * TM <= M && c0 + 32 * TN <= N;
  const int64_t lane0 = (r0 + 4 * h) * ldc + c0 + lr;  // offset of the lane's first element
  float* const Cl = C + lane0;
  constexpr bool kAux = EPI == kEpiMask || EPI == kEpiAdd || EPI == kEpiBiasAdd;
  // The loaded operands (bias, aux) are waited for once, explicitly, before
  // the stores.  Left to the compiler, the per-element bounds branches made
  // it wait for vmcnt(0) before every store that uses one (stores count in
  // vmcnt), one memory round trip per element: measured +10 us on a
  // 16384 x 1536 x 384 product with the bias epilogue.
  if constexpr (epi_has_bias(EPI)) wait_vm_lgkm0<0>();
  const float* const Xl = kAux ? ep.aux + lane0 : nullptr;
  // The aux values are loaded before any store they feed: C and aux may
  // alias (an in-place residual), so a load placed after a store would wait
  // for it, one memory round trip per element.  (Each element is read and
  // then written by the same lane, so an aliased aux still reads the old
  // values.)  BATCH (the DMA kernels, whose staging registers are free by
  // the epilogue): when the wave tile's aux values fit in 96 registers (the
  // accumulators' count for a 64 x 96 wave tile), all rows of blocks are
  // loaded in one batch and waited for once, one memory round trip per wave
  // instead of one per row of blocks.  Otherwise a row of blocks at a time
  // (in the register path the batch cost occupancy).
  constexpr int kRowsPerBatch = BATCH && kAux && TM * TN * 4 * NQ <= 96 ? TM : 1;
  auto load_aux = [&](int i, float (&xv)[TN][4 * NQ]) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t col = c0 + 32 * j + lr;
#pragma unroll
      for (int r = 0; r < 4 * NQ; ++r) {
        const int dr = 32 * i + 8 * (q0 + r / 4) + (r % 4);
        const int64_t off = (int64_t)dr * ldc + 32 * j;
        xv[j][r] = (interior || (r0 + 4 * h + dr < M && col < N)) ? Xl[off] : 0.0f;
      }
    }
  };
#pragma unroll
  for (int i0 = 0; i0 < TM; i0 += kRowsPerBatch) {
    float xv[kRowsPerBatch][TN][4 * NQ];
    if constexpr (kAux) {
#pragma unroll
      for (int ib = 0; ib < kRowsPerBatch; ++ib) load_aux(i0 + ib, xv[ib]);
      wait_vm_lgkm0<0>();
    }
#pragma unroll
    for (int ib = 0; ib < kRowsPerBatch; ++ib) {
      const int i = i0 + ib;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t col = c0 + 32 * j + lr;
        const float b = bias[j];
#pragma unroll
        for (int r = 0; r < 4 * NQ; ++r) {
          const int dr = 32 * i + 8 * (q0 + r / 4) + (r % 4);  // row - r0 - 4h
          const int64_t off = (int64_t)dr * ldc + 32 * j;
          if (interior || (r0 + 4 * h + dr < M && col < N)) {
            float v = acc[i][j][r];
            if constexpr (EPI == kEpiBias) v = v + b;
            if constexpr (EPI == kEpiBiasRelu) v = fmaxf(0.0f, v + b);
            if constexpr (EPI == kEpiMask) v = xv[ib][j][r] > 0.0f ? v : 0.0f;
            if constexpr (EPI == kEpiAdd) v = v + xv[ib][j][r];
            if constexpr (EPI == kEpiBiasAdd) v = (v + b) + xv[ib][j][r];
            Cl[off] = v;
          }
        }
      }
    }
  }
}

// ------------------------------------------------------- register path
// Operands that are not 16-byte aligned or whose contiguous extent is not a
// multiple of 4: predicated element loads into registers, stored to a padded,
// double-buffered LDS tile.
//   KC: operand is K-contiguous in HBM (element (r,k) at P[r*ld + k]); LDS [r][k].
//   else: operand is R-contiguous (element (r,k) at P[k*ld + r]); LDS [k][r].
// R is the operand's M or N extent (BR rows of the tile).
template <int BR, int BK, int NT, bool KC>
struct TileLoader {
  static constexpr int kUnits = BR * BK / 4;  // 4-element units per tile
  static_assert(kUnits % NT == 0, "tile must divide evenly over the workgroup");
  static constexpr int kPer = kUnits / NT;
  static constexpr int kLd = KC ? (BK + 4) : (BR + 8);  // padded LDS row (floats)
  static constexpr int kSize = KC ? BR * kLd : BK * kLd;

  f32x4 reg[kPer];

  __device__ __forceinline__ static void coords(int u, int& rr, int& kk) {
    if (KC) {
      rr = u / (BK / 4);
      kk = (u % (BK / 4)) * 4;
    } else {
      kk = u / (BR / 4);
      rr = (u % (BR / 4)) * 4;
    }
  }

  __device__ __forceinline__ void load(const float* __restrict__ P, int64_t ld, int64_t r0, int64_t R,
                                       int64_t k0, int64_t kend, int tid) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      int rr, kk;
      coords(tid + i * NT, rr, kk);
      const int64_t gr = r0 + rr;
      const int64_t gk = k0 + kk;
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (KC) {
        if (gr < R) {
          const float* p = P + gr * ld + gk;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (gk + e < kend) v[e] = p[e];
        }
      } else {
        if (gk < kend) {
          const float* p = P + gk * ld + gr;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (gr + e < R) v[e] = p[e];
        }
      }
      reg[i] = v;
    }
  }

  __device__ __forceinline__ void store(float* __restrict__ S, int tid) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      int rr, kk;
      coords(tid + i * NT, rr, kk);
      *reinterpret_cast<f32x4*>(S + (KC ? rr * kLd + kk : kk * kLd + rr)) = reg[i];
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

// WPE: waves per SIMD the register allocation must allow (resident
// workgroups per CU x waves per workgroup / 4).
template <int BM, int BN, int BK, int WM, int WN, int WPE, bool A_KC, bool B_KC, int EPI>
__global__ void __launch_bounds__((BM / WM) * (BN / WN) * 64, WPE)
gemm_f32_kernel(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C,
                int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                int64_t k_per_split, int64_t split_stride, int tiles_m, int tiles_n, int64_t sA, int64_t sB,
                int64_t sC, GemmEpi ep) {
  constexpr int NWM = BM / WM;
  constexpr int NT = NWM * (BN / WN) * 64;
  constexpr int TM = WM / 32;
  constexpr int TN = WN / 32;
  constexpr int NC = BK / 8;  // 8-deep k chunks per tile
  static_assert(BK % 8 == 0, "BK must be a multiple of 8");
  using LA = TileLoader<BM, BK, NT, A_KC>;
  using LB = TileLoader<BN, BK, NT, B_KC>;

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
  // batched launches: one grid layer per matrix (blockIdx.z)
  A += (int64_t)blockIdx.z * sA;
  B += (int64_t)blockIdx.z * sB;
  C += (int64_t)blockIdx.z * sC;

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
    for (int c = 0; c < NC; ++c) {
      f32x4 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = LA::frag(as, wm0 + 32 * i + lr, 8 * c, h);
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = LB::frag(bs, wn0 + 32 * j + lr, 8 * c, h);
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
  float bias[TN];
  load_bias<TN, EPI>(ep, N, n0 + wn0, lr, bias);
  store_tile<TM, TN, EPI>(acc, C, ep, bias, M, N, ldc, m0 + wm0, n0 + wn0, lr, h);
}

// ------------------------------------------------------------------ DMA path
// 16-byte aligned operands with extents % 4 == 0 skip register staging: tiles
// go HBM -> LDS with global_load_lds_dwordx4 into an S-stage ring, so the
// loads of tiles t+1..t+S-2 are in flight while tile t is computed and one
// wave spends no VGPRs or VALU issue slots on staging.  One DMA instruction
// writes 64 consecutive 16-byte LDS units (lane i -> unit i); the lane -> HBM
// address map realises XOR-swizzled layouts whose fragment reads are bank
// conflict free without padding:
//   K-contiguous operand:  unit(row, q) = row*(BK/4) + (q ^ swz(row)),  q = k/4
//   row-contiguous operand: unit(k, p)  = k*(BR/4) + (p ^ 8*((k/4)&1)), p = row/4
// A ragged last K tile is loaded through registers with K predicates and
// written to the same layout.  The ring is synchronised by an explicit
// s_waitcnt on this wave's outstanding DMAs plus s_barrier.
//
// K groups (KG > 1): the workgroup runs KG groups of NW waves over one output
// tile, group g taking the g-th of KG consecutive runs of the block's K tiles
// through its own ring.  This multiplies the waves per SIMD of a grid of about
// one workgroup per CU (1024^3 on 64x64 tiles, 2048^3 on 128x128, the N = 384
// input gradients of the GPT step) without a second launch or a workspace.
// The groups share the ring barriers (a group out of tiles still takes
// part); at the end groups 1..KG-1 write their accumulators to LDS and group 0
// adds them in group order and stores: deterministic, no atomics.


// Row swizzle of the K-contiguous layout: rows that one 8- or 16-lane LDS
// pass reads (8 or 16 consecutive rows, same q) land in distinct banks.
template <int BK>
__device__ __forceinline__ int kc_swz(int row) {
  static_assert(BK == 16 || BK == 32 || BK == 64, "swizzle defined for BK 16, 32 and 64");
  if (BK == 16) return ((row >> 1) + (row >> 3)) & 3;
  if (BK == 32) return (row ^ (row >> 3)) & 7;
  return row & 15;  // 16 float4 groups per row: 16 consecutive rows, 16 distinct groups
}

template <int BR, int BK, int NW, bool KC>
struct DmaTile {
  static constexpr int kUnits = BR * BK / 4;
  static_assert(kUnits % (64 * NW) == 0, "tile must divide into whole wave DMAs");
  static_assert(KC || BR % 64 == 0, "row-contiguous swizzle pairs float4 groups p and p ^ 8 within BR");
  static constexpr int kPerWave = kUnits / (64 * NW);  // DMA instructions per wave per tile
  static constexpr int kFloats = BR * BK;

  uint32_t off[kPerWave];  // byte offset from the tile origin (rows clamped)

  __device__ __forceinline__ static void coords(int U, int& rr, int& kk) {
    if (KC) {
      rr = U / (BK / 4);
      kk = ((U % (BK / 4)) ^ kc_swz<BK>(rr)) * 4;
    } else {
      kk = U / (BR / 4);
      rr = ((U % (BR / 4)) ^ (((kk >> 2) & 1) * 8)) * 4;
    }
  }

  __device__ __forceinline__ static const char* origin(const float* P, int64_t ld, int64_t r0, int64_t k0) {
    return reinterpret_cast<const char*>(KC ? P + r0 * ld + k0 : P + k0 * ld + r0);
  }

  // Rows past the operand's extent are clamped onto its last row (last
  // float4 for the row-contiguous layout); they feed only accumulator rows or
  // columns the epilogue never stores.  The host guarantees BR*ld*4 < 2^32.
  __device__ __forceinline__ void init(int64_t ld, int64_t r0, int64_t R, int wave, int lane) {
    const int lim = (int)min<int64_t>(R - r0 - (KC ? 1 : 4), BR);
    const uint32_t uld = (uint32_t)ld;
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) {
      int rr, kk;
      coords((wave * kPerWave + i) * 64 + lane, rr, kk);
      const uint32_t r = (uint32_t)min(rr, lim);
      off[i] = (KC ? r * uld + (uint32_t)kk : (uint32_t)kk * uld + r) * 4u;
    }
  }

  __device__ __forceinline__ void issue(const float* __restrict__ P, int64_t ld, int64_t r0, int64_t k0,
                                        float* stage, int wave) const {
    const char* base = origin(P, ld, r0, k0);
#pragma unroll
    for (int i = 0; i < kPerWave; ++i)
      dma16(base + off[i], (lds_void_t*)(stage + (wave * kPerWave + i) * 256));
  }

  // Ragged last tile: k >= kend reads as zero ((kend - k0) % 4 == 0 for the
  // K-contiguous operand, so a unit is all in or all out).
  __device__ __forceinline__ void tail(const float* __restrict__ P, int64_t ld, int64_t r0, int64_t k0,
                                       int64_t kend, float* stage, int wave, int lane) const {
    const char* base = origin(P, ld, r0, k0);
    const int klim = (int)(kend - k0);
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) {
      const int U = (wave * kPerWave + i) * 64 + lane;
      int rr, kk;
      coords(U, rr, kk);
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (kk < klim) v = *reinterpret_cast<const f32x4*>(base + off[i]);
      *reinterpret_cast<f32x4*>(stage + U * 4) = v;
    }
  }

  // Fragment of chunk c (k = 8c + 4h + {0..3}) for tile row `row`.
  __device__ __forceinline__ static f32x4 frag(const float* __restrict__ S, int row, int c, int h) {
    if (KC) {
      const int U = row * (BK / 4) + ((2 * c + h) ^ kc_swz<BK>(row));
      return *reinterpret_cast<const f32x4*>(S + U * 4);
    } else {
      const float* p = S + (8 * c + 4 * h) * BR + (((row >> 2) ^ (8 * h)) << 2) + (row & 3);
      f32x4 v;
      v[0] = p[0];
      v[1] = p[BR];
      v[2] = p[2 * BR];
      v[3] = p[3 * BR];
      return v;
    }
  }
};



template <int BM, int BN, int BK, int WM, int WN, int WPE, int S, bool A_KC, bool B_KC, int EPI, int KG>
__global__ void __launch_bounds__((BM / WM) * (BN / WN) * KG * 64, WPE)
gemm_f32_dma_kernel(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C,
                    int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                    int64_t k_per_split, int64_t split_stride, int tiles_m, int tiles_n, int64_t sA,
                    int64_t sB, int64_t sC, GemmEpi ep) {
  constexpr int NWM = BM / WM;
  constexpr int NW = NWM * (BN / WN);  // waves per K group
  constexpr int TM = WM / 32;
  constexpr int TN = WN / 32;
  constexpr int NC = BK / 8;
  static_assert(S >= 2 && S <= 4, "ring depth 2..4");
  static_assert(KG >= 1 && NW * KG <= 16, "at most 1024 threads per workgroup");
  using TA = DmaTile<BM, BK, NW, A_KC>;
  using TB = DmaTile<BN, BK, NW, B_KC>;
  constexpr int kStage = TA::kFloats + TB::kFloats;
  constexpr int kPerTile = TA::kPerWave + TB::kPerWave;  // DMA instructions per wave per tile
  static_assert((S - 2) * kPerTile < 64, "outstanding DMAs exceed the vmcnt range");
  constexpr int kAccFloats = TM * TN * 16 * 64;  // one wave's accumulators
  static_assert(KG == 1 || KG * NW * kAccFloats <= KG * S * kStage, "K-group hand-over fits in the rings");

  __shared__ __attribute__((aligned(16))) float smem[KG * S * kStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wave index read into a scalar register: the group's tile range, the
  // ragged-tile test and the out-of-tiles test are then scalar branches.
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wv / NW;   // K group
  const int wave = wv % NW;  // wave within the group
  const int lr = lane & 31;
  const int h = lane >> 5;
  const int wm0 = (wave % NWM) * WM;
  const int wn0 = (wave / NWM) * WN;

  int tm, tn;
  map_tile(tiles_m, tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * BM;
  const int64_t n0 = (int64_t)tn * BN;

  // This block's K range, then this group's run of its tiles: groups take
  // ceil(tiles / KG) tiles each, in order; the ragged last tile belongs to the
  // group that reaches the range end.
  const int64_t kbeg0 = (int64_t)blockIdx.y * k_per_split;
  const int64_t kend = min(K, kbeg0 + k_per_split);
  const int nt_all = kend > kbeg0 ? (int)ceil_div(kend - kbeg0, (int64_t)BK) : 0;
  const int ntg = KG == 1 ? nt_all : (nt_all + KG - 1) / KG;  // loop trips, the same for every group
  const int t0 = grp * ntg;
  const int ntiles = max(0, min(nt_all - t0, ntg));
  const int64_t kbeg = kbeg0 + (int64_t)t0 * BK;
  const bool ragged = ntiles > 0 && t0 + ntiles == nt_all && ((kend - kbeg0) % BK) != 0;
  float* const ring = smem + grp * (S * kStage);
  C += (int64_t)blockIdx.y * split_stride;
  // batched launches: one grid layer per matrix (blockIdx.z)
  A += (int64_t)blockIdx.z * sA;
  B += (int64_t)blockIdx.z * sB;
  C += (int64_t)blockIdx.z * sC;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  TA ta;
  TB tb;
  ta.init(lda, m0, M, wave, lane);
  tb.init(ldb, n0, N, wave, lane);
  float bias[TN];
  load_bias<TN, EPI>(ep, N, n0 + wn0, lr, bias);
  uint32_t words[TM][TN];
  load_bits<TM, TN, EPI>(ep, M, N, m0 + wm0, n0 + wn0, lr, words);
  float csum[TM] = {};  // kEpiColsumA: this lane's running sum of A column wm0 + 32 i + lr
  auto issue = [&](int t) {
    const int64_t k0 = kbeg + (int64_t)t * BK;
    float* st = ring + (t % S) * kStage;
    if (ragged && t == ntiles - 1) {
      ta.tail(A, lda, m0, k0, kend, st, wave, lane);
      tb.tail(B, ldb, n0, k0, kend, st + TA::kFloats, wave, lane);
    } else {
      ta.issue(A, lda, m0, k0, st, wave);
      tb.issue(B, ldb, n0, k0, st + TA::kFloats, wave);
    }
  };
#pragma unroll
  for (int p = 0; p < S - 1; ++p)
    if (p < ntiles) issue(p);
  // kEpiColsumA (one K group, kbeg a multiple of 64): the residue mod tiles_n
  // of the 64-row chunk of the current K tile, stepped at each chunk end
  // rather than divided out in every trip (a 64-bit modulo by a runtime value
  // in the loop cost the 1536 x 384 x 16384 product several microseconds)
  int cs_res = 0;
  if constexpr (EPI == kEpiColsumA) cs_res = (int)((kbeg >> 6) % tiles_n);

  for (int t = 0; t < ntg; ++t) {
    // Tile t has landed once at most the DMAs of the tiles issued after it
    // (t+1 .. t+S-2) are outstanding.  A ragged tile's register loads wait
    // for every earlier DMA before its LDS stores, so counting it as a full
    // tile stays safe.
    const int ahead = min(S - 2, ntiles - 1 - t);
    if (S >= 4 && ahead == 2) wait_vm_lgkm0<(S >= 4 ? 2 : 0) * kPerTile>();
    else if (S >= 3 && ahead == 1) wait_vm_lgkm0<(S >= 3 ? 1 : 0) * kPerTile>();
    else wait_vm_lgkm0<0>();
    ring_barrier();
    if (KG > 1 && t >= ntiles) continue;  // this group is out of tiles; it still meets the barriers
    if (t + S - 1 < ntiles) issue(t + S - 1);  // refills the stage computed in iteration t-1

    const float* as = ring + (t % S) * kStage;
    const float* bs = as + TA::kFloats;
    // kEpiColsumA: whether this wave sums the A columns of this K tile (a
    // wave-uniform branch)
    const int64_t k0 = kbeg + (int64_t)t * BK;
    const bool cs_on = EPI == kEpiColsumA && wave < NWM && cs_res == tn;
    // With K groups four waves share a SIMD; the one issuing matrix ops
    // keeps priority over those issuing loads (measured +2.5 % at 1024^3).
    // One-group kernels lose slightly with it, except the 128x128x64 tile on
    // TN products (A/B in one process: 2048^3 127.0 -> 129.0 TF, the GPT
    // step's weight gradients 384 x 1536 x 16384 and 1536 x 384 x 16384 -2
    // us of 161; its NN and NT lose up to 1 %).
    constexpr bool kPrio = KG > 1 || (!A_KC && !B_KC && BM == 128 && BN == 128 && BK == 64 && WM == 32);
    if constexpr (kPrio) __builtin_amdgcn_s_setprio(1);
    f32x4 af[2][TM], bf[2][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) af[0][i] = TA::frag(as, wm0 + 32 * i + lr, 0, h);
#pragma unroll
    for (int j = 0; j < TN; ++j) bf[0][j] = TB::frag(bs, wn0 + 32 * j + lr, 0, h);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int p = c & 1;
      if (c + 1 < NC) {
#pragma unroll
        for (int i = 0; i < TM; ++i) af[p ^ 1][i] = TA::frag(as, wm0 + 32 * i + lr, c + 1, h);
#pragma unroll
        for (int j = 0; j < TN; ++j) bf[p ^ 1][j] = TB::frag(bs, wn0 + 32 * j + lr, c + 1, h);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[p][i][s], bf[p][j][s], acc[i][j], 0, 0, 0);
      if constexpr (EPI == kEpiColsumA) {
        if (cs_on) {
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) csum[i] += af[p][i][e];
        }
      }
    }
    if constexpr (kPrio) __builtin_amdgcn_s_setprio(0);
    if constexpr (EPI == kEpiColsumA) {
      if (((k0 + BK) & 63) == 0) {  // the chunk's last K tile
        if (cs_on) {
#pragma unroll
          for (int i = 0; i < TM; ++i) {
            const float tot = csum[i] + __uint_as_float(partner_u32(__float_as_uint(csum[i])));
            const int64_t m = m0 + wm0 + 32 * i + lr;
            if (h == 0 && m < M) ep.part[(k0 >> 6) * M + m] = tot;
            csum[i] = 0.f;
          }
        }
        cs_res = cs_res + 1 == tiles_n ? 0 : cs_res + 1;
      }
    }
  }

  if constexpr (KG > 1) {
    // Hand-over: every wave's DMAs have landed (the last trip waits for all),
    // and the barrier ends every read of the rings, which the partial sums
    // then overwrite.  Every group writes its sums (lane-major float4s:
    // conflict-free stores and loads); group g then adds the KG groups'
    // values of register quads [g*4/KG, (g+1)*4/KG) of each accumulator in
    // group order and stores those rows, so the adds and the stores are
    // spread over all groups.
    static_assert(4 % KG == 0, "register quads split evenly over the K groups");
    constexpr int QPG = 4 / KG;
    __syncthreads();
    {
      float* dst = smem + (grp * NW + wave) * kAccFloats + lane * 4;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<f32x4*>(dst + ((i * TN + j) * 4 + q) * 256) =
                f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
    }
    __syncthreads();
    const int q0 = grp * QPG;
    const float* src = smem + wave * kAccFloats + lane * 4;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int qq = 0; qq < QPG; ++qq) {
          const int o = ((i * TN + j) * 4 + q0 + qq) * 256;
          f32x4 v = *reinterpret_cast<const f32x4*>(src + o);
#pragma unroll
          for (int g = 1; g < KG; ++g) v += *reinterpret_cast<const f32x4*>(src + g * NW * kAccFloats + o);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[i][j][4 * qq + e] = v[e];
        }
    store_tile<TM, TN, EPI, QPG, true>(acc, C, ep, bias, M, N, ldc, m0 + wm0, n0 + wn0, lr, h, q0);
    return;
  }

  if constexpr (epi_bits(EPI)) {
    store_tile_bits<TM, TN, EPI>(acc, C, ep, bias, words, M, N, ldc, m0 + wm0, n0 + wn0, lr, h);
  } else {
    store_tile<TM, TN, EPI, 4, true>(acc, C, ep, bias, M, N, ldc, m0 + wm0, n0 + wn0, lr, h);
  }
}

// ------------------------------------------------------------ thin outputs
// C[M, N] with N <= 128 and a short contraction (16 <= K <= 512, K % 16 == 0):
// tall-skinny products such as a vocabulary head (16384 tokens x 65 classes
// x 384).  The tile configurations waste most of their work there: a 64-wide
// tile leaves a one-column remainder tile, and B's rows (N floats) are not
// 16-byte aligned for NN/TN.  Instead a 16-wave workgroup holds all of B,
// padded to NC = 16*NB columns, in LDS, staged by untracked 4-byte (NN/TN) or
// 16-byte (NT) DMAs, and its 64 rows of A stream HBM -> registers.  Waves are
// 4 row slabs x 4 K parts; a wave computes 16 rows x NC columns of its K
// part with v_mfma_f32_16x16x4f32: in each 16-deep k block, lane (i, q)
// supplies A[row i][4q .. 4q+3] as four consecutive k steps (one 128-bit
// load), and B the same four k values of column 16*nb + i.  The four parts
// of a slab are summed through LDS in a fixed order (deterministic).  Rows
// past M are clamped onto row M - 1 and columns past N onto column N - 1;
// both feed only outputs that are not stored.
//   NN, TN: B is [K][N]; LDS holds it as [k][c], row stride NC + 4 (the
//           four k rows of one 32-bit read land 16 banks apart).
//   NT:     B is [N][K]; LDS holds it as [chunk][c][64] in 64-deep k chunks,
//           float4 group g of column c at g ^ (c & 15), so the 128-bit reads
//           of 16 consecutive columns at one k hit 16 distinct bank quads
//           (measured 5 % faster than [c][k] rows of stride K + 4).
constexpr int kThinThreads = 1024;
constexpr int kThinSlabs = 4, kThinParts = 4;
constexpr int kThinRows = 16 * kThinSlabs;  // rows per workgroup
constexpr int kThinMaxKb = 8;               // 16-deep k blocks per part: K <= 512
constexpr int kThinLds = 32768;             // floats of LDS (128 KB)

__host__ __device__ constexpr int thin_ld_kn(int nb) { return 16 * nb + 4; }

// TAIL: the last column block holds 1..4 columns (N % 16 in 1..4).  Those
// are computed with VALU FMAs from the same A fragments instead of a fifth of
// the MFMA work (N = 65: 64 columns on MFMA, one by VALU); per lane the
// partial dot products of its four k steps are summed over the four k lanes
// of a row (lane ^ 16, then lane ^ 32) and over the K parts in part order.
// FLAT (NN/TN with B contiguous and 16-byte aligned): B is copied into LDS
// as it lies in HBM ([k][c], row stride N) by 16-byte DMAs, a quarter of the
// instructions of the padded form's 4-byte row DMAs (their staging time is
// what the 16-byte form saves; the fragment reads then meet some bank
// conflicts).
template <int NB, int OP, bool TAIL, bool FLAT>
__global__ void __launch_bounds__(kThinThreads, 1)
gemm_f32_thin_kernel(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M,
                     int N, int K, int64_t lda, int64_t ldb, int64_t ldc) {
  constexpr bool kNT = OP == AAR_GEMM_NT;
  constexpr bool kTN = OP == AAR_GEMM_TN;
  constexpr int NC = 16 * NB;
  constexpr int NBM = TAIL ? NB - 1 : NB;  // column blocks on MFMA
  static_assert(!TAIL || NB >= 2, "a tail follows at least one full column block");
  constexpr int kLdKn = thin_ld_kn(NB);
  static_assert(!(FLAT && OP == AAR_GEMM_NT), "the flat copy is the [K][N] layout of NN/TN");
  static_assert(kThinParts * kThinSlabs * 64 == kThinThreads, "16 waves: 4 slabs x 4 K parts");
  __shared__ __attribute__((aligned(16))) float lds[kThinLds];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int slab = wave % kThinSlabs, part = wave / kThinSlabs;
  const int li = lane & 15, lq = lane >> 4;
  const int kpart = (K / 16 + kThinParts - 1) / kThinParts * 16;
  const int kbase = part * kpart;
  const int nkb = max(0, min(K - kbase, kpart)) / 16;
  const int ldk = FLAT ? N : kLdKn;  // LDS row stride of the staged [k][c] B (NN/TN)

  // A fragments first, so their HBM latency overlaps the staging of B.
  const int64_t row = min((int64_t)blockIdx.x * kThinRows + slab * 16 + li, (int64_t)M - 1);
  f32x4 a[kThinMaxKb];
#pragma unroll
  for (int i = 0; i < kThinMaxKb; ++i) {
    if (i < nkb) {
      const int k = kbase + 16 * i + 4 * lq;
      if constexpr (kTN) {
        a[i] = f32x4{A[(int64_t)k * lda + row], A[(int64_t)(k + 1) * lda + row], A[(int64_t)(k + 2) * lda + row],
                     A[(int64_t)(k + 3) * lda + row]};
      } else {
        a[i] = *reinterpret_cast<const f32x4*>(A + row * lda + k);
      }
    }
  }

  if constexpr (kNT) {
    // one 16-byte DMA per 4 columns of a 64-deep chunk; lane (cl, gl) takes
    // float4 group gl ^ (col & 15) of column col = 4u + cl
    const int nchk = (K + 63) / 64;
    const int cl = lane >> 4, gl = lane & 15;
    for (int v = wave; v < nchk * (NC / 4); v += kThinThreads / 64) {
      const int ch = v / (NC / 4), u = v % (NC / 4);
      const int col = 4 * u + cl;
      const int k = 64 * ch + 4 * (gl ^ (col & 15));
      if (k < K) {
        dma16_untracked_s((uint32_t)(min(col, N - 1) * ldb + k) * 4u, B, (lds_void_t*)(lds + (ch * NC + 4 * u) * 64));
      }
    }
  } else if constexpr (FLAT) {
    // K * N floats (a multiple of 16: K % 16 == 0), 1 KB per instruction
    const int n4 = K * N / 4;
    for (int u = wave; u * 64 < n4; u += kThinThreads / 64) {
      if (u * 64 + lane < n4) dma16_untracked_s(lane * 16, B + u * 256, (lds_void_t*)(lds + u * 256));
    }
  } else {
    for (int k = wave; k < K; k += kThinThreads / 64) {
      const float* src = B + (int64_t)k * ldb;
      float* dst = lds + k * kLdKn;
      if (lane < NC) dma4_untracked_s(min(lane, N - 1) * 4, src, (lds_void_t*)dst);
      if (NC > 64 && lane < NC - 64) dma4_untracked_s(min(64 + lane, N - 1) * 4, src, (lds_void_t*)(dst + 64));
    }
  }
  wait_vm_lgkm0<0>();
  __syncthreads();

  f32x4 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 tail = {0.f, 0.f, 0.f, 0.f};  // tail columns 16 * NBM + t of row li, this lane's k steps
#pragma unroll
  for (int i = 0; i < kThinMaxKb; ++i) {
    if (i < nkb) {
      const int k = kbase + 16 * i + 4 * lq;
      if constexpr (TAIL) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          f32x4 bt;
          if constexpr (kNT) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const int c = 16 * NBM + t;
              bt[t] = lds[((k >> 6) * NC + c) * 64 + 4 * (((k & 63) >> 2) ^ (c & 15)) + j];
            }
          } else if constexpr (FLAT) {
            // columns past N read the next row (or, in the last row, past
            // the copy: the launcher keeps 64 floats of LDS spare); they
            // feed only tail sums that are never stored
            const float* r = lds + (k + j) * ldk + 16 * NBM;
            bt = f32x4{r[0], r[1], r[2], r[3]};
          } else {
            bt = *reinterpret_cast<const f32x4*>(lds + (k + j) * kLdKn + 16 * NBM);
          }
#pragma unroll
          for (int t = 0; t < 4; ++t) tail[t] = fmaf(a[i][j], bt[t], tail[t]);
        }
      }
#pragma unroll
      for (int nb = 0; nb < NBM; ++nb) {
        f32x4 b;
        if constexpr (kNT) {
          // column 16 nb + li: its low four bits are li
          b = *reinterpret_cast<const f32x4*>(lds + ((k >> 6) * NC + 16 * nb + li) * 64 + 4 * (((k & 63) >> 2) ^ li));
        } else {
          const float* col = lds + k * ldk + 16 * nb + li;
          b = f32x4{col[0], col[ldk], col[2 * ldk], col[3 * ldk]};
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][j], b[j], acc[nb], 0, 0, 0);
      }
    }
  }

  // Every part writes its sums to LDS (B is no longer read); then wave
  // (slab, p) adds the four parts of column blocks p, p + 4, ... in part
  // order and stores them, so the combine and the stores are spread over all
  // 16 waves.  Accumulator layout of a 16x16 block: lane (i, q), register r
  // holds row 4q + r, column i.
  if constexpr (TAIL) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      tail[t] += __shfl_xor(tail[t], 16, 64);
      tail[t] += __shfl_xor(tail[t], 32, 64);
    }
  }
  __syncthreads();
  // per part and slab: NBM accumulator blocks (256 floats each), then the
  // tail sums of the slab's 16 rows (64 floats)
  constexpr int kSlabFloats = NBM * 256 + (TAIL ? 64 : 0);
  constexpr int kPartStride = kThinSlabs * kSlabFloats;
  static_assert(kThinParts * kPartStride <= kThinLds, "the part combine fits in LDS");
  float* const hand = lds + slab * kSlabFloats;
#pragma unroll
  for (int nb = 0; nb < NBM; ++nb)
    *reinterpret_cast<f32x4*>(hand + part * kPartStride + nb * 256 + lane * 4) = acc[nb];
  if (TAIL && lq == 0) *reinterpret_cast<f32x4*>(hand + part * kPartStride + NBM * 256 + li * 4) = tail;
  __syncthreads();
  if (TAIL && part == NBM % kThinParts && lq == 0) {
    f32x4 t = *reinterpret_cast<const f32x4*>(hand + NBM * 256 + li * 4);
#pragma unroll
    for (int q = 1; q < kThinParts; ++q) t += *reinterpret_cast<const f32x4*>(hand + q * kPartStride + NBM * 256 + li * 4);
    const int64_t trow = (int64_t)blockIdx.x * kThinRows + slab * 16 + li;
    if (trow < M) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (16 * NBM + c < N) C[trow * ldc + 16 * NBM + c] = t[c];
      }
    }
  }
  const int64_t r0 = (int64_t)blockIdx.x * kThinRows + slab * 16 + 4 * lq;
#pragma unroll
  for (int nb = 0; nb < NBM; ++nb) {
    if (nb % kThinParts != part) continue;
    f32x4 v = *reinterpret_cast<const f32x4*>(hand + nb * 256 + lane * 4);
#pragma unroll
    for (int q = 1; q < kThinParts; ++q) v += *reinterpret_cast<const f32x4*>(hand + q * kPartStride + nb * 256 + lane * 4);
    const int col = 16 * nb + li;
    if (col >= N) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (r0 + r < M) C[(r0 + r) * ldc + col] = v[r];
    }
  }
}

// C[i] = sum_s W[s*stride + i], s in order 0..splits-1 (deterministic), four
// consecutive outputs per thread with 128-bit loads (stride % 4 == 0 and
// 16-byte aligned W/C); the split loop is unrolled so its loads overlap.
// The split-K sum of splitk_reduce_vec_kernel (no epilogue) in workgroups
// 0 .. nb_reduce - 1 and aar_colsum_f32's stage 2 of the A column sums
// (kEpiColsumA) in the rest, 4 columns each: one launch for both reductions
// of aar_gemm_f32_colsum_a.
constexpr int kCsaCols = 4;
__global__ void __launch_bounds__(kColsumSlices * kCsaCols)
splitk_reduce_colsum_kernel(const f32x4* __restrict__ W, f32x4* __restrict__ C, int64_t n4, int64_t stride4,
                            int splits, int nb_reduce, const float* __restrict__ part, float* __restrict__ colsum,
                            int nparts, int64_t cols) {
  static_assert(kColsumSlices * kCsaCols == 256, "the reduce workgroups take 256 float4s");
  __shared__ float acc[kColsumSlices][kCsaCols];
  if ((int)blockIdx.x < nb_reduce) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    f32x4 s = W[i];
#pragma unroll 8
    for (int p = 1; p < splits; ++p) s += W[p * stride4 + i];
    C[i] = s;
    return;
  }
  colsum_stage2_block<kCsaCols>(part, colsum, nparts, cols, (int64_t)(blockIdx.x - nb_reduce) * kCsaCols, acc);
}

// The epilogue (kEpi*; bias row-broadcast over the N columns, aux with C's
// layout; the vector kernel needs N % 4 == 0) is applied to the finished sum.
__global__ void __launch_bounds__(256)
splitk_reduce_vec_kernel(const f32x4* __restrict__ W, f32x4* __restrict__ C, int64_t n4, int64_t stride4,
                         int splits, int epi, const f32x4* __restrict__ bias, const f32x4* __restrict__ aux,
                         int64_t n_cols4) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  f32x4 s = W[i];
#pragma unroll 8
  for (int p = 1; p < splits; ++p) s += W[p * stride4 + i];
  if (epi == kEpiBias || epi == kEpiBiasRelu || epi == kEpiBiasAdd) s += bias[i % n_cols4];
  if (epi == kEpiBiasRelu) {
#pragma unroll
    for (int e = 0; e < 4; ++e) s[e] = fmaxf(0.0f, s[e]);
  }
  if (epi == kEpiMask) {
    const f32x4 a = aux[i];
#pragma unroll
    for (int e = 0; e < 4; ++e) s[e] = a[e] > 0.0f ? s[e] : 0.0f;
  }
  if (epi == kEpiAdd || epi == kEpiBiasAdd) s += aux[i];
  C[i] = s;
}

__global__ void __launch_bounds__(256)
splitk_reduce_kernel(const float* __restrict__ W, float* __restrict__ C, int64_t n, int64_t stride,
                     int splits, int epi, const float* __restrict__ bias, const float* __restrict__ aux,
                     int64_t n_cols) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float s = W[i];
#pragma unroll 8
  for (int p = 1; p < splits; ++p) s += W[p * stride + i];
  if (epi == kEpiBias || epi == kEpiBiasRelu || epi == kEpiBiasAdd) s += bias[i % n_cols];
  if (epi == kEpiBiasRelu) s = fmaxf(0.0f, s);
  if (epi == kEpiMask) s = aux[i] > 0.0f ? s : 0.0f;
  if (epi == kEpiAdd || epi == kEpiBiasAdd) s += aux[i];
  C[i] = s;
}

// Tile configurations.  `resident` is the number of workgroups one CU holds
// (LDS and register budget; it sets the kernel's launch bounds), `stages` the
// LDS ring depth of the DMA path, `eff` the fraction of the MFMA peak the
// configuration sustains on a fully occupied GPU (measured on MI355X at
// 4096^3, DMA path; the 256x128 shapes are rated below 128x128 because they
// lose to it at short K), `slots` the workgroups per CU below which the cost
// model charges an occupancy penalty, and `ops` the layouts the planner may
// pick it for.
constexpr int kAllOps = (1 << AAR_GEMM_NN) | (1 << AAR_GEMM_NT) | (1 << AAR_GEMM_TN);
struct Cfg {
  int bm, bn, bk, wm, wn, resident, stages;
  float eff;
  int slots, ops;
  int kg = 1;                  // K groups of the DMA path
  int split_ops = kAllOps;     // layouts for which the planner may split its K
};
constexpr Cfg kCfgs[] = {
    {256, 256, 32, 64, 128, 1, 2, 0.866f, 1, kAllOps},  // 0: 8 waves, 2 waves/SIMD; BK 32 halves the barriers
    {256, 128, 16, 128, 64, 2, 3, 0.83f, 2, kAllOps},   // 1
    {128, 256, 16, 64, 128, 2, 3, 0.83f, 2, kAllOps},   // 2
    {128, 128, 16, 64, 64, 2, 3, 0.84f, 2, kAllOps},    // 3
    {64, 64, 16, 32, 32, 4, 4, 0.77f, 4, kAllOps},      // 4
    {128, 64, 16, 64, 32, 3, 3, 0.78f, 3, kAllOps},     // 5
    {64, 128, 16, 32, 64, 3, 3, 0.80f, 3, kAllOps},     // 6
    {192, 192, 16, 96, 96, 1, 3, 0.80f, 1, kAllOps},    // 7: 4 waves; split-K weight gradients (N or M = 384, 1536)
    // 8: 4 waves of 64x96; for NN with N a multiple of 192 (the dX products
    // of the GPT step: +4-5 % over the 64x128 tile).  It keeps full speed
    // with one workgroup per CU, hence one model slot; as NT it loses at
    // N = 1152, so it is not planned there.  Unsplit TN products with many
    // rows take it too (16384 x 384 x 1536: 147.6 against 176.5 us); split
    // TN products lose with it (+25-28 % at 8 or 32 splits), so only NN
    // splits it.
    {128, 192, 32, 64, 96, 2, 2, 0.87f, 1, kAllOps, 1, 1 << AAR_GEMM_NN},
    // 9-12: K groups (see gemm_f32_dma_kernel), for grids of about one
    // workgroup per CU.  12 has a 96-wide N tile for thin outputs (the GPT
    // head, N = 65); its row-contiguous DMA layout needs BN % 64 == 0, so it
    // serves NT only.
    {64, 64, 32, 32, 32, 1, 2, 0.587f, 1, kAllOps, 4},           // 9: 16 waves
    {128, 128, 32, 64, 64, 1, 2, 0.826f, 1, kAllOps, 2},         // 10: 8 waves
    {64, 64, 32, 32, 32, 1, 3, 0.60f, 1, kAllOps, 2},            // 11: 8 waves
    {64, 96, 32, 32, 96, 1, 2, 0.55f, 1, 1 << AAR_GEMM_NT, 4},   // 12: 8 waves
    // 13: 8 waves, BK 64: half the barriers of 11 per K (1024^3: 22.0-22.9
    // us against 23.0-23.2 for 9 and 11)
    {64, 64, 64, 32, 32, 1, 2, 0.615f, 1, kAllOps, 2, 0},
    // 14: 8 waves of 32x64 over a 128x128 tile, BK 64, one K group (128 KB
    // of LDS): for grids of about one 128x128 tile per CU (2048^3: 129.2 /
    // 128.8 / 127.2 TF NN/NT/TN against 127.2 / 123.5 / 127.6 for 10)
    {128, 128, 64, 32, 64, 1, 2, 0.83f, 1, kAllOps},
    // 15: configuration 6 with two resident workgroups per CU and a 4-deep
    // ring (48 KB).  Not a candidate of its own: the planner substitutes it
    // for an unsplit plan on 6 whose grid holds at least 3 tiles per CU
    // (kDeepRingFor6).  A/B in one process, 6 -> 15, over 8 shapes of 3 to 16
    // tiles per CU (384 x 16384 x 384, 192 x 32768 x 1024, 16384 x 1152 x
    // 1536, 16384 x 2048 x 256, ...): faster in all 24 shape/layout pairs by
    // 0.7-4.6 %, e.g. the GPT qkv shape 16384 x 1152 x 384 NN/NT/TN 126.8 /
    // 124.7 / 130.2 -> 123.9 / 122.6 / 126.6 us.  (Changing 6 itself in the
    // planner's model moved 1140 of 17496 plans over a shape grid, mostly
    // small-M split products that were not measured, so 6 keeps its role.)
    {64, 128, 16, 32, 64, 2, 4, 0.80f, 3, kAllOps},
    // 16: configuration 8's 128x192 tile as 8 waves of 32x96 (one K group,
    // 80 KB).  Not a candidate of its own: the planner substitutes it for an
    // unsplit NN or NT plan on 8 whose grid is one workgroup per CU or a bit
    // less (kEightWaveFor8), where 8 runs one 4-wave workgroup per CU, one
    // wave per SIMD, and for an unsplit NT or TN plan on 6 whose 128 x 192
    // grid is three or more whole rounds (see plan_gemm).  Timed against 8
    // in one process: 16384 x 384 x 384 NN / NT 45.3 / 45.7 -> 42.5 / 42.6
    // us, x 1152 114.9 / 118.2 -> 110.9 / 113.1, x 1536 150.7 / 155.1 ->
    // 145.7 / 149.1 (bit-identical); TN lost 1 %, and grids of four tiles per
    // CU lost up to 9 %.  Its 32-row wave tiles do not take the mask-bit
    // epilogue.
    {128, 192, 32, 32, 96, 1, 2, 0.87f, 1, kAllOps},
};
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);
constexpr int kDeepRingFor6 = 15;
constexpr int kEightWaveFor8 = 16;
constexpr int kMaxSplits = 64;

struct Plan {
  int cfg;
  int splits;
  int64_t k_per_split;
};

int64_t split_chunk(int64_t K, int splits, int bk) { return ceil_div(ceil_div(K, (int64_t)splits), (int64_t)bk) * bk; }

// Cost model: blocks are spread evenly over the CUs; a CU holding fewer
// blocks than it has resident slots runs at reduced efficiency (down to 60%
// of `eff` with one block); split-K adds the partial-sum traffic and the
// reduction launch.  `eff` is fitted to the measured time of every
// (configuration, split) pair on the square, MLP and weight-gradient shapes
// of the GPT step plus a held-out shape set; the split counts tried are the
// measured ones.
constexpr int kPlanSplits[] = {1, 2, 3, 4, 6, 8, 12, 16, 24, 32};
constexpr int kNumPlanSplits = sizeof(kPlanSplits) / sizeof(kPlanSplits[0]);

// The thin-output kernel (gemm_f32_thin_kernel) has configuration id
// kThinCfg, past the tile configurations.  thin_shape_ok: the shapes it
// runs (B padded to 16-column blocks fits in its LDS); thin_operands_ok: the
// alignment its 128-bit A loads and (NT) 16-byte B DMAs need.
constexpr int kThinCfg = kNumCfgs;
bool thin_shape_ok(int op, int64_t M, int64_t N, int64_t K) {
  if (M < 1 || N < 1 || N > 128 || K < 16 || K > 16 * kThinMaxKb * kThinParts || K % 16 != 0) return false;
  const int64_t nb = ceil_div(N, (int64_t)16);
  const int64_t lds = op == AAR_GEMM_NT ? ceil_div(K, (int64_t)64) * 64 * 16 * nb : K * thin_ld_kn((int)nb);
  return lds <= kThinLds && ceil_div(M, (int64_t)kThinRows) * kThinThreads <= (int64_t)UINT32_MAX;
}
bool thin_operands_ok(int op, const float* A, const float* B, int64_t lda, int64_t ldb) {
  if (op != AAR_GEMM_TN && (!aligned16(A) || lda % 4 != 0)) return false;
  if (op == AAR_GEMM_NT && (!aligned16(B) || ldb % 4 != 0)) return false;
  return true;
}
// Where the thin kernel is planned.  Measured on MI355X (time against the
// best tile configuration and split): at M = 16384, NN/TN 0.51-0.55 for
// N = 65, K = 384 (the vocabulary head), 0.56-0.68 for N = 16, 0.77-0.83
// for N = 96, 0.97-0.99 for N = 128; NT 0.93 at N = 65, 1.00 at N = 96, 1.18
// at N = 128; M = 65536 0.77 (NN/TN); at M = 4096 (64 workgroups) it loses
// (1.07-1.35).  A workgroup takes a fixed ~5 us of staging on top of its
// MFMA work, so it needs rows enough to spread over most CUs.
bool thin_plan_wins(int op, int64_t M, int64_t N, int64_t K) {
  return M >= 8192 && K >= 64 && N <= (op == AAR_GEMM_NT ? 80 : 96);
}

// The short-operand kernels (gemm_small.hip) have configuration id
// kShortCfg: TN with at most 260 output rows (split over K) and NN with a
// contraction of at most 128.  They are planned for plain products whose
// operands the DMA path cannot stage (rows not 16-byte aligned), in place of
// the predicated register path: at the GPT step's vocabulary-65 shapes
// (16384 x 384 x 65 NN, 65 x 384 x 16384 TN) that path ran 20-27 us.
constexpr int kShortCfg = kThinCfg + 1;
bool short_plan_ok(int op, int64_t M, int64_t N, int64_t K) {
  if (op == AAR_GEMM_TN) return shortm_shape_ok(M, N, K) && K >= 1024;
  if (op == AAR_GEMM_NN) return shortk_shape_ok(M, N, K);
  return false;
}
// gemm_vec_ok's shape conditions alone (contiguous operands, aligned bases)
bool shape_vec_ok(int op, int64_t M, int64_t N, int64_t K) {
  switch (op) {
    case AAR_GEMM_NN: return K % 4 == 0 && N % 4 == 0;
    case AAR_GEMM_NT: return K % 4 == 0;
    default: return M % 4 == 0 && N % 4 == 0;
  }
}

// vec_ok: whether the DMA path can stage the operands (gemm_vec_ok); when it
// cannot, a plain product with a short operand takes the short kernels.
Plan plan_gemm(int op, int64_t M, int64_t N, int64_t K, size_t ws_bytes, bool allow_split, int64_t batch = 1,
               bool allow_thin = false, int epi = kEpiNone, bool vec_ok = true) {
  if (allow_thin && batch == 1 && thin_shape_ok(op, M, N, K) && thin_plan_wins(op, M, N, K)) return Plan{kThinCfg, 1, K};
  if (!vec_ok && batch == 1 && epi == kEpiNone && short_plan_ok(op, M, N, K)) {
    const int s = op == AAR_GEMM_TN ? shortm_splits(M, N, K, allow_split ? ws_bytes : 0) : 1;
    return Plan{kShortCfg, s, K};
  }
  const int cus = device_cu_count();
  const double cu_flops = 157.3e12 / 256;  // fp32 MFMA FLOP/s per CU
  Plan best{3, 1, K};
  double best_t = 1e300;
  for (int c = 0; c < kNumCfgs; ++c) {
    const Cfg& cf = kCfgs[c];
    if (!(cf.ops & (1 << op)) || c == kDeepRingFor6 || c == kEightWaveFor8) continue;
    const int64_t tiles = ceil_div(M, (int64_t)cf.bm) * ceil_div(N, (int64_t)cf.bn) * batch;
    // Configuration 8 as NT or TN: only grids of at most one round of its
    // resident workgroups, or of two or three whole rounds.  Measured at
    // 16384 rows (64 row tiles x N / 192), a partial last round loses to 3
    // and 6 by 9-17 % (N = 960, 1152) and grids of four or more rounds lose
    // to 0 by up to 4 %, while whole short grids gain 1-19 %.  With the bias
    // + relu and bias + residual epilogues of the GPT MLP it gains 1.5-2 %
    // over 3 and 6 (16384 x 1536 x 384: 158.5 against 161.0 us;
    // 16384 x 384 x 1536: 158.8 against 161.7 us).
    if (c == 8 && op != AAR_GEMM_NN) {
      const int64_t round = (int64_t)cus * cf.resident;
      if (!(tiles <= round || (tiles % round == 0 && tiles / round <= 3))) continue;
    }
    // the measured split counts, then the one that fills the CUs' slots in
    // one round
    const int64_t fill = (int64_t)cus * cf.slots / std::max<int64_t>(tiles, 1);
    for (int si = 0; si <= kNumPlanSplits; ++si) {
      const int splits = si < kNumPlanSplits ? kPlanSplits[si] : (int)std::min<int64_t>(fill, 64);
      if (si == kNumPlanSplits && (splits < 2 || std::count(kPlanSplits, kPlanSplits + kNumPlanSplits, splits))) break;
      if (splits > 1) {
        if (!allow_split || !(cf.split_ops & (1 << op))) break;
        if (K / splits < 256) {
          if (si < kNumPlanSplits) si = kNumPlanSplits - 1;  // still try the filling count
          continue;
        }
      }
      const int64_t kps = split_chunk(K, splits, cf.bk);
      const int64_t real_splits = ceil_div(K, kps);
      // the workspace the plan uses: its real split count, which rounding the
      // chunk to the tile depth can make smaller than the one asked for (and
      // the one aar_gemm_f32_workspace_bytes reports)
      if (real_splits > 1 && (size_t)real_splits * M * N * sizeof(float) > ws_bytes) {
        if (si < kNumPlanSplits) si = kNumPlanSplits - 1;
        continue;
      }
      const int64_t per_cu = ceil_div(tiles * real_splits, (int64_t)cus);
      const double occ = std::min(1.0, 0.6 + 0.4 * (double)per_cu / cf.slots);
      double t = (double)per_cu * 2.0 * cf.bm * cf.bn * (double)kps / (cf.eff * occ * cu_flops);
      if (real_splits > 1) t += 6e-6 + (double)(real_splits + 1) * M * N * 4.0 / 3e12;
      if (t < best_t) {
        best_t = t;
        best = Plan{c, (int)real_splits, kps};
      }
    }
  }
  // (the substitutions were measured on the DMA path; unaligned operands keep
  // the planned configuration)
  if (best.cfg == 6 && best.splits == 1 && vec_ok) {
    const int64_t tiles = ceil_div(M, (int64_t)kCfgs[6].bm) * ceil_div(N, (int64_t)kCfgs[6].bn) * batch;
    if (tiles >= 3 * (int64_t)cus) best.cfg = kDeepRingFor6;
  }
  if (best.splits == 1 && vec_ok && epi != kEpiMaskBits) {
    const int64_t tiles = ceil_div(M, (int64_t)kCfgs[8].bm) * ceil_div(N, (int64_t)kCfgs[8].bn) * batch;
    // an NN or NT plan on 8 over at most one tile per CU
    if (best.cfg == 8 && op != AAR_GEMM_TN && 2 * tiles > (int64_t)cus && tiles <= (int64_t)cus)
      best.cfg = kEightWaveFor8;
    // an NT or TN plan on 6 (or 15) whose 128 x 192 grid is three or more
    // whole rounds (16384 x 1152 x 384 to 32768 x 1152 x 384: -1.2 to -1.8 %
    // against 15; a partial last round, 4.5 rounds, lost 5 %)
    if ((best.cfg == 6 || best.cfg == kDeepRingFor6) && op != AAR_GEMM_NN && tiles % cus == 0 && tiles >= 3 * cus)
      best.cfg = kEightWaveFor8;
  }
  return best;
}

// Batched launches: `count` matrices at element strides sA / sB / sC.
struct Batch {
  int64_t count, sA, sB, sC;
};
constexpr Batch kSingle{1, 0, 0, 0};

template <int BM, int BN, int BK, int WM, int WN, int RES, int STAGES, int KG, bool A_KC, bool B_KC>
int launch_cfg(bool vec, const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
               int64_t lda, int64_t ldb, int64_t ldc, int splits, int64_t kps, int64_t split_stride,
               const Batch& bt, int epi, const GemmEpi& ep, hipStream_t st) {
  constexpr int kWaves = (BM / WM) * (BN / WN);
  constexpr int kWpe = (RES * kWaves * KG + 3) / 4;  // DMA path: KG groups of kWaves waves
  constexpr int kWpeReg = (RES * kWaves + 3) / 4;    // register path: one group
  const int tiles_m = (int)ceil_div(M, (int64_t)BM);
  const int tiles_n = (int)ceil_div(N, (int64_t)BN);
  // A dispatch holds each grid extent as a 32-bit work-item count.
  if ((int64_t)tiles_m * tiles_n * kWaves * KG * 64 > (int64_t)UINT32_MAX) return AAR_EUNSUPPORTED;
  dim3 grid((unsigned)(tiles_m * tiles_n), (unsigned)splits, (unsigned)bt.count);
  auto go = [&](auto epi_tag) {
    constexpr int E = decltype(epi_tag)::value;
    // The mask-bit epilogues and the A column sums run on the DMA path with
    // one K group only; kEpiMaskBits needs 64-row wave tiles (one column-sum
    // chunk per wave), kEpiColsumA K tiles that divide the 64-row chunks.
    if constexpr (epi_dma_only(E) && (KG > 1 || (E == kEpiMaskBits && WM != 64) ||
                                      (E == kEpiColsumA && 64 % BK != 0) || (!A_KC && BM % 64 != 0) ||
                                      (!B_KC && BN % 64 != 0))) {
      return AAR_EUNSUPPORTED;
    } else if constexpr (epi_dma_only(E)) {
      if (!vec) return AAR_EUNSUPPORTED;
      gemm_f32_dma_kernel<BM, BN, BK, WM, WN, kWpe, STAGES, A_KC, B_KC, E, KG><<<grid, dim3(kWaves * KG * 64), 0, st>>>(
          A, B, C, M, N, K, lda, ldb, ldc, kps, split_stride, tiles_m, tiles_n, bt.sA, bt.sB, bt.sC, ep);
      return launch_status();
    } else {
      if constexpr ((!A_KC && BM % 64 != 0) || (!B_KC && BN % 64 != 0)) {
        if (vec) return AAR_EUNSUPPORTED;  // no DMA layout for this row-contiguous tile
      } else if (vec) {
        gemm_f32_dma_kernel<BM, BN, BK, WM, WN, kWpe, STAGES, A_KC, B_KC, E, KG>
            <<<grid, dim3(kWaves * KG * 64), 0, st>>>(A, B, C, M, N, K, lda, ldb, ldc, kps, split_stride, tiles_m,
                                                      tiles_n, bt.sA, bt.sB, bt.sC, ep);
        return launch_status();
      }
      gemm_f32_kernel<BM, BN, BK, WM, WN, kWpeReg, A_KC, B_KC, E><<<grid, dim3(kWaves * 64), 0, st>>>(
          A, B, C, M, N, K, lda, ldb, ldc, kps, split_stride, tiles_m, tiles_n, bt.sA, bt.sB, bt.sC, ep);
      return launch_status();
    }
  };
  // bias + relu and the residual adds are instantiated for the linear layer's
  // x W^T (NT) only, the relu mask for its input gradient dY W (NN) only.
  switch (epi) {
    case kEpiNone: return go(std::integral_constant<int, kEpiNone>{});
    case kEpiBias: return go(std::integral_constant<int, kEpiBias>{});
    case kEpiBiasRelu:
      if constexpr (A_KC && B_KC) return go(std::integral_constant<int, kEpiBiasRelu>{});
      return AAR_EUNSUPPORTED;
    case kEpiAdd:
      if constexpr (A_KC && B_KC) return go(std::integral_constant<int, kEpiAdd>{});
      return AAR_EUNSUPPORTED;
    case kEpiBiasAdd:
      if constexpr (A_KC && B_KC) return go(std::integral_constant<int, kEpiBiasAdd>{});
      return AAR_EUNSUPPORTED;
    case kEpiMask:
      if constexpr (A_KC && !B_KC) return go(std::integral_constant<int, kEpiMask>{});
      return AAR_EUNSUPPORTED;
    case kEpiBiasReluBits:
      if constexpr (A_KC && B_KC) return go(std::integral_constant<int, kEpiBiasReluBits>{});
      return AAR_EUNSUPPORTED;
    case kEpiMaskBits:
      if constexpr (A_KC && !B_KC) return go(std::integral_constant<int, kEpiMaskBits>{});
      return AAR_EUNSUPPORTED;
    case kEpiColsumA:
      if constexpr (!A_KC && !B_KC) return go(std::integral_constant<int, kEpiColsumA>{});
      return AAR_EUNSUPPORTED;
    default: return AAR_EINVAL;
  }
}

template <bool A_KC, bool B_KC>
int launch_op(int cfg, bool vec, const float* A, const float* B, float* C, int64_t M, int64_t N,
              int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int splits, int64_t kps,
              int64_t split_stride, const Batch& bt, int epi, const GemmEpi& ep, hipStream_t st) {
#define AAR_GEMM_CFG(I)                                                                                   \
  case I:                                                                                                 \
    return launch_cfg<kCfgs[I].bm, kCfgs[I].bn, kCfgs[I].bk, kCfgs[I].wm, kCfgs[I].wn, kCfgs[I].resident, \
                      kCfgs[I].stages, kCfgs[I].kg, A_KC, B_KC>(vec, A, B, C, M, N, K, lda, ldb, ldc, splits, kps, \
                                                                split_stride, bt, epi, ep, st);
  switch (cfg) {
    AAR_GEMM_CFG(0)
    AAR_GEMM_CFG(1)
    AAR_GEMM_CFG(2)
    AAR_GEMM_CFG(3)
    AAR_GEMM_CFG(4)
    AAR_GEMM_CFG(5)
    AAR_GEMM_CFG(6)
    AAR_GEMM_CFG(7)
    AAR_GEMM_CFG(8)
    AAR_GEMM_CFG(9)
    AAR_GEMM_CFG(10)
    AAR_GEMM_CFG(11)
    AAR_GEMM_CFG(12)
    AAR_GEMM_CFG(13)
    AAR_GEMM_CFG(14)
    AAR_GEMM_CFG(15)
    AAR_GEMM_CFG(16)
    default:
      return AAR_EINVAL;
  }
#undef AAR_GEMM_CFG
}
static_assert(kNumCfgs == 17, "launch_op lists every configuration");

// 128-bit loads need 16-byte aligned operands whose contiguous extents and
// leading dimensions are multiples of 4, and the 32-bit per-thread offsets
// need BR*ld*4 < 2^32.
constexpr int64_t kMaxLd = (int64_t(1) << 32) / (4 * 256) - 1;
bool gemm_vec_ok(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B, int64_t lda,
                 int64_t ldb) {
  if (!aligned16(A) || !aligned16(B)) return false;
  if (lda % 4 != 0 || ldb % 4 != 0 || lda > kMaxLd || ldb > kMaxLd) return false;
  switch (op) {
    case AAR_GEMM_NN: return (K % 4 == 0) && (N % 4 == 0);
    case AAR_GEMM_NT: return (K % 4 == 0);
    default: return (M % 4 == 0) && (N % 4 == 0);
  }
}

int default_ld(int op, int64_t M, int64_t N, int64_t K, int64_t& lda, int64_t& ldb) {
  switch (op) {
    case AAR_GEMM_NN: lda = K; ldb = N; break;
    case AAR_GEMM_NT: lda = K; ldb = K; break;
    default: lda = M; ldb = N; break;
  }
  return AAR_OK;
}

int dispatch_op(int op, int cfg, bool vec, const float* A, const float* B, float* C, int64_t M, int64_t N,
                int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int splits, int64_t kps, int64_t split_stride,
                const Batch& bt, hipStream_t st, int epi = kEpiNone, const GemmEpi& ep = GemmEpi{}) {
  switch (op) {
    case AAR_GEMM_NN:
      return launch_op<true, false>(cfg, vec, A, B, C, M, N, K, lda, ldb, ldc, splits, kps, split_stride, bt, epi,
                                    ep, st);
    case AAR_GEMM_NT:
      return launch_op<true, true>(cfg, vec, A, B, C, M, N, K, lda, ldb, ldc, splits, kps, split_stride, bt, epi,
                                   ep, st);
    default:
      return launch_op<false, false>(cfg, vec, A, B, C, M, N, K, lda, ldb, ldc, splits, kps, split_stride, bt,
                                     epi, ep, st);
  }
}

template <int OP>
int launch_thin(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                int64_t ldc, hipStream_t st) {
  const dim3 grid((unsigned)ceil_div(M, (int64_t)kThinRows));
  const bool tail = N > 16 && N % 16 >= 1 && N % 16 <= 4;
  // (the fragment reads of padding columns run up to 15 floats past the copy)
  const bool flat = OP != AAR_GEMM_NT && ldb == N && aligned16(B) && K * N + 64 <= kThinLds;
  auto go = [&](auto nb_tag) {
    constexpr int NBV = decltype(nb_tag)::value;
    auto launch = [&](auto kern) {
      kern<<<grid, dim3(kThinThreads), 0, st>>>(A, B, C, (int)M, (int)N, (int)K, lda, ldb, ldc);
      return launch_status();
    };
    if constexpr (OP != AAR_GEMM_NT) {
      if constexpr (NBV >= 2) {
        if (tail) return flat ? launch(gemm_f32_thin_kernel<NBV, OP, true, true>)
                              : launch(gemm_f32_thin_kernel<NBV, OP, true, false>);
      }
      return flat ? launch(gemm_f32_thin_kernel<NBV, OP, false, true>)
                  : launch(gemm_f32_thin_kernel<NBV, OP, false, false>);
    } else {
      if constexpr (NBV >= 2) {
        if (tail) return launch(gemm_f32_thin_kernel<NBV, OP, true, false>);
      }
      return launch(gemm_f32_thin_kernel<NBV, OP, false, false>);
    }
  };
  switch (ceil_div(N, (int64_t)16)) {
    case 1: return go(std::integral_constant<int, 1>{});
    case 2: return go(std::integral_constant<int, 2>{});
    case 3: return go(std::integral_constant<int, 3>{});
    case 4: return go(std::integral_constant<int, 4>{});
    case 5: return go(std::integral_constant<int, 5>{});
    case 6: return go(std::integral_constant<int, 6>{});
    case 7: return go(std::integral_constant<int, 7>{});
    case 8: return go(std::integral_constant<int, 8>{});
    default: return AAR_EUNSUPPORTED;
  }
}

// The thin-output kernel on contiguous operands (no epilogue, no split).
int run_thin(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B, float* C, hipStream_t st) {
  int64_t lda, ldb;
  default_ld(op, M, N, K, lda, ldb);
  if (!thin_shape_ok(op, M, N, K) || !thin_operands_ok(op, A, B, lda, ldb)) return AAR_EUNSUPPORTED;
  switch (op) {
    case AAR_GEMM_NN: return launch_thin<AAR_GEMM_NN>(A, B, C, M, N, K, lda, ldb, N, st);
    case AAR_GEMM_NT: return launch_thin<AAR_GEMM_NT>(A, B, C, M, N, K, lda, ldb, N, st);
    default: return launch_thin<AAR_GEMM_TN>(A, B, C, M, N, K, lda, ldb, N, st);
  }
}

// epi / ep: the epilogue (kEpi*), applied in an unsplit launch or after the
// split-K reduction.  C is contiguous (ldc = N), and so is ep.aux.
int run_gemm(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B, float* C,
             void* workspace, const Plan& p, hipStream_t st, int epi = kEpiNone, const GemmEpi& ep = GemmEpi{}) {
  int64_t lda, ldb;
  default_ld(op, M, N, K, lda, ldb);
  const bool vec = gemm_vec_ok(op, M, N, K, A, B, lda, ldb);
  float* out = p.splits > 1 ? static_cast<float*>(workspace) : C;
  const int64_t split_stride = p.splits > 1 ? M * N : 0;
  // kEpiColsumA works in the main loop of every split; the others apply to
  // the finished sum, in the reduction when K is split
  const int main_epi = p.splits > 1 && epi != kEpiColsumA ? kEpiNone : epi;
  int rc = dispatch_op(op, p.cfg, vec, A, B, out, M, N, K, lda, ldb, N, p.splits, p.k_per_split, split_stride,
                       kSingle, st, main_epi, ep);
  if (rc != AAR_OK || p.splits <= 1) return rc;
  if (epi == kEpiColsumA) epi = kEpiNone;
  const int64_t n = M * N;
  if (n % 4 == 0 && aligned16(out) && aligned16(C) && (!ep.bias || (N % 4 == 0 && aligned16(ep.bias))) &&
      (!ep.aux || aligned16(ep.aux))) {
    splitk_reduce_vec_kernel<<<dim3((unsigned)ceil_div(n / 4, (int64_t)256)), dim3(256), 0, st>>>(
        reinterpret_cast<const f32x4*>(out), reinterpret_cast<f32x4*>(C), n / 4, split_stride / 4, p.splits, epi,
        reinterpret_cast<const f32x4*>(ep.bias), reinterpret_cast<const f32x4*>(ep.aux), N / 4);
  } else {
    splitk_reduce_kernel<<<dim3((unsigned)ceil_div(n, (int64_t)256)), dim3(256), 0, st>>>(
        out, C, n, split_stride, p.splits, epi, ep.bias, ep.aux, N);
  }
  return launch_status();
}

// The short-operand kernels on contiguous operands (no epilogue).
int run_short(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B, float* C, int splits,
              void* workspace, size_t ws_bytes, hipStream_t st) {
  if (op == AAR_GEMM_TN) return run_shortm(A, nullptr, B, C, M, N, K, splits, workspace, ws_bytes, st);
  if (op == AAR_GEMM_NN && splits == 1) return run_shortk(A, B, C, M, N, K, st);
  return op == AAR_GEMM_NN ? AAR_EINVAL : AAR_EUNSUPPORTED;
}

// Shared argument checks; returns AAR_OK to proceed, 1 when there is nothing
// to compute, or an error code.
int check_gemm_args(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B, float* C,
                    void* stream) {
  if (op < 0 || op > 2 || M < 0 || N < 0 || K < 0) return AAR_EINVAL;
  if (M == 0 || N == 0) return 1;
  if (!C) return AAR_EINVAL;
  if (K == 0) {
    const int rc = aar_memset_zero(C, (size_t)M * N * sizeof(float), stream);
    return rc == AAR_OK ? 1 : rc;
  }
  if (!A || !B) return AAR_EINVAL;
  if (M > INT32_MAX / 2 || N > INT32_MAX / 2) return AAR_EUNSUPPORTED;
  return AAR_OK;
}

}  // namespace
}  // namespace aar

using namespace aar;

extern "C" size_t aar_gemm_f32_workspace_bytes(int op, int64_t M, int64_t N, int64_t K) {
  if (op < 0 || op > 2 || M <= 0 || N <= 0 || K <= 0) return 0;
  const Plan p = plan_gemm(op, M, N, K, (size_t)-1, true, 1, true, kEpiNone, shape_vec_ok(op, M, N, K));
  if (p.cfg == kShortCfg) return shortm_workspace_bytes(M, N, K, p.splits);
  if (p.splits <= 1) return 0;
  return (size_t)p.splits * (size_t)M * (size_t)N * sizeof(float);
}

extern "C" int aar_gemm_f32(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B,
                            float* C, void* workspace, size_t workspace_bytes, void* stream) {
  const int chk = check_gemm_args(op, M, N, K, A, B, C, stream);
  if (chk != AAR_OK) return chk == 1 ? AAR_OK : chk;
  int64_t lda, ldb;
  default_ld(op, M, N, K, lda, ldb);
  const bool vec = gemm_vec_ok(op, M, N, K, A, B, lda, ldb);
  Plan p = plan_gemm(op, M, N, K, workspace ? workspace_bytes : 0, workspace != nullptr, 1,
                     thin_operands_ok(op, A, B, lda, ldb), kEpiNone, vec);
  if (p.cfg == kThinCfg) return run_thin(op, M, N, K, A, B, C, as_stream(stream));
  if (p.cfg == kShortCfg) {
    const int rc = run_short(op, M, N, K, A, B, C, p.splits, workspace, workspace_bytes, as_stream(stream));
    if (rc != AAR_EUNSUPPORTED) return rc;
    // (an operand alignment the short kernels do not take either)
    p = plan_gemm(op, M, N, K, workspace ? workspace_bytes : 0, workspace != nullptr, 1, false);
  }
  return run_gemm(op, M, N, K, A, B, C, workspace, p, as_stream(stream));
}

extern "C" int aar_gemm_f32_bias(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B,
                                 const float* bias, float* C, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  if (op < 0 || op > 2 || M < 0 || N < 0 || K < 0) return AAR_EINVAL;
  if (M == 0 || N == 0) return AAR_OK;
  if (!bias) return AAR_EINVAL;
  if (K == 0) return AAR_EUNSUPPORTED;  // C = bias rows: not a product, left to the caller
  const int chk = check_gemm_args(op, M, N, K, A, B, C, stream);
  if (chk != AAR_OK) return chk;
  const Plan p = plan_gemm(op, M, N, K, workspace ? workspace_bytes : 0, workspace != nullptr, 1, false, kEpiBias);
  return run_gemm(op, M, N, K, A, B, C, workspace, p, as_stream(stream), kEpiBias, GemmEpi{bias, nullptr});
}

extern "C" int aar_gemm_f32_bias_relu(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B,
                                      const float* bias, float* C, void* workspace, size_t workspace_bytes,
                                      void* stream) {
  if (op < 0 || op > 2 || M < 0 || N < 0 || K < 0) return AAR_EINVAL;
  if (M == 0 || N == 0) return AAR_OK;
  if (!bias) return AAR_EINVAL;
  if (op != AAR_GEMM_NT || K == 0) return AAR_EUNSUPPORTED;
  const int chk = check_gemm_args(op, M, N, K, A, B, C, stream);
  if (chk != AAR_OK) return chk;
  const Plan p = plan_gemm(op, M, N, K, workspace ? workspace_bytes : 0, workspace != nullptr, 1, false, kEpiBiasRelu);
  return run_gemm(op, M, N, K, A, B, C, workspace, p, as_stream(stream), kEpiBiasRelu, GemmEpi{bias, nullptr});
}

// C = op(A, B) + R (R with C's layout), the product planned as the plain
// aar_gemm_f32 plans it, so C is bit for bit the plain product followed by
// an add (a plan that takes the thin-output kernel, which has no epilogue,
// runs the product and then the add).  NT only (the linear layer's layout).
extern "C" int aar_gemm_f32_add(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B,
                                const float* R, float* C, void* workspace, size_t workspace_bytes, void* stream) {
  if (op < 0 || op > 2 || M < 0 || N < 0 || K < 0) return AAR_EINVAL;
  if (M == 0 || N == 0) return AAR_OK;
  if (!R) return AAR_EINVAL;
  if (op != AAR_GEMM_NT || K == 0) return AAR_EUNSUPPORTED;
  const int chk = check_gemm_args(op, M, N, K, A, B, C, stream);
  if (chk != AAR_OK) return chk;
  int64_t lda, ldb;
  default_ld(op, M, N, K, lda, ldb);
  const Plan p = plan_gemm(op, M, N, K, workspace ? workspace_bytes : 0, workspace != nullptr, 1,
                           thin_operands_ok(op, A, B, lda, ldb));
  if (p.cfg == kThinCfg) {
    const int rc = run_thin(op, M, N, K, A, B, C, as_stream(stream));
    return rc != AAR_OK ? rc : aar_add_f32(C, R, C, M * N, stream);
  }
  return run_gemm(op, M, N, K, A, B, C, workspace, p, as_stream(stream), kEpiAdd, GemmEpi{nullptr, R});
}

// C = (op(A, B) + bias) + R, planned as aar_gemm_f32_bias plans it: bit for
// bit that call followed by an add.  NT only.
extern "C" int aar_gemm_f32_bias_add(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B,
                                     const float* bias, const float* R, float* C, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  if (op < 0 || op > 2 || M < 0 || N < 0 || K < 0) return AAR_EINVAL;
  if (M == 0 || N == 0) return AAR_OK;
  if (!bias || !R) return AAR_EINVAL;
  if (op != AAR_GEMM_NT || K == 0) return AAR_EUNSUPPORTED;
  const int chk = check_gemm_args(op, M, N, K, A, B, C, stream);
  if (chk != AAR_OK) return chk;
  const Plan p = plan_gemm(op, M, N, K, workspace ? workspace_bytes : 0, workspace != nullptr, 1, false, kEpiBias);
  return run_gemm(op, M, N, K, A, B, C, workspace, p, as_stream(stream), kEpiBiasAdd, GemmEpi{bias, R});
}

extern "C" int aar_gemm_f32_relu_mask(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B,
                                      const float* mask, float* C, void* workspace, size_t workspace_bytes,
                                      void* stream) {
  if (op < 0 || op > 2 || M < 0 || N < 0 || K < 0) return AAR_EINVAL;
  if (M == 0 || N == 0) return AAR_OK;
  if (!mask) return AAR_EINVAL;
  if (op != AAR_GEMM_NN) return AAR_EUNSUPPORTED;
  const int chk = check_gemm_args(op, M, N, K, A, B, C, stream);
  if (chk != AAR_OK) return chk == 1 ? AAR_OK : chk;  // K == 0: C = 0, which the mask keeps
  // planned as aar_gemm_f32 plans the product (the mask does not change the
  // NN plan), so C is bit for bit that product masked; a thin-kernel plan,
  // which has no epilogue, runs the product and then the mask pass
  int64_t lda, ldb;
  default_ld(op, M, N, K, lda, ldb);
  const Plan p = plan_gemm(op, M, N, K, workspace ? workspace_bytes : 0, workspace != nullptr, 1,
                           thin_operands_ok(op, A, B, lda, ldb), kEpiMask);
  if (p.cfg == kThinCfg) {
    const int rc = run_thin(op, M, N, K, A, B, C, as_stream(stream));
    return rc != AAR_OK ? rc : aar_relu_bwd_f32(C, mask, C, M * N, stream);
  }
  return run_gemm(op, M, N, K, A, B, C, workspace, p, as_stream(stream), kEpiMask, GemmEpi{nullptr, mask});
}

// aar_gemm_f32_bias_relu's plan and values, plus the relu's mask as bits
// (kEpiBiasReluBits).  Plans without that epilogue return AAR_EUNSUPPORTED
// before anything is launched.
extern "C" int aar_gemm_f32_bias_relu_bits(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B,
                                           const float* bias, float* C, uint32_t* bits, void* workspace,
                                           size_t workspace_bytes, void* stream) {
  if (op < 0 || op > 2 || M < 0 || N < 0 || K < 0) return AAR_EINVAL;
  if (M == 0 || N == 0) return AAR_OK;
  if (!bias || !bits) return AAR_EINVAL;
  if (op != AAR_GEMM_NT || K == 0) return AAR_EUNSUPPORTED;
  const int chk = check_gemm_args(op, M, N, K, A, B, C, stream);
  if (chk != AAR_OK) return chk;
  const Plan p = plan_gemm(op, M, N, K, workspace ? workspace_bytes : 0, workspace != nullptr, 1, false, kEpiBiasRelu);
  if (p.splits > 1) return AAR_EUNSUPPORTED;
  GemmEpi ep{bias, nullptr};
  ep.bits = bits;
  return run_gemm(op, M, N, K, A, B, C, nullptr, p, as_stream(stream), kEpiBiasReluBits, ep);
}

extern "C" size_t aar_gemm_f32_mask_bits_colsum_workspace_bytes(int64_t M, int64_t N) {
  if (M <= 0 || N <= 0) return 0;
  return (size_t)ceil_div(M, (int64_t)64) * (size_t)N * sizeof(float);
}

// The product planned as aar_gemm_f32 plans it with the workspace it asks
// for, masked by the bits in the epilogue (kEpiMaskBits), which also writes
// aar_colsum_f32's stage-1 partials of the masked product; colsum's stage 2
// finishes them.  Plans without that epilogue return AAR_EUNSUPPORTED before
// anything is launched.
extern "C" int aar_gemm_f32_mask_bits_colsum(int op, int64_t M, int64_t N, int64_t K, const float* A,
                                             const float* B, const uint32_t* bits, float* C, float* colsum,
                                             void* workspace, size_t workspace_bytes, void* stream) {
  if (op < 0 || op > 2 || M < 0 || N < 0 || K < 0) return AAR_EINVAL;
  if (N == 0) return AAR_OK;
  if (M == 0) return colsum ? aar_memset_zero(colsum, (size_t)N * sizeof(float), stream) : AAR_OK;
  if (!bits) return AAR_EINVAL;
  if (op != AAR_GEMM_NN || K == 0 || (colsum && !colsum_chunks_of_64(M))) return AAR_EUNSUPPORTED;
  const int chk = check_gemm_args(op, M, N, K, A, B, C, stream);
  if (chk != AAR_OK) return chk;
  if (colsum && (!workspace || workspace_bytes < aar_gemm_f32_mask_bits_colsum_workspace_bytes(M, N))) {
    return AAR_EWORKSPACE;
  }
  int64_t lda, ldb;
  default_ld(op, M, N, K, lda, ldb);
  const bool vec = gemm_vec_ok(op, M, N, K, A, B, lda, ldb);
  const Plan p = plan_gemm(op, M, N, K, (size_t)-1, true, 1, thin_operands_ok(op, A, B, lda, ldb), kEpiMaskBits, vec);
  if (p.splits > 1 || p.cfg >= kNumCfgs) return AAR_EUNSUPPORTED;
  GemmEpi ep{nullptr, nullptr};
  ep.bits = const_cast<uint32_t*>(bits);
  ep.part = colsum ? static_cast<float*>(workspace) : nullptr;  // no colsum: the mask only
  hipStream_t st = as_stream(stream);
  const int rc = run_gemm(op, M, N, K, A, B, C, nullptr, p, st, kEpiMaskBits, ep);
  if (rc != AAR_OK || !colsum) return rc;
  return colsum_finish(ep.part, colsum, (int)(M / 64), N, st);
}

// The product planned as aar_gemm_f32 plans it with the workspace it asks for
// (its split partials first in the workspace), with aar_colsum_f32's stage-1
// partials of A ([K, M]) summed in the main loop (kEpiColsumA) after them;
// colsum's stage 2 finishes them.
namespace aar {
namespace {
Plan colsum_a_plan(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B, bool& vec) {
  int64_t lda, ldb;
  default_ld(op, M, N, K, lda, ldb);
  vec = gemm_vec_ok(op, M, N, K, A, B, lda, ldb);
  return plan_gemm(op, M, N, K, (size_t)-1, true, 1, thin_operands_ok(op, A, B, lda, ldb), kEpiNone, vec);
}
size_t colsum_a_split_bytes(const Plan& p, int64_t M, int64_t N) {
  return p.splits > 1 ? ceil_div((int64_t)p.splits * M * N * (int64_t)sizeof(float), (int64_t)256) * 256 : 0;
}
}  // namespace
}  // namespace aar

extern "C" size_t aar_gemm_f32_colsum_a_workspace_bytes(int op, int64_t M, int64_t N, int64_t K) {
  if (op != AAR_GEMM_TN || M <= 0 || N <= 0 || K <= 0) return 0;
  bool vec;
  const Plan p = colsum_a_plan(op, M, N, K, nullptr, nullptr, vec);  // the shape's plan (aligned operands)
  return colsum_a_split_bytes(p, M, N) + (size_t)ceil_div(K, (int64_t)64) * (size_t)M * sizeof(float);
}

extern "C" int aar_gemm_f32_colsum_a(int op, int64_t M, int64_t N, int64_t K, const float* A, const float* B,
                                     float* C, float* colsum, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  if (op < 0 || op > 2 || M < 0 || N < 0 || K < 0) return AAR_EINVAL;
  if (M == 0) return AAR_OK;
  if (!colsum) return AAR_EINVAL;
  if (op != AAR_GEMM_TN || N == 0 || K == 0 || !colsum_chunks_of_64(K)) return AAR_EUNSUPPORTED;
  const int chk = check_gemm_args(op, M, N, K, A, B, C, stream);
  if (chk != AAR_OK) return chk;
  bool vec;
  const Plan p = colsum_a_plan(op, M, N, K, A, B, vec);
  if (!vec || p.cfg >= kNumCfgs || p.k_per_split % 64 != 0) return AAR_EUNSUPPORTED;
  const size_t split_bytes = colsum_a_split_bytes(p, M, N);
  if (!workspace || workspace_bytes < split_bytes + (size_t)(K / 64) * (size_t)M * sizeof(float)) {
    return AAR_EWORKSPACE;
  }
  GemmEpi ep{nullptr, nullptr};
  ep.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + split_bytes);
  hipStream_t st = as_stream(stream);
  const int nparts = (int)(K / 64);
  float* out = p.splits > 1 ? static_cast<float*>(workspace) : C;
  if (p.splits <= 1 || !aligned16(C) || !aligned16(workspace)) {
    const int rc = run_gemm(op, M, N, K, A, B, C, workspace, p, st, kEpiColsumA, ep);
    if (rc != AAR_OK) return rc;
    return colsum_finish(ep.part, colsum, nparts, M, st);
  }
  // split: the products, then one launch for the split-K sum and colsum's
  // stage 2 (M * N % 4 == 0: TN on the DMA path has M % 4 == N % 4 == 0)
  int64_t lda, ldb;
  default_ld(op, M, N, K, lda, ldb);
  const int64_t split_stride = M * N;
  int rc = dispatch_op(op, p.cfg, vec, A, B, out, M, N, K, lda, ldb, N, p.splits, p.k_per_split, split_stride,
                       kSingle, st, kEpiColsumA, ep);
  if (rc != AAR_OK) return rc;
  const int64_t n4 = M * N / 4;
  const int nb = (int)ceil_div(n4, (int64_t)256);
  splitk_reduce_colsum_kernel<<<dim3((unsigned)(nb + ceil_div(M, (int64_t)kCsaCols))), dim3(256), 0, st>>>(
      reinterpret_cast<const f32x4*>(out), reinterpret_cast<f32x4*>(C), n4, split_stride / 4, p.splits, nb, ep.part,
      colsum, nparts, M);
  return launch_status();
}

extern "C" int aar_gemm_f32_tile_config(int config, int* tile_m, int* tile_n, int* tile_k) {
  if (config < 0 || config >= kNumCfgs) return AAR_EINVAL;
  if (tile_m) *tile_m = kCfgs[config].bm;
  if (tile_n) *tile_n = kCfgs[config].bn;
  if (tile_k) *tile_k = kCfgs[config].bk;
  return AAR_OK;
}

extern "C" int aar_gemm_f32_plan(int op, int64_t M, int64_t N, int64_t K, size_t workspace_bytes,
                                 int* config, int* splits) {
  if (op < 0 || op > 2 || M <= 0 || N <= 0 || K <= 0) return AAR_EINVAL;
  const Plan p = plan_gemm(op, M, N, K, workspace_bytes, workspace_bytes > 0, 1, true, kEpiNone,
                           shape_vec_ok(op, M, N, K));
  if (config) *config = p.cfg;
  if (splits) *splits = p.splits;
  return AAR_OK;
}

extern "C" int aar_gemm_f32_with_config(int op, int64_t M, int64_t N, int64_t K, const float* A,
                                        const float* B, float* C, void* workspace, size_t workspace_bytes,
                                        int config, int splits, void* stream) {
  if (config < 0 || config > kShortCfg || splits < 1 || splits > kMaxSplits) return AAR_EINVAL;
  if (config == kThinCfg && splits != 1) return AAR_EINVAL;
  const int chk = check_gemm_args(op, M, N, K, A, B, C, stream);
  if (chk != AAR_OK) return chk == 1 ? AAR_OK : chk;
  if (config == kThinCfg) return run_thin(op, M, N, K, A, B, C, as_stream(stream));
  if (config == kShortCfg) {
    if ((op == AAR_GEMM_TN && !shortm_shape_ok(M, N, K)) || (op == AAR_GEMM_NN && !shortk_shape_ok(M, N, K)))
      return AAR_EUNSUPPORTED;
    return run_short(op, M, N, K, A, B, C, splits, workspace, workspace_bytes, as_stream(stream));
  }
  const int64_t kps = split_chunk(K, splits, kCfgs[config].bk);
  const int real_splits = (int)ceil_div(K, kps);
  if (real_splits > 1 && (!workspace || workspace_bytes < (size_t)real_splits * M * N * sizeof(float)))
    return AAR_EWORKSPACE;
  return run_gemm(op, M, N, K, A, B, C, workspace, Plan{config, real_splits, kps}, as_stream(stream));
}

extern "C" int aar_gemm_f32_batched(int op, int64_t batch, int64_t M, int64_t N, int64_t K, const float* A,
                                    int64_t lda, int64_t strideA, const float* B, int64_t ldb, int64_t strideB,
                                    float* C, int64_t ldc, int64_t strideC, void* stream) {
  if (op < 0 || op > 2 || batch < 0 || M < 0 || N < 0 || K < 0) return AAR_EINVAL;
  if (batch == 0 || M == 0 || N == 0) return AAR_OK;
  if (!C || ldc < N) return AAR_EINVAL;
  if (K == 0) {
    if (ldc != N || (batch > 1 && strideC != M * N)) return AAR_EUNSUPPORTED;
    return aar_memset_zero(C, (size_t)(batch * M * N) * sizeof(float), stream);
  }
  if (!A || !B) return AAR_EINVAL;
  const int64_t need_a = op == AAR_GEMM_TN ? M : K, need_b = op == AAR_GEMM_NT ? K : N;
  if (lda < need_a || ldb < need_b) return AAR_EINVAL;
  if (M > INT32_MAX / 2 || N > INT32_MAX / 2) return AAR_EUNSUPPORTED;
  const bool vec = gemm_vec_ok(op, M, N, K, A, B, lda, ldb) && strideA % 4 == 0 && strideB % 4 == 0;
  // the operands' alignment keeps the DMA-path substitutions off unaligned
  // batches; a short-kernel plan (one unaligned matrix) is not run here, so
  // that case plans the tile kernels
  Plan p = plan_gemm(op, M, N, K, 0, false, batch, false, kEpiNone, vec);
  if (p.cfg >= kNumCfgs) p = plan_gemm(op, M, N, K, 0, false, batch);
  // Batches ride blockIdx.z (at most 65535 per launch): larger counts go in
  // consecutive launches (offsets keep the 16-byte alignment, strides % 4 == 0).
  constexpr int64_t kMaxGridZ = 65535;
  for (int64_t b0 = 0; b0 < batch; b0 += kMaxGridZ) {
    const int64_t nb = std::min(kMaxGridZ, batch - b0);
    const int rc = dispatch_op(op, p.cfg, vec, A + b0 * strideA, B + b0 * strideB, C + b0 * strideC, M, N, K, lda,
                               ldb, ldc, 1, p.k_per_split, 0, Batch{nb, strideA, strideB, strideC},
                               as_stream(stream));
    if (rc != AAR_OK) return rc;
  }
  return AAR_OK;
}
