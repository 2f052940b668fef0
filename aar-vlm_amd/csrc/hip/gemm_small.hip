// Short-operand fp32 GEMMs on CDNA4 matrix cores (v_mfma_f32_32x32x2f32):
// the vocabulary-sized products of a language-model step, whose operands have
// rows of an odd number of floats (a 65-character vocabulary), so the tiled
// DMA kernels of gemm_f32.hip, which need 16-byte aligned rows, do not apply.
//   TN short M  C[M, N] = A[K, M]^T . B[K, N], M <= 260, long K: the head's
//               weight gradient dlogits^T . x (reference matmul_at_b,
//               cppsrc/ops/matmul.cu:549-645), and the embedding weight
//               gradient onehot(ids)^T . dY with the one-hot values made in
//               registers from the ids (reference embedding backward,
//               cppsrc/ops/embedding.cpp:60-104, which adds rows atomically).
//   NN short K  C[M, N] = A[M, K] . B[K, N], K <= 128: the head's input
//               gradient dlogits . W (reference matmul, matmul.cu:345-444).
// Design:
//  * A block of consecutive rows of a contiguous operand is one contiguous
//    run of memory whatever its row length, so it is copied HBM -> LDS flat,
//    by 16-byte DMAs when it starts 16-byte aligned (4-byte DMAs otherwise),
//    and read from LDS with the row stride it has in HBM.  An odd stride
//    (65) puts 32 consecutive rows of one column in 32 distinct banks.
//  * MFMA covers 32-row blocks; the last M % 32 <= 4 rows (TN) or K % 8 <= 7
//    contraction steps (NN) that do not fill an MFMA step are done by VALU
//    FMAs, so a 65-row product does 64 rows of MFMA work, not 96.
//  * TN splits K over workgroups; the partial products are summed in split
//    order by a second launch, so results are deterministic (no atomics).
//  * MFMA operand convention as in gemm_f32.hip: in chunk step s (0..3) lane
//    half h supplies k = kc + 4h + s; accumulator register r of lane
//    (lr, h) holds row 8*(r/4) + 4h + r%4, column lr of its 32x32 block.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "gemm_small.hpp"

namespace aar {
namespace {

// ------------------------------------------------------------ TN, short M
constexpr int kSmBK = 64;        // k rows per staged tile
constexpr int kSmBN = 64;        // output columns per workgroup (two 32-column blocks)
constexpr int kSmThreads = 256;  // 4 waves: 2 column blocks x 2 row-block phases
constexpr int kSmMaxIds = 2048;  // one-hot form: ids staged per workgroup (bounds its K chunk)
constexpr int kSmMinChunk = 128; // K rows per workgroup, at least

// MT: 32-row blocks on MFMA (even: each wave takes MT/2 of them in one
// column block); M <= 32*MT + 4, the rows past 32*MT done by VALU.
//   kRa   A DMA instructions per wave per k tile (the same count for every
//         wave: lanes past the tile load a clamped address into padding, so
//         the wait for a tile is one compile-time vmcnt)
//   kD    all DMA instructions per wave per k tile (A, then 2 for B)
//   kS    LDS ring stages: up to 4, as LDS allows, with every DMA of the
//         ring countable by vmcnt (kS * kD <= 63); 0: not supported
template <int MT, bool ONEHOT, bool A16>
struct ShortM {
  static constexpr int kAFloats = ONEHOT ? 4 : (2 * MT + 1) * 1024;  // >= 64*(32*MT+4) + 32*MT over-read
  static constexpr int kRa = ONEHOT ? 0 : (A16 ? 2 * MT + 1 : 8 * MT + 1);
  static constexpr int kD = kRa + kSmBK * kSmBN / 4 / kSmThreads;
  static constexpr int kStage = kAFloats + kSmBK * kSmBN;
  static constexpr int kIds = ONEHOT ? kSmMaxIds * 4 : 0;
  // stages for two workgroups per CU if at least two fit, else for one
  static constexpr int kS2 = (80 * 1024 - kIds) / (kStage * 4);
  static constexpr int kS1 = (160 * 1024 - kIds) / (kStage * 4);
  static constexpr int kSLds = kS2 >= 2 ? kS2 : kS1;
  static constexpr int kSv = kSLds < 4 ? kSLds : 4;
  static constexpr int kS = kSv * kD <= 63 ? kSv : 63 / kD;
  static constexpr bool kOk = kS >= 2;
  static constexpr int kSafeS = kOk ? kS : 1;  // an unsupported instance (never launched) still compiles
};

// One workgroup: output columns [n0, n0 + 64) of all M rows, over K rows
// [kb, kb + kc) of its split; writes its partial product to out + split *
// split_stride (C itself when there is one split).  k tiles of 64 rows go
// through a kS-stage LDS ring: kS - 1 tiles are in flight while one is
// computed (untracked DMAs; the wait at the top of an iteration leaves the
// later tiles' kD instructions each outstanding, the barrier after it frees
// the stage computed last).  A ragged last tile is loaded by plain loads and
// zero-padded.
template <int MT, bool ONEHOT, bool A16>
__global__ void __launch_bounds__(kSmThreads)
gemm_tn_shortm_kernel(const float* __restrict__ A, const int64_t* __restrict__ ids, const float* __restrict__ B,
                      float* __restrict__ out, int M, int N, int64_t K, int64_t kc, int64_t split_stride) {
  using P = ShortM<MT, ONEHOT, A16>;
  constexpr int TMW = MT / 2;
  constexpr int S = P::kSafeS, D = P::kD;
  constexpr int kW1 = D < 63 ? D : 63, kW2 = 2 * D < 63 ? 2 * D : 63, kW3 = 3 * D < 63 ? 3 * D : 63;
  __shared__ __attribute__((aligned(16))) float As[S][P::kAFloats];
  __shared__ __attribute__((aligned(16))) float Bs[S][kSmBK * kSmBN];
  __shared__ int Is[ONEHOT ? kSmMaxIds : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, h = lane >> 5;
  const int ntn = (N + kSmBN - 1) / kSmBN;
  // The hardware deals workgroups round-robin over the 8 XCDs: block b runs
  // on XCD b % 8.  All column tiles of one split get the same b % 8, so the
  // split's A rows (read by each of them) and B rows (a slice each) are
  // fetched into one XCD's L2.  Blocks past the last split exit.
  const unsigned xcd = blockIdx.x & 7u, r8 = blockIdx.x >> 3;
  const int tn = (int)(r8 % (unsigned)ntn);
  const int split = (int)(8u * (r8 / (unsigned)ntn) + xcd);
  if ((int64_t)split * kc >= K) return;
  const int n0 = tn * kSmBN;
  const int64_t kb = (int64_t)split * kc;
  const int nk = (int)(min(K, kb + kc) - kb);  // >= 1: the grid has no empty split
  const int ntiles = (nk + kSmBK - 1) / kSmBK;
  const bool ragged = nk % kSmBK != 0;
  constexpr int mt = 32 * MT;
  const int tail = M > mt ? M - mt : 0;        // 0..4 rows by VALU
  const int nb = wave & 1, mb0 = wave >> 1;

  if constexpr (ONEHOT) {
    for (int i = tid; i < nk; i += kSmThreads) {
      const int64_t v = ids[kb + i];
      Is[i] = (v >= 0 && v < M) ? (int)v : -1;
    }
  }

  // DMA instruction j (0 .. kD-1) of full tile t: A rounds, then B rounds
  auto dma_one = [&](int t, int j) {
    const int st = t % S;
    const int64_t k0 = kb + (int64_t)t * kSmBK;
    if (j < P::kRa) {
      const float* asrc = A + k0 * M;
      const int u = j * kSmThreads + wave * kWave;
      if constexpr (A16) {
        const int last = kSmBK / 4 * M - 1;  // float4 units of the tile: kSmBK rows x M floats
        dma16_untracked(asrc + 4 * min(u + lane, last), (lds_void_t*)(&As[st][4 * u]));
      } else {
        const int last = kSmBK * M - 1;
        dma4_untracked(asrc + min(u + lane, last), (lds_void_t*)(&As[st][u]));
      }
    } else {
      // B: kSmBK rows x 16 float4 groups; groups past N are clamped onto the
      // last one (they feed only columns that are not stored)
      const int u = (j - P::kRa) * kSmThreads + wave * kWave;
      const int g = u + lane;
      const int row = g / (kSmBN / 4);
      const int col = min(n0 + 4 * (g % (kSmBN / 4)), N - 4);
      dma16_untracked(B + (k0 + row) * N + col, (lds_void_t*)(&Bs[st][u * 4]));
    }
  };
  auto is_ragged = [&](int t) { return ragged && t == ntiles - 1; };
  // a ragged last tile: plain loads, zero-padded
  auto load_ragged = [&](int t) {
    const int st = t % S;
    const int64_t k0 = kb + (int64_t)t * kSmBK;
    const int kr = nk - t * kSmBK;
    if constexpr (!ONEHOT) {
      const float* asrc = A + k0 * M;
      for (int i = tid; i < kSmBK * M; i += kSmThreads) As[st][i] = i < kr * M ? asrc[i] : 0.0f;
    }
    const float* bsrc = B + k0 * N;
    for (int i = tid; i < kSmBK * kSmBN; i += kSmThreads) {
      const int row = i / kSmBN, col = min(n0 + i % kSmBN, N - 1);
      Bs[st][i] = row < kr ? bsrc[(int64_t)row * N + col] : 0.0f;
    }
  };
  auto stage = [&](int t) {
    if (is_ragged(t)) {
      load_ragged(t);
      return;
    }
#pragma unroll
    for (int j = 0; j < D; ++j) dma_one(t, j);
  };

  // two accumulators per row block, for even and odd MFMA steps: a chain of
  // dependent MFMAs issues one per MFMA latency, two interleaved chains keep
  // the matrix pipe busy; they are added at the end
  f32x16 acc[TMW], acc2[TMW];
#pragma unroll
  for (int i = 0; i < TMW; ++i) acc[i] = acc2[i] = f32x16{};
  float tacc[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // rows mt .. mt + tail - 1, this wave's k slices

  // vmcnt wait leaving `later` tiles' DMAs (kD each) in flight; counts past
  // 63 wait for more than needed
  auto wait_later = [&](int later) {
    if (later <= 0) {
      wait_vm_lgkm0<0>();
    } else if (later == 1) {
      wait_vm_lgkm0<kW1>();
    } else if (later == 2) {
      wait_vm_lgkm0<kW2>();
    } else {
      wait_vm_lgkm0<kW3>();
    }
  };

  for (int t = 0; t < min(S - 1, ntiles); ++t) stage(t);
  for (int t = 0; t < ntiles; ++t) {
    // tiles t+1 .. min(ntiles-1, t+S-2) may stay in flight; the barrier
    // after the wait also frees the stage computed last, which takes tile
    // t + S - 1
    wait_later(min(ntiles - 1, t + S - 2) - t);
    __syncthreads();
    // Tile t + S - 1: a dense-A tile's DMAs are spread through this tile's
    // MFMA chain (one every few MFMAs): a SIMD issuing MFMAs back to back
    // was measured to hold off DMA traffic that was issued ahead of them.
    const int tn_next = t + S - 1;
    const bool spread = !ONEHOT && tn_next < ntiles && !is_ragged(tn_next);
    if (tn_next < ntiles && !spread) stage(tn_next);
    const int st = t % S;
    const float* as = As[st];
    const float* bs = Bs[st];
    // step q of the MFMA chain is k = 8 (q / 4) + 4h + q % 4; the tile's
    // operands are read first, one batch, the chains follow
    constexpr int Q = kSmBK / 2;
    float bf[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) bf[q] = bs[(8 * (q >> 2) + 4 * h + (q & 3)) * kSmBN + 32 * nb + lr];
    if constexpr (ONEHOT) {
      // A row block none of whose 32 ids occurs in this tile is all zeros:
      // its MFMAs are skipped (a wave-uniform test).  With position ids
      // (consecutive) one block of the tile is non-zero.
      int idk[Q];
#pragma unroll
      for (int q = 0; q < Q; ++q) idk[q] = Is[t * kSmBK + 8 * (q >> 2) + 4 * h + (q & 3)];
      unsigned long long present[TMW];
#pragma unroll
      for (int i = 0; i < TMW; ++i) present[i] = 0;
#pragma unroll
      for (int u = 0; u < kSmBK / 32; ++u) {
        const int blk = Is[t * kSmBK + 32 * u + lr] >> 5;  // -1 for ids out of range
#pragma unroll
        for (int i = 0; i < TMW; ++i) present[i] |= __ballot(blk == mb0 + 2 * i);
      }
#pragma unroll
      for (int i = 0; i < TMW; ++i) {
        if (present[i] == 0) continue;
        const int m = 32 * (mb0 + 2 * i) + lr;
#pragma unroll
        for (int q = 0; q < Q; q += 2) {
          acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(idk[q] == m ? 1.0f : 0.0f, bf[q], acc[i], 0, 0, 0);
          acc2[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(idk[q + 1] == m ? 1.0f : 0.0f, bf[q + 1], acc2[i], 0, 0, 0);
        }
      }
    } else {
      float af[TMW][Q];
#pragma unroll
      for (int i = 0; i < TMW; ++i) {
#pragma unroll
        for (int q = 0; q < Q; ++q) af[i][q] = as[(8 * (q >> 2) + 4 * h + (q & 3)) * M + 32 * (mb0 + 2 * i) + lr];
      }
      constexpr int kEvery = Q / 2 / D > 0 ? Q / 2 / D : 1;  // MFMA pairs per DMA
#pragma unroll
      for (int q = 0; q < Q; q += 2) {
#pragma unroll
        for (int i = 0; i < TMW; ++i) {
          acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][q], bf[q], acc[i], 0, 0, 0);
          acc2[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][q + 1], bf[q + 1], acc2[i], 0, 0, 0);
        }
        if ((q / 2) % kEvery == 0 && (q / 2) / kEvery < D) {
          if (spread) dma_one(tn_next, (q / 2) / kEvery);
        }
      }
      if constexpr (Q / 2 / kEvery < D) {  // the rest, if the chain is shorter than kD pairs
        if (spread) {
#pragma unroll
          for (int j = Q / 2 / kEvery; j < D; ++j) dma_one(tn_next, j);
        }
      }
    }
    // rows past the MFMA blocks: lane = column, wave w takes the tile's k in
    // [w KW, (w + 1) KW)
    if (tail > 0) {
      constexpr int KW = kSmBK / 4;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (r >= tail) break;
        const int m = mt + r;
#pragma unroll
        for (int kk = 0; kk < KW; ++kk) {
          const int k = KW * wave + kk;
          float a;
          if constexpr (ONEHOT) {
            a = Is[t * kSmBK + k] == m ? 1.0f : 0.0f;
          } else {
            a = as[k * M + m];
          }
          tacc[r] = fmaf(a, bs[k * kSmBN + lane], tacc[r]);
        }
      }
    }
  }

  if (tail > 0) {  // the four waves' k slices, summed in wave order
    __syncthreads();
    float* red = Bs[0];
#pragma unroll
    for (int r = 0; r < 4; ++r) red[(wave * 4 + r) * kWave + lane] = tacc[r];
    __syncthreads();
    if (wave < tail && n0 + lane < N) {
      float v = red[(0 * 4 + wave) * kWave + lane];
#pragma unroll
      for (int w = 1; w < 4; ++w) v += red[(w * 4 + wave) * kWave + lane];
      tacc[0] = v;
    }
  }

  float* o = out + (int64_t)split * split_stride;
  const int col = n0 + 32 * nb + lr;
  if (col < N) {
#pragma unroll
    for (int i = 0; i < TMW; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 32 * (mb0 + 2 * i) + 8 * (r / 4) + 4 * h + (r % 4);
        if (row < M) o[(int64_t)row * N + col] = acc[i][r] + acc2[i][r];
      }
    }
  }
  if (wave < tail && n0 + lane < N) o[(int64_t)(mt + wave) * N + n0 + lane] = tacc[0];
}

// C[i] = sum over the splits of W[s * stride + i], four outputs per group
// of four lanes: lane q of a group sums splits [q*c, (q+1)*c) in order (its
// loads issued together), and the four sums are combined as (s0 + s1) +
// (s2 + s3) by two lane exchanges, so the order is fixed (deterministic) and
// each lane waits for one round of loads instead of all the splits in turn.
__global__ void __launch_bounds__(256)
shortm_reduce_kernel(const f32x4* __restrict__ W, f32x4* __restrict__ C, int64_t n4, int64_t stride4, int splits) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t i = t >> 2;
  const int q = (int)(t & 3);
  const int per = (splits + 3) >> 2;
  const int p0 = q * per, p1 = min(splits, p0 + per);
  f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
  if (i < n4) {
#pragma unroll 16
    for (int p = p0; p < p1; ++p) s += W[p * stride4 + i];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) s[e] += __shfl_xor(s[e], 1, 64);
#pragma unroll
  for (int e = 0; e < 4; ++e) s[e] += __shfl_xor(s[e], 2, 64);
  if (i < n4 && q == 0) C[i] = s;
}

// MFMA row blocks for M rows: the rows past an even number of 32-row blocks
// go to VALU when there are at most 4 of them, else the blocks are padded.
int shortm_blocks(int64_t M) {
  const int full = (int)(M / 32), rem = (int)(M % 32);
  if (full >= 2 && full % 2 == 0 && rem <= 4) return full;
  const int up = (int)ceil_div(M, (int64_t)32);
  return std::max(2, up + (up & 1));
}

int64_t shortm_chunk(int64_t K, int splits, bool onehot) {
  int64_t kc = ceil_div(ceil_div(K, (int64_t)splits), (int64_t)kSmBK) * kSmBK;
  if (onehot) kc = std::min<int64_t>(kc, kSmMaxIds);
  return kc;
}

// ------------------------------------------------------------ NN, short K
constexpr int kSkBM = 128;        // rows per workgroup: 4 row slabs of 32
constexpr int kSkThreads = 512;   // 8 waves: 4 row slabs x 2 column halves

template <int KMAX, int BN>
struct ShortK {
  static constexpr int kA = (kSkBM * KMAX + 3) / 4 * 4;
  static constexpr int kFloats = kA + KMAX * BN;
};

// One workgroup: C rows [m0, m0 + 128) x columns [n0, n0 + BN); a wave owns
// 32 rows x BN/2 columns (BN/64 MFMA blocks).  The A rows (one contiguous
// run of 128*K floats) and the K x BN block of B are staged once; rows of A
// past M are left unloaded (they feed only rows that are not stored),
// columns of B past N are clamped onto the last float4 group.  BN = 192 makes
// the GPT head's input gradient (16384 x 384 x 65) 256 workgroups, one per
// CU, so every SIMD gets the same MFMA work.
template <int KMAX, int BN, bool A16>
__global__ void __launch_bounds__(kSkThreads)
gemm_nn_shortk_kernel(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N,
                      int K) {
  constexpr int TNW = BN / 64;
  __shared__ __attribute__((aligned(16))) float lds[ShortK<KMAX, BN>::kFloats];
  float* const As = lds;
  float* const Bs = lds + ShortK<KMAX, BN>::kA;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, h = lane >> 5;
  const int ntn = (N + BN - 1) / BN;
  // block b runs on XCD b % 8: the column tiles of one row tile share it, so
  // their A rows are fetched into one L2; blocks past the last row tile exit
  const unsigned xcd = blockIdx.x & 7u, r8 = blockIdx.x >> 3;
  const int tn = (int)(r8 % (unsigned)ntn);
  const int64_t m0 = (int64_t)(8u * (r8 / (unsigned)ntn) + xcd) * kSkBM;
  if (m0 >= M) return;
  const int n0 = tn * BN;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * (BN / 2);

  {
    const float* asrc = A + m0 * K;
    const int na = (int)std::min<int64_t>(kSkBM, M - m0) * K;
    int done = 0;
    if constexpr (A16) {
      const int n4 = na / 4;
      for (int u = wave * kWave; u < n4; u += kSkThreads) {
        if (u + lane < n4) dma16_untracked(asrc + (u + lane) * 4, (lds_void_t*)(As + u * 4));
      }
      done = n4 * 4;
    }
    for (int u = done + wave * kWave; u < na; u += kSkThreads) {
      if (u + lane < na) dma4_untracked(asrc + u + lane, (lds_void_t*)(As + u));
    }
    const int n4b = K * (BN / 4);
    for (int u = wave * kWave; u < n4b; u += kSkThreads) {
      const int g = u + lane;
      if (g < n4b) {
        const int row = g / (BN / 4);
        const int col = min(n0 + 4 * (g % (BN / 4)), N - 4);
        dma16_untracked(B + (int64_t)row * N + col, (lds_void_t*)(Bs + u * 4));
      }
    }
  }
  wait_vm_lgkm0<0>();
  __syncthreads();

  f32x16 acc[TNW];
#pragma unroll
  for (int j = 0; j < TNW; ++j) acc[j] = f32x16{};
  const int nchunk = K / 8, k8 = 8 * nchunk;
  // fragments of 8-deep chunk c (k = 8c + 4h + s): loaded one chunk ahead of
  // its MFMAs, so the LDS latency runs under the previous chunk's work
  auto load = [&](int c, float (&a)[4], float (&b)[4][TNW]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int k = 8 * c + 4 * h + s;
      a[s] = As[(wm + lr) * K + k];
#pragma unroll
      for (int j = 0; j < TNW; ++j) b[s][j] = Bs[k * BN + wn + 32 * j + lr];
    }
  };
  auto mma = [&](const float (&a)[4], const float (&b)[4][TNW]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int j = 0; j < TNW; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b[s][j], acc[j], 0, 0, 0);
    }
  };
  float a0[4], b0[4][TNW], a1[4], b1[4][TNW];
  if (nchunk > 0) load(0, a0, b0);
  for (int c = 0; c < nchunk; c += 2) {
    if (c + 1 < nchunk) load(c + 1, a1, b1);
    mma(a0, b0);
    if (c + 1 < nchunk) {
      if (c + 2 < nchunk) load(c + 2, a0, b0);
      mma(a1, b1);
    }
  }
  for (int k = k8; k < K; ++k) {  // the last K % 8 steps: rank-1 updates
    float bk[TNW];
#pragma unroll
    for (int j = 0; j < TNW; ++j) bk[j] = Bs[k * BN + wn + 32 * j + lr];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float a = As[(wm + 8 * (r / 4) + 4 * h + (r % 4)) * K + k];
#pragma unroll
      for (int j = 0; j < TNW; ++j) acc[j][r] = fmaf(a, bk[j], acc[j][r]);
    }
  }

#pragma unroll
  for (int j = 0; j < TNW; ++j) {
    const int col = n0 + wn + 32 * j + lr;
    if (col >= N) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = m0 + wm + 8 * (r / 4) + 4 * h + (r % 4);
      if (row < M) C[row * N + col] = acc[j][r];
    }
  }
}

}  // namespace

bool shortm_shape_ok(int64_t M, int64_t N, int64_t K) {
  return M >= 1 && M <= kShortMMax && N >= 4 && N % 4 == 0 && N <= INT32_MAX / 2 && K >= 1 &&
         ceil_div(N, (int64_t)kSmBN) * ceil_div(K, (int64_t)kSmBK) <= (int64_t)UINT32_MAX;
}

int shortm_splits(int64_t M, int64_t N, int64_t K, size_t ws_bytes) {
  // The fewest k tiles per split (at least kSmMinChunk rows) whose grid fits
  // two workgroups per CU in one round: 65 x 384 x 16384 takes 4 tiles of 64
  // rows, 64 splits, 384 workgroups (3 tiles would need 516, a second round).
  const int64_t ntn = ceil_div(N, (int64_t)kSmBN);
  const int64_t tiles = ceil_div(K, (int64_t)kSmBK);
  const int64_t slots = 2 * (int64_t)device_cu_count();
  int64_t tp = std::max<int64_t>(kSmMinChunk / kSmBK, ceil_div(tiles * ntn, slots));
  while (tp < tiles && ntn * ceil_div(tiles, tp) > slots) ++tp;
  int64_t s = ceil_div(tiles, std::min(tp, tiles));
  const size_t per = (size_t)M * (size_t)N * sizeof(float);
  while (s > 1 && (size_t)s * per > ws_bytes) --s;
  return (int)std::max<int64_t>(s, 1);
}

size_t shortm_workspace_bytes(int64_t M, int64_t N, int64_t K, int splits, bool onehot) {
  const int64_t real = ceil_div(K, shortm_chunk(K, splits, onehot));
  if (real <= 1) return 0;
  return (size_t)real * (size_t)M * (size_t)N * sizeof(float);
}

int run_shortm(const float* A, const int64_t* ids, const float* B, float* C, int64_t M, int64_t N, int64_t K,
               int splits, void* workspace, size_t ws_bytes, hipStream_t st) {
  if (!shortm_shape_ok(M, N, K) || splits < 1 || !aligned16(B)) return AAR_EUNSUPPORTED;
  const bool onehot = ids != nullptr;
  const int64_t kc = shortm_chunk(K, splits, onehot);
  const int64_t real = ceil_div(K, kc);
  if (real > 1 && (!workspace || !aligned16(workspace) || ws_bytes < (size_t)real * M * N * sizeof(float)))
    return AAR_EWORKSPACE;
  float* out = real > 1 ? static_cast<float*>(workspace) : C;
  const int64_t stride = real > 1 ? M * N : 0;
  // 8 XCD lanes x column tiles x split groups of 8 (see the kernel)
  const dim3 grid((unsigned)(8 * ceil_div(N, (int64_t)kSmBN) * ceil_div(real, (int64_t)8)));
  const bool a16 = !onehot && aligned16(A);
  auto go = [&](auto mt_tag) {
    constexpr int MT = decltype(mt_tag)::value;
    if (!onehot && !(a16 ? ShortM<MT, false, true>::kOk : ShortM<MT, false, false>::kOk)) return (int)AAR_EUNSUPPORTED;
    if (onehot) {
      gemm_tn_shortm_kernel<MT, true, false><<<grid, dim3(kSmThreads), 0, st>>>(A, ids, B, out, (int)M, (int)N, K,
                                                                               kc, stride);
    } else if (a16) {
      gemm_tn_shortm_kernel<MT, false, true><<<grid, dim3(kSmThreads), 0, st>>>(A, ids, B, out, (int)M, (int)N, K,
                                                                               kc, stride);
    } else {
      gemm_tn_shortm_kernel<MT, false, false><<<grid, dim3(kSmThreads), 0, st>>>(A, ids, B, out, (int)M, (int)N,
                                                                                K, kc, stride);
    }
    return launch_status();
  };
  int rc;
  switch (shortm_blocks(M)) {
    case 2: rc = go(std::integral_constant<int, 2>{}); break;
    case 4: rc = go(std::integral_constant<int, 4>{}); break;
    case 6: rc = go(std::integral_constant<int, 6>{}); break;
    case 8: rc = go(std::integral_constant<int, 8>{}); break;
    default: return AAR_EUNSUPPORTED;
  }
  if (rc != AAR_OK || real <= 1) return rc;
  const int64_t n4 = M * N / 4;
  shortm_reduce_kernel<<<dim3((unsigned)ceil_div(4 * n4, (int64_t)256)), dim3(256), 0, st>>>(
      reinterpret_cast<const f32x4*>(out), reinterpret_cast<f32x4*>(C), n4, stride / 4, (int)real);
  return launch_status();
}

bool shortk_shape_ok(int64_t M, int64_t N, int64_t K) {
  return M >= 1 && K >= 1 && K <= kShortKMax && N >= 4 && N % 4 == 0 && N <= INT32_MAX / 2 &&
         M <= INT32_MAX / 2 && ceil_div(M, (int64_t)kSkBM) * ceil_div(N, (int64_t)128) <= (int64_t)UINT32_MAX;
}

int run_shortk(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K, hipStream_t st) {
  if (!shortk_shape_ok(M, N, K) || !aligned16(B)) return AAR_EUNSUPPORTED;
  // 192-column tiles where they divide N (the GPT head: 2 x 128 row tiles =
  // one workgroup per CU), else 128
  const bool wide = N % 192 == 0 && K <= 72;
  const int64_t bn = wide ? 192 : 128;
  const dim3 grid((unsigned)(8 * ceil_div(N, bn) * ceil_div(ceil_div(M, (int64_t)kSkBM), (int64_t)8)));
  // 16-byte DMAs of A's rows need every workgroup's first row 16-byte aligned
  const bool a16 = aligned16(A) && (kSkBM * K) % 4 == 0;
  auto go = [&](auto kern) {
    kern<<<grid, dim3(kSkThreads), 0, st>>>(A, B, C, (int)M, (int)N, (int)K);
    return launch_status();
  };
  if (wide) return a16 ? go(gemm_nn_shortk_kernel<72, 192, true>) : go(gemm_nn_shortk_kernel<72, 192, false>);
  if (K <= 72) return a16 ? go(gemm_nn_shortk_kernel<72, 128, true>) : go(gemm_nn_shortk_kernel<72, 128, false>);
  return a16 ? go(gemm_nn_shortk_kernel<128, 128, true>) : go(gemm_nn_shortk_kernel<128, 128, false>);
}

}  // namespace aar
