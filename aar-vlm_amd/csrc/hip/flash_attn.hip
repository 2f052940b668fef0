// fp32 flash attention on CDNA4 matrix cores (v_mfma_f32_32x32x2f32).
// Reference semantics: flash_attn_fwd_kernel / flash_attn_bwd_kernel
// (cppsrc/ops/flash_attention.cu:13-224): O = softmax(scale*Q K^T, causal
// mask j <= i) V, lse = m + ln(l); backward dQ, dK, dV.
//
// Layout trick: every product is issued "transposed" so that the dimension a
// wave owns (its 32 queries in forward / dQ, its 32 keys in dK/dV) is the MFMA
// output *column*, i.e. the lane index (lane % 32), while the reduced-over
// dimension sits in the 16 accumulator registers of that lane:
//   forward   S^T = K Q^T        lane = query, regs = 16 keys of the tile
//             O^T += V^T P^T     lane = query, regs = head-dim entries
// so the online-softmax row max / row sum are 16 in-register ops plus one
// exchange with lane ^ 32, and the rescale of O by alpha is lane-local.  The
// P tile produced by the first MFMA is consumed directly, register s of the
// S^T accumulator, as the B operand of the second MFMA: P never touches LDS.
//
// In a 32x32x2 MFMA, lane (r = lane%32, h = lane/32) supplies A[r][k], B[k][r]
// for k = h; accumulator register i of that lane is row 8*(i/4) + 4h + (i%4),
// column r.  Over a chunk of 8 contraction steps we let step s in 0..3 use
// k = 4h + s for the head-dim contractions (so one ds_read_b128 feeds 4
// MFMAs) and k = 8*(s/4) + 4h + (s%4) for the key/query contractions (so the
// accumulator register s is exactly the operand of step s).
//
// Backward (no float atomics, deterministic):
//   pass 0  D[i] = sum_d dO[i][d] O[i][d]
//   pass 1  workgroup per 128 keys (wave per 32 keys, K and V in registers),
//           loop over query tiles:  S = Q K^T, dP = dO V^T (lane = key),
//           P = exp(S*scale - lse), dS = P (dP - D),
//           dV^T += dO^T P,  dK^T += Q^T dS   (lane = key, accumulated in regs)
//   pass 2  workgroup per 128 queries (wave per 32 queries, Q and dO in regs),
//           loop over key tiles: S^T, dP^T (lane = query), dS^T,
//           dQ^T += K^T dS^T.
// With a large enough workspace (HBM is plentiful on MI355X: 3.2 GB for
// causal B8 H12 T4096), pass 1 also stores every dS tile it computes, in the
// order pass 2's MFMA operands consume it, and pass 2 becomes dQ^T += K^T
// dS^T over the stored tiles: 5 GEMM-equivalents per tile pair instead of 7.
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>
#include <initializer_list>
#include <stdint.h>

#include "common.hpp"

namespace aar {
namespace {

constexpr int kFaThreads = 256;  // 4 waves
constexpr int kTile = 32;        // keys (or queries) per inner tile
constexpr int kBlock = 128;      // queries (or keys) per workgroup
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ f32x16 mfma32(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// 2^x on the transcendental unit (v_exp_f32): inputs are scaled logits minus
// a running max, so results below 2^-126 (flushed to zero) carry no weight.
// The builtin exists only for the device target; the host pass never runs it.
__device__ __forceinline__ float fast_exp2(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_exp2f(x);
#else
  return x;
#endif
}

// Row index (within a 32-row tile) of accumulator register r for lane half h.
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// 4 consecutive floats p[0..3] of a row with `valid` leading entries (zeros
// past it).  VEC: the row is 16-byte aligned and valid is 0 or >= 4.
template <bool VEC>
__device__ __forceinline__ f32x4 load4(const float* __restrict__ p, int valid) {
  f32x4 v = {0.f, 0.f, 0.f, 0.f};
  if (VEC) {
    if (valid >= 4) v = *reinterpret_cast<const f32x4*>(p);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (e < valid) v[e] = p[e];
  }
  return v;
}

template <bool VEC>
__device__ __forceinline__ void store4(float* __restrict__ p, f32x4 v, int valid) {
  if (VEC) {
    if (valid >= 4) *reinterpret_cast<f32x4*>(p) = v;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (e < valid) p[e] = v[e];
  }
}

// Row swizzle of a transposed tile: column c's 32 rows are stored XOR
// 4 * ((c / 16) % 4).  The copy writes 16 consecutive columns of one row per
// 16 lanes; with a row stride of 36 floats they would share 4 LDS banks
// (4-way conflicts), the XOR spreads them over 16.  Groups of 4 consecutive
// rows stay together, so the 128-bit column reads are unchanged.  Measured on
// MI355X, the conflict-free layout is faster for d = 128 (-9 %) and without
// the causal mask (-2 %), but slower for causal d <= 64 (+5 % at T = 4096),
// so the forward kernel uses it only there.
template <bool SWZ>
__device__ __forceinline__ int vt_swz(int c, int r) { return SWZ ? r ^ (((c >> 4) & 3) << 2) : r; }
template <int DP, bool CAUSAL>
constexpr bool kVtSwizzle = DP == 128 || !CAUSAL;
// The dQ-from-dS pass stages K transposed the same way; there the swizzled
// layout is faster also for causal d = 64 (T = 4096: 6.47 -> 6.40 ms per
// fwd+bwd step; T = 1024: -0.6 %), with bit-identical dQ.
template <int DP, bool CAUSAL>
constexpr bool kKtSwizzle = true;

// Cooperative copy of a [32][DP] tile (rows row0.., head dim padded to DP with
// zeros, rows past T zero) from global into registers, then into LDS with row
// stride LD.
template <int DP, bool VEC>
struct TileCopy {
  static constexpr int kUnits = kTile * DP / 4;
  static constexpr int kPer = (kUnits + kFaThreads - 1) / kFaThreads;
  f32x4 reg[kPer];

  __device__ __forceinline__ void load(const float* __restrict__ base, int64_t st, int row0, int T, int d,
                                       int tid) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int u = tid + i * kFaThreads;
      const int r = u / (DP / 4);
      const int c = (u % (DP / 4)) * 4;
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (u < kUnits && row0 + r < T) v = load4<VEC>(base + (int64_t)(row0 + r) * st + c, d - c);
      reg[i] = v;
    }
  }

  template <int LD>
  __device__ __forceinline__ void store(float* __restrict__ s, int tid) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int u = tid + i * kFaThreads;
      if (u < kUnits) {
        const int r = u / (DP / 4);
        const int c = (u % (DP / 4)) * 4;
        *reinterpret_cast<f32x4*>(s + r * LD + c) = reg[i];
      }
    }
  }

  // Transposed: element (row r, column c) to s[c * LDT + vt_swz(c, r)], so
  // that 4 consecutive rows of one column are one 128-bit LDS read.
  template <int LDT, bool SWZ>
  __device__ __forceinline__ void store_t(float* __restrict__ s, int tid) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int u = tid + i * kFaThreads;
      if (u < kUnits) {
        const int r = u / (DP / 4);
        const int c = (u % (DP / 4)) * 4;
#pragma unroll
        for (int e = 0; e < 4; ++e) s[(c + e) * LDT + vt_swz<SWZ>(c + e, r)] = reg[i][e];
      }
    }
  }
};

// A [B, H, T, d] operand with element (b, h, t, c) at p[b*sb + h*sh + t*st + c]
// (the head dim is contiguous).  Contiguous [B*H, T, d] tensors, the q/k/v
// views of a packed [B, T, 3, H, d] projection and outputs in [B, T, H, d]
// are all of this form.
struct FaIn {
  const float* p;
  int64_t sb, sh, st;
  __device__ __forceinline__ const float* head(int bh, int H) const {
    return p + (int64_t)(bh / H) * sb + (int64_t)(bh % H) * sh;
  }
};
struct FaOut {
  float* p;
  int64_t sb, sh, st;
  __device__ __forceinline__ float* head(int bh, int H) const {
    return p + (int64_t)(bh / H) * sb + (int64_t)(bh % H) * sh;
  }
};

// Row stride of a transposed [DP][32] tile: 36 keeps the 128-bit reads of 32
// consecutive columns (one per lane) bank-conflict free.
constexpr int kLdt = kTile + 4;

// Stored dS: one 32x32 tile per (query tile, key tile) pair with work, 1024
// floats each, pairs of a head numbered row by row (the lower triangle only
// when causal).  Inside a tile dS[q][k] sits at k * 32 + q: the dK/dV pass
// (lane = key, accumulator registers 4g..4g+3 = four consecutive queries)
// writes 128-bit runs, and each 32-bit load of the dQ pass (lane = query)
// reads 128 contiguous bytes per half-wave.
constexpr int kDsTile = kTile * kTile;

__host__ __device__ __forceinline__ int64_t ds_pairs(int64_t nt, bool causal) {
  return causal ? nt * (nt + 1) / 2 : nt * nt;
}
__device__ __forceinline__ int64_t ds_pair(int qt, int kt, int nt, bool causal) {
  return causal ? (int64_t)qt * (qt + 1) / 2 + kt : (int64_t)qt * nt + kt;
}

// Causal forward split.  The query blocks of a head differ in work (block qb
// sees 4(qb+1) key tiles), and when the grid holds at most one workgroup per
// resident slot each CU ends on its longest block with the matrix cores
// mostly idle.  Then (fa_fwd_split_blocks says when) the longest S = nqb/2
// blocks have their key range cut in two halves, each half a workgroup of its
// own that writes its normalised partial O and log2-sum-exp to the workspace,
// and a combine pass merges the two halves of every split row.  item[] lists a head's work items longest
// first (qb << 2 | part; part 0 whole block, 1 first half, 2 second half);
// workgroup j*BH + bh runs item j of head bh.  Both halves of a split block
// see every key they hold (the first half ends before the block's first
// query, the second holds the diagonal), so every partial row has l > 0.
constexpr int kFaMaxItems = 96;
constexpr int64_t kFaSplitMaxGrid = 2048;  // largest grid (workgroups) that may split
struct FaSplit {
  int S;                           // blocks split in two; 0: no split, item[] unused
  uint16_t item[kFaMaxItems];      // per-head work items, longest first
  float* part_o;                   // [BH][S][2][kBlock][DP] normalised partial O
  float* part_l;                   // [BH][S][2][kBlock] m + log2(l) of each partial row
};

// Partial-row index of (head bh, split slot s, half p, row r of the block).
__host__ __device__ __forceinline__ int64_t fa_part_row(int bh, int S, int s, int p, int r) {
  return (((int64_t)bh * S + s) * 2 + p) * kBlock + r;
}

// ------------------------------------------------------------------ forward

// Software pipeline: K runs one tile ahead of V.  Iteration t holds K tile
// t+1 and V tile t in LDS and issues S_{t+1} = K_{t+1} Q^T on the matrix
// cores in the same basic block as the online softmax of S_t (VALU,
// independent), so the exp/max/sum work executes in the shadow of the MFMAs;
// then O += V_t P_t.  V is staged transposed so each 128-bit LDS read feeds
// four PV steps.  Only tiles that cross the causal diagonal or the sequence
// end are masked.  One barrier per tile.
template <int DP, bool CAUSAL, bool VEC, bool SPLIT>
__global__ void __launch_bounds__(kFaThreads)
flash_fwd_kernel(FaIn Qv, FaIn Kv, FaIn Vv, FaOut Ov, float* __restrict__ Lse, int T, int d, int H,
                 int nqb, int BH, float scale_log2, FaSplit sp) {
  constexpr int NC = DP / 8;   // head-dim chunks
  constexpr int NB = DP / 32;  // head-dim output blocks
  constexpr int LD = DP + 4;
  constexpr bool kSwz = kVtSwizzle<DP, CAUSAL>;
  __shared__ __attribute__((aligned(16))) float ks[2][kTile * LD];
  __shared__ __attribute__((aligned(16))) float vts[2][DP * kLdt];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, h = lane >> 5;
  // Longest work first: the last query blocks have the most key tiles.
  const int item = (int)(blockIdx.x / BH);
  const int qb = SPLIT ? sp.item[item] >> 2 : (CAUSAL ? nqb - 1 - item : item);
  const int part = SPLIT ? sp.item[item] & 3 : 0;
  const int bh = blockIdx.x % BH;
  const float* __restrict__ Q = Qv.head(bh, H);
  const float* __restrict__ K = Kv.head(bh, H);
  const float* __restrict__ V = Vv.head(bh, H);
  const int q0 = qb * kBlock + wave * kTile;  // first query of this wave
  const int qi = q0 + lr;                     // this lane's query

  f32x4 qr[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int dd = 8 * c + 4 * h;
    qr[c] = qi < T ? load4<VEC>(Q + (int64_t)qi * Qv.st + dd, d - dd) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  f32x16 o[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) o[b] = zero16();
  float m = -INFINITY, l = 0.f;

  const int kv_end = CAUSAL ? min(T, qb * kBlock + kBlock) : T;
  // Key tiles [tb, te) of this work item.
  const int nt_block = (kv_end + kTile - 1) / kTile;
  const int tb = SPLIT && part == 2 ? nt_block / 2 : 0;
  const int te = SPLIT && part == 1 ? nt_block / 2 : nt_block;
  const int ntiles = te - tb;
  // Last key tile that holds a key this wave's queries may see.
  const int wlast = CAUSAL ? min(te - 1, (q0 + kTile - 1) / kTile) : te - 1;

  // S^T tile from K rows in LDS: lane = query, register r = key acc_row(r, h).
  auto qk = [&](const float* kt) {
    f32x16 s = zero16();
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const f32x4 kf = *reinterpret_cast<const f32x4*>(kt + lr * LD + 8 * c + 4 * h);
#pragma unroll
      for (int e = 0; e < 4; ++e) s = mfma32(kf[e], qr[c][e], s);
    }
    return s;
  };
  // Online softmax of tile t (S in s) and O += V_t P_t.
  auto soft_pv = [&](f32x16 s, const float* vt, int kv0) {
    float mx = -INFINITY;
    if ((CAUSAL && kv0 + kTile - 1 > q0) || kv0 + kTile > T) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kv0 + acc_row(r, h);
        float v = s[r] * scale_log2;
        if (key >= T || (CAUSAL && key > qi)) v = -INFINITY;
        s[r] = v;
        mx = fmaxf(mx, v);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] *= scale_log2;
        mx = fmaxf(mx, s[r]);
      }
    }
    mx = half_swap_max(mx);
    const float m_new = fmaxf(m, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(m - m_use);
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = fast_exp2(s[r] - m_use);
      s[r] = p;
      ps += p;
    }
    ps = half_swap_sum(ps);
    l = l * alpha + ps;
    m = m_new;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int r = 0; r < 16; ++r) o[b][r] *= alpha;
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int vc = b * 32 + lr;
        const f32x4 vf = *reinterpret_cast<const f32x4*>(vt + vc * kLdt + vt_swz<kSwz>(vc, 8 * g + 4 * h));
#pragma unroll
        for (int e = 0; e < 4; ++e) o[b] = mfma32(vf[e], s[4 * g + e], o[b]);
      }
    }
  };

  // Iteration t works on key tile tb + t (buffers indexed by t).
  TileCopy<DP, VEC> kc, vc;
  kc.load(K, Kv.st, tb * kTile, T, d, tid);
  vc.load(V, Vv.st, tb * kTile, T, d, tid);
  kc.template store<LD>(ks[0], tid);
  vc.template store_t<kLdt, kSwz>(vts[0], tid);
  if (ntiles > 1) {
    kc.load(K, Kv.st, (tb + 1) * kTile, T, d, tid);
    kc.template store<LD>(ks[1], tid);
  }
  __syncthreads();
  f32x16 s_cur = qk(ks[0]);
  __syncthreads();  // K tile 0's buffer is refilled in iteration 0

  const int wl = wlast - tb;
  for (int t = 0; t < ntiles; ++t) {
    const bool load_k = t + 2 < ntiles;  // K_{t+2} -> ks[t & 1]
    const bool load_v = t + 1 < ntiles;  // V_{t+1} -> vts[(t + 1) & 1]
    if (load_k) kc.load(K, Kv.st, (tb + t + 2) * kTile, T, d, tid);
    if (load_v) vc.load(V, Vv.st, (tb + t + 1) * kTile, T, d, tid);
    f32x16 s_next = zero16();
    if (t + 1 <= wl) {
      s_next = qk(ks[(t + 1) & 1]);
      soft_pv(s_cur, vts[t & 1], (tb + t) * kTile);
    } else if (t <= wl) {
      soft_pv(s_cur, vts[t & 1], (tb + t) * kTile);
    }
    if (load_k) kc.template store<LD>(ks[t & 1], tid);
    if (load_v) vc.template store_t<kLdt, kSwz>(vts[(t + 1) & 1], tid);
    __syncthreads();
    s_cur = s_next;
  }

  if (SPLIT && part != 0) {
    // Half of a split block: normalised partial row and its m + log2(l).
    if (qi < T) {
      const float inv_l = 1.0f / l;
      const int64_t prow = fa_part_row(bh, sp.S, qb - (nqb - sp.S), part - 1, qi - qb * kBlock);
      float* po = sp.part_o + prow * DP;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int dd = b * 32 + 8 * g + 4 * h;
          *reinterpret_cast<f32x4*>(po + dd) = f32x4{o[b][4 * g] * inv_l, o[b][4 * g + 1] * inv_l,
                                                     o[b][4 * g + 2] * inv_l, o[b][4 * g + 3] * inv_l};
        }
      }
      if (h == 0) sp.part_l[prow] = m + log2f(l);
    }
    return;
  }
  if (qi < T) {
    const float inv_l = 1.0f / l;
    float* orow = Ov.head(bh, H) + (int64_t)qi * Ov.st;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dd = b * 32 + 8 * g + 4 * h;
        f32x4 v = {o[b][4 * g] * inv_l, o[b][4 * g + 1] * inv_l, o[b][4 * g + 2] * inv_l,
                   o[b][4 * g + 3] * inv_l};
        if (dd < d) store4<VEC>(orow + dd, v, d - dd);
      }
    }
    if (h == 0) Lse[(int64_t)bh * T + qi] = (m + log2f(l)) * kLn2;
  }
}

// ------------------------------------------------- DMA-staged 32 x 64 tiles
// The paired kernels stage their [32][64] operand tiles HBM -> LDS by DMA:
// no staging registers, no LDS stores.  A tile is [32][64] unpadded; float4
// group g of row r sits at group g ^ (r & 15) (16 groups per row), so the
// 128-bit row reads (32 rows, one group) and the 32-bit column reads (one
// row, 32 columns) are bank-conflict free.  Rows past T are clamped onto row
// T - 1: the caller masks them.  The DMAs are the untracked form: each
// kernel's loop orders them with its own wait and barrier at the end of an
// iteration, so the next iteration's DMA runs under the current MFMA work
// instead of before its first LDS read.  Requires d == 64 and 16-byte
// aligned rows.
struct FaDmaTile64 {
  static constexpr int kGroups = 16;
  static constexpr int kFloats = kTile * 64;
  static constexpr int kPerWave = kTile * kGroups / (kWave * 4);  // 2 DMA instructions per wave (4 waves)

  // One operand as a wave stages it: the head's row 0 and row stride, and
  // the byte offset of each of the wave's DMA lanes within a tile.  `wave`
  // must be wave-uniform to the compiler (readfirstlane), so tile bases and
  // LDS addresses stay scalar.
  struct Src {
    const float* base;
    int64_t st;
    uint32_t off[kPerWave];
    bool small;  // 31 rows of stride st fit the 32-bit lane offsets
  };
  __device__ __forceinline__ static int lane_row(int wave, int i, int lane) {
    return ((wave * kPerWave + i) * kWave + lane) / kGroups;
  }
  __device__ __forceinline__ static int lane_col(int wave, int i, int lane) {
    const int u = (wave * kPerWave + i) * kWave + lane;
    return ((u % kGroups) ^ ((u / kGroups) & 15)) * 4;
  }
  __device__ __forceinline__ static Src src(const float* __restrict__ base, int64_t st, int wave, int lane) {
    Src s{base, st, {}, st < (int64_t(1) << 25)};
#pragma unroll
    for (int i = 0; i < kPerWave; ++i)
      s.off[i] = (uint32_t)((lane_row(wave, i, lane) * st + lane_col(wave, i, lane)) * 4);
    return s;
  }
  // Stages rows row0 .. row0 + 31 of `s`.  A tile inside [0, T) takes the
  // scalar-base form; one that crosses T clamps its rows onto T - 1.
  __device__ __forceinline__ static void issue(const Src& s, int row0, int T, float* stage, int wave, int lane) {
    if (row0 + kTile <= T && s.small) {
      const float* tile = s.base + (int64_t)row0 * s.st;
#pragma unroll
      for (int i = 0; i < kPerWave; ++i)
        dma16_untracked_s(s.off[i], tile, (lds_void_t*)(stage + (wave * kPerWave + i) * kWave * 4));
    } else {
#pragma unroll
      for (int i = 0; i < kPerWave; ++i) {
        const int row = min(row0 + lane_row(wave, i, lane), T - 1);
        dma16_untracked(s.base + (int64_t)row * s.st + lane_col(wave, i, lane),
                        (lds_void_t*)(stage + (wave * kPerWave + i) * kWave * 4));
      }
    }
  }
  // float4 group `grp` of row `row`
  __device__ __forceinline__ static f32x4 group(const float* S, int row, int grp) {
    return *reinterpret_cast<const f32x4*>(S + (row * kGroups + (grp ^ (row & 15))) * 4);
  }
  // Column reads of the dV/dK products: lane (lr, h) reads row
  // q = 8*(st/4) + 4h + st%4, column 32b + lr.  The float offset splits into a
  // lane part that depends on st only through st % 4 (lane_off(k), four
  // values per lane) and a compile-time part (ct_off).
  __device__ __forceinline__ static int lane_off(int k, int lr, int h) {
    return 4 * h * 64 + ((((lr >> 2) ^ (4 * h)) ^ k) << 2) + (lr & 3);
  }
  __host__ __device__ static constexpr int ct_off(int st, int b) {
    return (8 * (st >> 2) + (st & 3)) * 64 + ((b ^ ((st >> 2) & 1)) << 5);
  }
};

// ------------------------------------------------------ forward, paired
// Causal forward over 64-query workgroups for short sequences, where the
// 128-query grid is about one round of resident workgroups and its longest
// items (the last query block, every key tile in turn) set the time: four
// waves as 2 query tiles x 2 key phases.  Each iteration stages key tiles t
// and t + 1 of K and V by DMA (FaDmaTile64).  STAGES = 2 double-buffers
// them (64 KB, two workgroups per CU: the next pair's DMA runs under this
// pair's MFMA work); STAGES = 1 stages a pair after the previous one is
// consumed (32 KB, three workgroups per CU that cover each other's DMA
// latency), which is faster for short workgroups (T = 256: -6 %) and slower
// for long ones (T = 4096: +9 %).  Wave (a, p)
// runs the online softmax of query tile a over key tile t + p, so the two
// phases of a query tile split its key range and the longest chain of tiles
// is half that of the 128-query kernel.  S^T takes 128-bit K row reads; O +=
// V^T P takes one 32-bit V column read per MFMA (the layout of the dK/dV
// pair kernel's dO^T P product).  At the end the two phases exchange
// (m, l) and half of O through LDS, and each merges the two partial
// softmaxes for its half of O's columns in a fixed order (m = max(m0, m1),
// w_p = 2^(m_p - m), l = w0 l0 + w1 l1, O = w0 O0 + w1 O1; deterministic),
// normalises and stores it; phase 0 stores lse.
// Requires d == DP == 64 and 16-byte aligned rows.
template <int DP, bool CAUSAL, int STAGES>
__global__ void __launch_bounds__(kFaThreads, STAGES == 1 ? 3 : 2)
flash_fwd_pair_kernel(FaIn Qv, FaIn Kv, FaIn Vv, FaOut Ov, float* __restrict__ Lse, int T, int H, int nqb,
                      int BH, float scale_log2) {
  static_assert(DP == 64, "the paired forward is built for head dim 64");
  constexpr int NC = DP / 8;   // head-dim chunks
  constexpr int NB = DP / 32;  // head-dim output blocks
  constexpr int kQueries = 2 * kTile;           // queries per workgroup
  constexpr int kHand = (NB * 16 + 4) * kWave;  // O blocks, then m and l of both phases, lane-major
  using Tile = FaDmaTile64;
  static_assert(STAGES == 1 || STAGES == 2, "one or two staged tile pairs");
  __shared__ __attribute__((aligned(16))) float ks[STAGES][2][Tile::kFloats];  // key tiles t, t + 1
  __shared__ __attribute__((aligned(16))) float vs[STAGES][2][Tile::kFloats];
  static_assert(kHand <= 2 * Tile::kFloats, "a query tile's hand-over fits in one stage's K (or V) tiles");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform to the compiler
  const int lr = lane & 31, h = lane >> 5;
  const int qt_local = wave & 1;  // query tile of this wave
  const int phase = wave >> 1;    // key tile t + phase of each staged pair
  const int qb = CAUSAL ? nqb - 1 - (int)(blockIdx.x / BH) : (int)(blockIdx.x / BH);  // longest first
  const int bh = blockIdx.x % BH;
  const float* __restrict__ Q = Qv.head(bh, H);
  const float* __restrict__ K = Kv.head(bh, H);
  const float* __restrict__ V = Vv.head(bh, H);
  const int q0 = qb * kQueries + qt_local * kTile;  // first query of this wave
  const int qi = q0 + lr;                           // this lane's query

  f32x4 qr[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int dd = 8 * c + 4 * h;
    qr[c] = qi < T ? *reinterpret_cast<const f32x4*>(Q + (int64_t)qi * Qv.st + dd) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  f32x16 o[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) o[b] = zero16();
  float m = -INFINITY, l = 0.f;

  const int kv_end = CAUSAL ? min(T, qb * kQueries + kQueries) : T;
  const int ntiles = (kv_end + kTile - 1) / kTile;
  // Last key tile that holds a key this wave's queries may see.
  const int wlast = CAUSAL ? min(ntiles - 1, (q0 + kTile - 1) / kTile) : ntiles - 1;
  // Lane offset of the V column reads for st % 4 == 0 (st % 4 == k: XOR k << 2).
  const int col_off = Tile::lane_off(0, lr, h);

  // S^T tile from a staged K tile: lane = query, register r = key acc_row(r, h).
  auto qk = [&](const float* kt) {
    f32x16 sc = zero16();
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const f32x4 kf = Tile::group(kt, lr, 2 * c + h);
#pragma unroll
      for (int e = 0; e < 4; ++e) sc = mfma32(kf[e], qr[c][e], sc);
    }
    return sc;
  };
  // Online softmax of one key tile (S in sc) and O += V_t^T P_t.
  auto soft_pv = [&](f32x16 sc, const float* vt, int kv0) {
    float mx = -INFINITY;
    if ((CAUSAL && kv0 + kTile - 1 > q0) || kv0 + kTile > T) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kv0 + acc_row(r, h);
        float v = sc[r] * scale_log2;
        if (key >= T || (CAUSAL && key > qi)) v = -INFINITY;
        sc[r] = v;
        mx = fmaxf(mx, v);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sc[r] *= scale_log2;
        mx = fmaxf(mx, sc[r]);
      }
    }
    mx = half_swap_max(mx);
    const float m_new = fmaxf(m, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(m - m_use);
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float pr = fast_exp2(sc[r] - m_use);
      sc[r] = pr;
      ps += pr;
    }
    ps = half_swap_sum(ps);
    l = l * alpha + ps;
    m = m_new;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int r = 0; r < 16; ++r) o[b][r] *= alpha;
    }
    // Lane (lr, h) of step st reads V row acc_row(st, h), column 32 b + lr.
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const int off = Tile::ct_off(st, b) + (col_off ^ ((st & 3) << 2));
        o[b] = mfma32(vt[off], sc[st], o[b]);
      }
    }
  };

  const Tile::Src ksrc = Tile::src(K, Kv.st, wave, lane), vsrc = Tile::src(V, Vv.st, wave, lane);
  auto issue_tiles = [&](int t, int buf) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      Tile::issue(ksrc, (t + p) * kTile, T, ks[buf][p], wave, lane);
      Tile::issue(vsrc, (t + p) * kTile, T, vs[buf][p], wave, lane);
    }
  };
  issue_tiles(0, 0);
  wait_vm_lgkm0<0>();
  ring_barrier();

  for (int t = 0; t < ntiles; t += 2) {
    const int cur = STAGES == 2 ? (t >> 1) & 1 : 0;
    if (STAGES == 2 && t + 2 < ntiles) issue_tiles(t + 2, cur ^ 1);
    if (t + phase <= wlast) soft_pv(qk(ks[cur][phase]), vs[cur][phase], (t + phase) * kTile);
    if (t + 2 >= ntiles) break;
    if (STAGES == 1) {
      // every read of this pair is done before the next pair lands in the
      // same buffers
      ring_barrier();
      issue_tiles(t + 2, 0);
    }
    // the next pair's DMAs have landed before any wave reads them (two
    // stages: and every read of this pair is done before the pair after
    // next is issued into its buffers)
    wait_vm_lgkm0<0>();
    ring_barrier();
  }
  __syncthreads();

  // The two phases of a query tile exchange (O, m, l) through LDS (every
  // wave is past the loop's last read of the staged tiles and no DMA is in
  // flight): query tile 0 through the K tiles, query tile 1 through V.  Each
  // phase merges and stores half of O's column blocks (phase p: blocks
  // b % 2 == p), so each writes the blocks the other stores, plus its m and
  // l.  Both compute the merge weights from the same values with the same
  // operations, so every stored element is w0*O0 + w1*O1 as one phase would
  // form it.
  static_assert(NB % 2 == 0, "the column blocks of O split evenly over the two phases");
  float* const hs = qt_local == 0 ? &ks[0][0][0] : &vs[0][0][0];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (b % 2 == phase) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) hs[(b * 16 + r) * kWave + lane] = o[b][r];
  }
  hs[(NB * 16 + 2 * phase) * kWave + lane] = m;
  hs[(NB * 16 + 2 * phase + 1) * kWave + lane] = l;
  __syncthreads();
  if (qi >= T) return;
  const float mo = hs[(NB * 16 + 2 * (1 - phase)) * kWave + lane];
  const float lo = hs[(NB * 16 + 2 * (1 - phase) + 1) * kWave + lane];
  const float m0 = phase == 0 ? m : mo, l0 = phase == 0 ? l : lo;
  const float m1 = phase == 0 ? mo : m, l1 = phase == 0 ? lo : l;
  const float mm = fmaxf(m0, m1);
  const float mu = mm == -INFINITY ? 0.f : mm;
  const float w0 = fast_exp2(m0 - mu), w1 = fast_exp2(m1 - mu);
  l = fmaf(w0, l0, w1 * l1);
  const float inv_l = 1.0f / l;
  float* orow = Ov.head(bh, H) + (int64_t)qi * Ov.st;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (b % 2 != phase) continue;
    float ob[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float x = o[b][r], y = hs[(b * 16 + r) * kWave + lane];
      const float o0 = phase == 0 ? x : y, o1 = phase == 0 ? y : x;
      ob[r] = fmaf(w0, o0, w1 * o1);  // w0 O0 + w1 O1, one form in both phases
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int dd = b * 32 + 8 * g + 4 * h;
      f32x4 v = {ob[4 * g] * inv_l, ob[4 * g + 1] * inv_l, ob[4 * g + 2] * inv_l, ob[4 * g + 3] * inv_l};
      *reinterpret_cast<f32x4*>(orow + dd) = v;
    }
  }
  if (phase == 0 && h == 0) Lse[(int64_t)bh * T + qi] = (mm + log2f(l)) * kLn2;
}

// Merge of the two halves of every split row: with L_p = m_p + log2(l_p) and
// M = max(L_0, L_1), w_p = 2^(L_p - M),
//   O = (w_0 O_0 + w_1 O_1) / (w_0 + w_1),   lse = (M + log2(w_0 + w_1)) ln 2,
// the softmax over the union of the two key ranges.  DP/4 lanes per row.
template <int DP, bool VEC>
__global__ void __launch_bounds__(256)
flash_fwd_combine_kernel(FaSplit sp, FaOut Ov, float* __restrict__ Lse, int T, int d, int H, int nqb,
                         int BH) {
  constexpr int kLanes = DP / 4;
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = u / kLanes;  // over BH x S x kBlock
  if (row >= (int64_t)BH * sp.S * kBlock) return;
  const int c = (int)(u % kLanes) * 4;
  const int r = (int)(row % kBlock);
  const int s = (int)((row / kBlock) % sp.S);
  const int bh = (int)(row / ((int64_t)kBlock * sp.S));
  const int qi = (nqb - sp.S + s) * kBlock + r;
  if (qi >= T) return;
  const int64_t p0 = fa_part_row(bh, sp.S, s, 0, r), p1 = fa_part_row(bh, sp.S, s, 1, r);
  const float l0 = sp.part_l[p0], l1 = sp.part_l[p1];
  const float mx = fmaxf(l0, l1);
  const float w0 = fast_exp2(l0 - mx), w1 = fast_exp2(l1 - mx);
  const float inv = 1.0f / (w0 + w1);
  const f32x4 a = *reinterpret_cast<const f32x4*>(sp.part_o + p0 * DP + c);
  const f32x4 b = *reinterpret_cast<const f32x4*>(sp.part_o + p1 * DP + c);
  const f32x4 v = {(w0 * a[0] + w1 * b[0]) * inv, (w0 * a[1] + w1 * b[1]) * inv, (w0 * a[2] + w1 * b[2]) * inv,
                   (w0 * a[3] + w1 * b[3]) * inv};
  if (c < d) store4<VEC>(Ov.head(bh, H) + (int64_t)qi * Ov.st + c, v, d - c);
  if (c == 0) Lse[(int64_t)bh * T + qi] = (mx + log2f(w0 + w1)) * kLn2;
}

// ------------------------------------------------------------- backward 0

// D[bh*T + t] = sum_c dO[bh][t][c] * O[bh][t][c]; 16 lanes per row, R
// consecutive rows of one head per 16-lane group (R divides T).  VEC
// (d % 4 == 0, 16-byte aligned rows): each lane takes float4 groups sub,
// sub + 16, ... with 128-bit loads, the first group of all R rows issued
// before any is used (2R loads in flight per lane); else element-wise.
template <bool VEC, int R>
__global__ void __launch_bounds__(256)
flash_bwd_dot_kernel(FaIn dOv, FaIn Ov, float* __restrict__ D, int64_t rows, int T, int H, int d) {
  const int64_t row0 = (((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4) * R;
  const int sub = threadIdx.x & 15;
  float acc[R];
#pragma unroll
  for (int i = 0; i < R; ++i) acc[i] = 0.f;
  if (row0 < rows) {
    const int bh = (int)(row0 / T), t0 = (int)(row0 - (int64_t)bh * T);
    const float* a = dOv.head(bh, H) + (int64_t)t0 * dOv.st;
    const float* b = Ov.head(bh, H) + (int64_t)t0 * Ov.st;
    if (VEC) {
      // lanes past the row's end (d < 64) load nothing
      const bool on = 4 * sub < d;
      f32x4 x[R], y[R];
#pragma unroll
      for (int i = 0; i < R; ++i) {
        x[i] = on ? *reinterpret_cast<const f32x4*>(a + i * dOv.st + 4 * sub) : f32x4{0.f, 0.f, 0.f, 0.f};
        y[i] = on ? *reinterpret_cast<const f32x4*>(b + i * Ov.st + 4 * sub) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int i = 0; i < R; ++i) acc[i] = x[i][0] * y[i][0] + x[i][1] * y[i][1] + x[i][2] * y[i][2] + x[i][3] * y[i][3];
      for (int c = 4 * sub + 64; c < d; c += 64) {
#pragma unroll
        for (int i = 0; i < R; ++i) {
          const f32x4 u = *reinterpret_cast<const f32x4*>(a + i * dOv.st + c);
          const f32x4 v = *reinterpret_cast<const f32x4*>(b + i * Ov.st + c);
          acc[i] += u[0] * v[0] + u[1] * v[1] + u[2] * v[2] + u[3] * v[3];
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < R; ++i)
        for (int c = sub; c < d; c += 16) acc[i] += a[i * dOv.st + c] * b[i * Ov.st + c];
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i) {
    float v = acc[i];
    v += dpp_quad_xor1(v);
    v += dpp_quad_xor2(v);
    v += dpp_half_mirror(v);
    v += dpp_row_mirror(v);
    if (row0 < rows && sub == 0) D[row0 + i] = v;
  }
}

// ------------------------------------------------------------- backward 1

template <int DP, bool CAUSAL, bool VEC, bool STORE_DS>
__global__ void __launch_bounds__(kFaThreads, DP <= 64 && (CAUSAL || !STORE_DS) ? 2 : 1)
flash_bwd_dkdv_kernel(FaIn Qv, FaIn Kv, FaIn Vv, FaIn dOv, const float* __restrict__ Lse,
                      const float* __restrict__ Dv, FaOut dKv, FaOut dVv, float* __restrict__ dS, int T, int d,
                      int H, int nkb, int BH, float scale, float scale_log2) {
  constexpr int NC = DP / 8;
  constexpr int NB = DP / 32;
  constexpr int LD = DP + 4;
  __shared__ __attribute__((aligned(16))) float qs[2][kTile * LD];
  __shared__ __attribute__((aligned(16))) float dos[2][kTile * LD];
  __shared__ __attribute__((aligned(16))) float ls[2][kTile];
  __shared__ __attribute__((aligned(16))) float dsum[2][kTile];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, h = lane >> 5;
  // Longest work first: under the causal mask the first key blocks see the
  // most query tiles.
  const int kb = (int)(blockIdx.x / BH);
  const int bh = blockIdx.x % BH;
  const float* __restrict__ Q = Qv.head(bh, H);
  const float* __restrict__ K = Kv.head(bh, H);
  const float* __restrict__ V = Vv.head(bh, H);
  const float* __restrict__ dO = dOv.head(bh, H);
  const int k0 = kb * kBlock + wave * kTile;  // first key of this wave
  const int kj = k0 + lr;                     // this lane's key
  const bool key_ok = kj < T;

  f32x4 kr[NC], vr[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int dd = 8 * c + 4 * h;
    const bool ok = kj < T;
    kr[c] = ok ? load4<VEC>(K + (int64_t)kj * Kv.st + dd, d - dd) : f32x4{0.f, 0.f, 0.f, 0.f};
    vr[c] = ok ? load4<VEC>(V + (int64_t)kj * Vv.st + dd, d - dd) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  f32x16 dk[NB], dv[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    dk[b] = zero16();
    dv[b] = zero16();
  }

  const int q_begin = CAUSAL ? kb * kBlock : 0;  // first query tile with work
  const int t0 = q_begin / kTile;
  const int ntiles = (T + kTile - 1) / kTile;
  // This lane's slot in a stored dS tile (key k = lr of the wave's key tile).
  float* dS_head = STORE_DS ? dS + (int64_t)bh * ds_pairs(ntiles, CAUSAL) * kDsTile : nullptr;
  // dS[acc_row(4g + e, h)][lr] = dS[8g + 4h + e][lr] sits at lr * 32 + 4h + 8g + e.
  const int ds_lane = lr * kTile + 4 * h;
  const int ktile = k0 / kTile;
  const float* Lb = Lse + (int64_t)bh * T;
  const float* Db = Dv + (int64_t)bh * T;

  TileCopy<DP, VEC> qc, dc;
  float lreg = 0.f, dreg = 0.f;
  auto load_tile = [&](int t) {
    qc.load(Q, Qv.st, t * kTile, T, d, tid);
    dc.load(dO, dOv.st, t * kTile, T, d, tid);
    if (tid < kTile) {
      const int q = t * kTile + tid;
      // Past-the-end queries get lse = +inf so that their P is exactly 0.
      lreg = q < T ? Lb[q] * kLog2e : INFINITY;
      dreg = q < T ? Db[q] : 0.f;
    }
  };
  auto store_tile = [&](int buf) {
    qc.template store<LD>(qs[buf], tid);
    dc.template store<LD>(dos[buf], tid);
    if (tid < kTile) {
      ls[buf][tid] = lreg;
      dsum[buf][tid] = dreg;
    }
  };
  if (t0 < ntiles) {
    load_tile(t0);
    store_tile(0);
  }
  __syncthreads();

  for (int t = t0; t < ntiles; ++t) {
    const int cur = (t - t0) & 1;
    const int qt0 = t * kTile;
    const bool has_next = t + 1 < ntiles;
    if (has_next) load_tile(t + 1);
    if (!CAUSAL || qt0 + kTile - 1 >= k0) {
      const float* qt = qs[cur];
      const float* dot = dos[cur];
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const f32x4 qf = *reinterpret_cast<const f32x4*>(qt + lr * LD + 8 * c + 4 * h);
        const f32x4 df = *reinterpret_cast<const f32x4*>(dot + lr * LD + 8 * c + 4 * h);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s = mfma32(qf[e], kr[c][e], s);
          dp = mfma32(df[e], vr[c][e], dp);
        }
      }
      // s, dp: lane = key kj, register r = query qt0 + acc_row(r, h).
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 l4 = *reinterpret_cast<const f32x4*>(&ls[cur][8 * g + 4 * h]);
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(&dsum[cur][8 * g + 4 * h]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g + e;
          float p = fast_exp2(s[r] * scale_log2 - l4[e]);
          // Keys past the end (zero-filled K) get P = 0, so a stored dS
          // tile is exactly zero there whatever the query's lse.
          if ((CAUSAL && kj > qt0 + acc_row(r, h)) || !key_ok) p = 0.f;
          s[r] = p;
          dp[r] = p * (dp[r] - d4[e]);
        }
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int st = 0; st < 16; ++st) {
          const int q = acc_row(st, h);
          dv[b] = mfma32(dot[q * LD + b * 32 + lr], s[st], dv[b]);
          dk[b] = mfma32(qt[q * LD + b * 32 + lr], dp[st], dk[b]);
        }
      }
      if (STORE_DS && k0 < T) {  // waves past the last key tile own no stored tile
        float* tile = dS_head + ds_pair(t, ktile, ntiles, CAUSAL) * kDsTile + ds_lane;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 v = {dp[4 * g], dp[4 * g + 1], dp[4 * g + 2], dp[4 * g + 3]};
          *reinterpret_cast<f32x4*>(tile + 8 * g) = v;
        }
      }
    }
    if (has_next) store_tile(cur ^ 1);
    __syncthreads();
  }

  if (kj < T) {
    float* krow = dKv.head(bh, H) + (int64_t)kj * dKv.st;
    float* vrow = dVv.head(bh, H) + (int64_t)kj * dVv.st;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dd = b * 32 + 8 * g + 4 * h;
        if (dd >= d) continue;
        f32x4 a = {dk[b][4 * g] * scale, dk[b][4 * g + 1] * scale, dk[b][4 * g + 2] * scale,
                   dk[b][4 * g + 3] * scale};
        f32x4 c = {dv[b][4 * g], dv[b][4 * g + 1], dv[b][4 * g + 2], dv[b][4 * g + 3]};
        store4<VEC>(krow + dd, a, d - dd);
        store4<VEC>(vrow + dd, c, d - dd);
      }
    }
  }
}

// ------------------------------------------------------ backward 1, paired
// The dK/dV pass over 64-key workgroups for grids of about one round: four
// waves as 2 key tiles x 2 query phases.  Per iteration the workgroup stages
// two query tiles (t and t + 1) of Q, dO, lse and D; wave (a, p) takes query
// tile t + p against key tile a, so the two phases of a key tile walk the
// query range in step and each works half of it.  Against 128-key
// workgroups this halves the longest work item and the idle diagonal steps
// (causal T = 256, 384 heads: 8 instead of 12 rounds of tile work on 512
// slots).  At the end the two phases of a key tile add their accumulators
// through LDS (phase 0 finishes dK, phase 1 dV; each a sum of two terms):
// deterministic, no atomics.  Stored dS tiles are written exactly as by
// flash_bwd_dkdv_kernel.
//
// Q and dO tiles go HBM -> LDS by DMA in the FaDmaTile64 layout (no staging
// registers: the 128-key kernel already uses all 256 VGPRs of a
// 2-wave-per-SIMD launch), double-buffered; the lse and D of the staged rows
// by 4-byte DMAs.  Rows past T are clamped onto row T - 1 (their P is 0
// through lse = +inf).  Requires d == DP == 64 and 16-byte aligned rows.

template <int DP, bool CAUSAL, bool STORE_DS>
__global__ void __launch_bounds__(kFaThreads, DP <= 64 && (CAUSAL || !STORE_DS) ? 2 : 1)
flash_bwd_dkdv_pair_kernel(FaIn Qv, FaIn Kv, FaIn Vv, FaIn dOv, const float* __restrict__ Lse,
                           const float* __restrict__ Dv, FaOut dKv, FaOut dVv, float* __restrict__ dS, int T,
                           int d, int H, int nkb, int BH, float scale, float scale_log2) {
  static_assert(DP == 64, "the paired kernel is built for head dim 64");
  constexpr int NC = DP / 8;
  constexpr int NB = DP / 32;
  constexpr int kKeys = 2 * kTile;  // keys per workgroup
  using Tile = FaDmaTile64;
  __shared__ __attribute__((aligned(16))) float qs[2][2][Tile::kFloats];
  __shared__ __attribute__((aligned(16))) float dos[2][2][Tile::kFloats];
  __shared__ __attribute__((aligned(16))) float ls[2][2 * kTile];    // raw lse of the 64 staged rows
  __shared__ __attribute__((aligned(16))) float dsum[2][2 * kTile];  // D of the 64 staged rows
  static_assert(2 * kTile == kWave, "one 4-byte DMA per staged statistic");
  static_assert(Tile::kFloats >= NB * 16 * kWave, "phase hand-over of one key tile fits in one staged tile");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform to the compiler
  const int lr = lane & 31, h = lane >> 5;
  const int kt_local = wave & 1;  // key tile of this wave
  const int phase = wave >> 1;    // query tile t + phase of each staged pair
  const int kb = (int)(blockIdx.x / BH);  // longest work first under the causal mask
  const int bh = blockIdx.x % BH;
  const float* __restrict__ Q = Qv.head(bh, H);
  const float* __restrict__ K = Kv.head(bh, H);
  const float* __restrict__ V = Vv.head(bh, H);
  const float* __restrict__ dO = dOv.head(bh, H);
  const int k0 = kb * kKeys + kt_local * kTile;  // first key of this wave
  const int kj = k0 + lr;
  const bool key_ok = kj < T;

  f32x4 kr[NC], vr[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int dd = 8 * c + 4 * h;
    kr[c] = key_ok ? *reinterpret_cast<const f32x4*>(K + (int64_t)kj * Kv.st + dd) : f32x4{0.f, 0.f, 0.f, 0.f};
    vr[c] = key_ok ? *reinterpret_cast<const f32x4*>(V + (int64_t)kj * Vv.st + dd) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  f32x16 dk[NB], dv[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    dk[b] = zero16();
    dv[b] = zero16();
  }

  const int t0 = CAUSAL ? kb * 2 : 0;  // first query tile with work (64 keys = 2 tiles)
  const int ntiles = (T + kTile - 1) / kTile;
  float* dS_head = STORE_DS ? dS + (int64_t)bh * ds_pairs(ntiles, CAUSAL) * kDsTile : nullptr;
  const int ds_lane = lr * kTile + 4 * h;
  const int ktile = k0 / kTile;
  const float* Lb = Lse + (int64_t)bh * T;
  const float* Db = Dv + (int64_t)bh * T;

  // Stages query tiles t, t + 1 into buffer `buf`, all by DMA: Q and dO tiles
  // (two instructions per wave each), and the raw lse and D of the 64 rows
  // (one 4-byte-per-lane instruction each, waves 0 and 1; rows past T read
  // row T - 1 and are masked where P is formed).  No staging registers.
  const Tile::Src qsrc = Tile::src(Q, Qv.st, wave, lane), dosrc = Tile::src(dO, dOv.st, wave, lane);
  auto issue_tiles = [&](int t, int buf) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      Tile::issue(qsrc, (t + p) * kTile, T, qs[buf][p], wave, lane);
      Tile::issue(dosrc, (t + p) * kTile, T, dos[buf][p], wave, lane);
    }
    // __lane_id() recomputes the lane index here (kept live, it would be
    // spilled, and its reload would wait for every DMA in flight)
    if (wave < 2) {
      const float* stat = wave == 0 ? Lb : Db;
      float* dst = wave == 0 ? ls[buf] : dsum[buf];
      if (t * kTile + kWave <= T) {
        dma4_untracked_s(__lane_id() * 4, stat + t * kTile, (lds_void_t*)dst);
      } else {
        dma4_untracked(stat + min(t * kTile + (int)__lane_id(), T - 1), (lds_void_t*)dst);
      }
    }
  };
  // Lane offset of the column reads for st % 4 == 0; the one for st % 4 == k
  // is col_off ^ (k << 2) (see FaDmaTile64::lane_off: the XOR only touches
  // bits 2-3 of its field).
  const int col_off = Tile::lane_off(0, lr, h);
  if (t0 < ntiles) issue_tiles(t0, 0);
  wait_vm_lgkm0<0>();
  ring_barrier();

  for (int t = t0; t < ntiles; t += 2) {
    const int cur = ((t - t0) >> 1) & 1;
    const int qt0 = (t + phase) * kTile;  // this wave's query tile
    const bool has_next = t + 2 < ntiles;
    if (has_next) issue_tiles(t + 2, cur ^ 1);
    const bool work = qt0 < T && (!CAUSAL || qt0 + kTile - 1 >= k0);
    if (work) {
      const float* qt = qs[cur][phase];
      const float* dot = dos[cur][phase];
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const f32x4 qf = Tile::group(qt, lr, 2 * c + h);
        const f32x4 df = Tile::group(dot, lr, 2 * c + h);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s = mfma32(qf[e], kr[c][e], s);
          dp = mfma32(df[e], vr[c][e], dp);
        }
      }
      // s, dp: lane = key kj, register r = query qt0 + acc_row(r, h).
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 l4 = *reinterpret_cast<const f32x4*>(&ls[cur][phase * kTile + 8 * g + 4 * h]);
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(&dsum[cur][phase * kTile + 8 * g + 4 * h]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g + e;
          const int q = qt0 + acc_row(r, h);
          float p = fast_exp2(s[r] * scale_log2 - l4[e] * kLog2e);
          // Keys past the end (zero-filled K) and queries past the end get
          // P = 0, so a stored dS tile is exactly zero there.
          if ((CAUSAL && kj > q) || !key_ok || q >= T) p = 0.f;
          s[r] = p;
          dp[r] = p * (dp[r] - d4[e]);
        }
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int st = 0; st < 16; ++st) {
          const int q = acc_row(st, h);
          const int o = Tile::ct_off(st, b) + (col_off ^ ((st & 3) << 2));
          dv[b] = mfma32(dot[o], s[st], dv[b]);
          dk[b] = mfma32(qt[o], dp[st], dk[b]);
        }
      }
      if (STORE_DS && k0 < T) {
        float* tile = dS_head + ds_pair(t + phase, ktile, ntiles, CAUSAL) * kDsTile + ds_lane;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 v = {dp[4 * g], dp[4 * g + 1], dp[4 * g + 2], dp[4 * g + 3]};
          *reinterpret_cast<f32x4*>(tile + 8 * g) = v;
        }
      }
    }
    // The next pair's DMAs were issued before this tile's four dS stores, and
    // vector memory operations retire in issue order: a wave that stored
    // waits for all but the last four (every DMA), without waiting for its
    // stores to reach memory.
    if (STORE_DS && work && k0 < T) {
      wait_vm_lgkm0<4>();
    } else {
      wait_vm_lgkm0<0>();
    }
    ring_barrier();
  }

  // The two phases of a key tile exchange halves of their accumulators
  // through the staging buffers (every wave is past the loop's last barrier,
  // no DMA is in flight), lane-major so the writes and reads are conflict
  // free: phase 1 hands its dK to phase 0 (qs[0][kt_local]), which adds and
  // stores dK; phase 0 hands its dV to phase 1 (dos[0][kt_local]), which
  // adds and stores dV.  Each sum has two terms, so it is the same in either
  // order.
  float* hk = qs[0][kt_local];
  float* hv = dos[0][kt_local];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if (phase == 1) {
        hk[(b * 16 + r) * kWave + lane] = dk[b][r];
      } else {
        hv[(b * 16 + r) * kWave + lane] = dv[b][r];
      }
    }
  }
  __syncthreads();
  if (!key_ok) return;
  if (phase == 0) {
    float* krow = dKv.head(bh, H) + (int64_t)kj * dKv.st;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int r = 0; r < 16; ++r) dk[b][r] += hk[(b * 16 + r) * kWave + lane];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dd = b * 32 + 8 * g + 4 * h;
        f32x4 a = {dk[b][4 * g] * scale, dk[b][4 * g + 1] * scale, dk[b][4 * g + 2] * scale,
                   dk[b][4 * g + 3] * scale};
        *reinterpret_cast<f32x4*>(krow + dd) = a;
      }
    }
  } else {
    float* vrow = dVv.head(bh, H) + (int64_t)kj * dVv.st;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int r = 0; r < 16; ++r) dv[b][r] = hv[(b * 16 + r) * kWave + lane] + dv[b][r];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dd = b * 32 + 8 * g + 4 * h;
        f32x4 c = {dv[b][4 * g], dv[b][4 * g + 1], dv[b][4 * g + 2], dv[b][4 * g + 3]};
        *reinterpret_cast<f32x4*>(vrow + dd) = c;
      }
    }
  }
}

// ------------------------------------------------------------- backward 2

template <int DP, bool CAUSAL, bool VEC>
__global__ void __launch_bounds__(kFaThreads)
flash_bwd_dq_kernel(FaIn Qv, FaIn Kv, FaIn Vv, FaIn dOv, const float* __restrict__ Lse,
                    const float* __restrict__ Dv, FaOut dQv, int T, int d, int H, int nqb, int BH,
                    float scale, float scale_log2) {
  constexpr int NC = DP / 8;
  constexpr int NB = DP / 32;
  constexpr int LD = DP + 4;
  __shared__ __attribute__((aligned(16))) float ks[2][kTile * LD];
  __shared__ __attribute__((aligned(16))) float vs[2][kTile * LD];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, h = lane >> 5;
  const int qb = CAUSAL ? nqb - 1 - (int)(blockIdx.x / BH) : (int)(blockIdx.x / BH);
  const int bh = blockIdx.x % BH;
  const float* __restrict__ Q = Qv.head(bh, H);
  const float* __restrict__ K = Kv.head(bh, H);
  const float* __restrict__ V = Vv.head(bh, H);
  const float* __restrict__ dO = dOv.head(bh, H);
  const int q0 = qb * kBlock + wave * kTile;
  const int qi = q0 + lr;

  f32x4 qr[NC], dor[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int dd = 8 * c + 4 * h;
    const bool ok = qi < T;
    qr[c] = ok ? load4<VEC>(Q + (int64_t)qi * Qv.st + dd, d - dd) : f32x4{0.f, 0.f, 0.f, 0.f};
    dor[c] = ok ? load4<VEC>(dO + (int64_t)qi * dOv.st + dd, d - dd) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float l2 = qi < T ? Lse[(int64_t)bh * T + qi] * kLog2e : INFINITY;
  const float dq_sum = qi < T ? Dv[(int64_t)bh * T + qi] : 0.f;
  f32x16 dq[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) dq[b] = zero16();

  const int kv_end = CAUSAL ? min(T, qb * kBlock + kBlock) : T;
  const int ntiles = (kv_end + kTile - 1) / kTile;

  TileCopy<DP, VEC> kc, vc;
  kc.load(K, Kv.st, 0, T, d, tid);
  vc.load(V, Vv.st, 0, T, d, tid);
  kc.template store<LD>(ks[0], tid);
  vc.template store<LD>(vs[0], tid);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int cur = t & 1;
    const int kv0 = t * kTile;
    const bool has_next = t + 1 < ntiles;
    if (has_next) {
      kc.load(K, Kv.st, kv0 + kTile, T, d, tid);
      vc.load(V, Vv.st, kv0 + kTile, T, d, tid);
    }
    if (!CAUSAL || kv0 <= q0 + kTile - 1) {
      const float* kt = ks[cur];
      const float* vt = vs[cur];
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const f32x4 kf = *reinterpret_cast<const f32x4*>(kt + lr * LD + 8 * c + 4 * h);
        const f32x4 vf = *reinterpret_cast<const f32x4*>(vt + lr * LD + 8 * c + 4 * h);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s = mfma32(kf[e], qr[c][e], s);
          dp = mfma32(vf[e], dor[c][e], dp);
        }
      }
      // s, dp: lane = query qi, register r = key kv0 + acc_row(r, h).
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kv0 + acc_row(r, h);
        float p = fast_exp2(s[r] * scale_log2 - l2);
        if (key >= T || (CAUSAL && key > qi)) p = 0.f;
        dp[r] = p * (dp[r] - dq_sum);
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int st = 0; st < 16; ++st) {
          dq[b] = mfma32(kt[acc_row(st, h) * LD + b * 32 + lr], dp[st], dq[b]);
        }
      }
    }
    if (has_next) {
      kc.template store<LD>(ks[cur ^ 1], tid);
      vc.template store<LD>(vs[cur ^ 1], tid);
    }
    __syncthreads();
  }

  if (qi < T) {
    float* qrow = dQv.head(bh, H) + (int64_t)qi * dQv.st;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dd = b * 32 + 8 * g + 4 * h;
        if (dd >= d) continue;
        f32x4 v = {dq[b][4 * g] * scale, dq[b][4 * g + 1] * scale, dq[b][4 * g + 2] * scale,
                   dq[b][4 * g + 3] * scale};
        store4<VEC>(qrow + dd, v, d - dd);
      }
    }
  }
}

// ------------------------------------------------ backward 2, stored dS

// dQ^T += K^T dS^T over the dS tiles pass 1 stored (lane = query): per key
// tile, K staged transposed in LDS (double-buffered; one 128-bit read feeds 4
// MFMA steps) and the wave's dS tile as sixteen coalesced 32-bit loads per
// lane, fetched one tile ahead.
template <int DP, bool CAUSAL, bool VEC>
__global__ void __launch_bounds__(kFaThreads)
flash_bwd_dq_ds_kernel(FaIn Kv, const float* __restrict__ dS, FaOut dQv, int T, int d, int H, int nqb, int BH,
                       float scale) {
  constexpr int NB = DP / 32;
  __shared__ __attribute__((aligned(16))) float kts[2][DP * kLdt];  // K tiles, transposed

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 31, h = lane >> 5;
  const int qb = CAUSAL ? nqb - 1 - (int)(blockIdx.x / BH) : (int)(blockIdx.x / BH);
  const int bh = blockIdx.x % BH;
  const float* __restrict__ K = Kv.head(bh, H);
  const int q0 = qb * kBlock + wave * kTile;
  const int qi = q0 + lr;
  const int qtile = q0 / kTile;
  const int nt = (T + kTile - 1) / kTile;
  const bool active = q0 < T;  // tiles past the end were never stored
  // step st reads dS[lr][acc_row(st, h)] at (8 * (st / 4) + 4h + st % 4) * 32 + lr
  const float* __restrict__ dS_head = dS + (int64_t)bh * ds_pairs(nt, CAUSAL) * kDsTile + 4 * h * kTile + lr;

  f32x16 dq[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) dq[b] = zero16();

  const int kv_end = CAUSAL ? min(T, qb * kBlock + kBlock) : T;
  const int ntiles = (kv_end + kTile - 1) / kTile;
  auto has_work = [&](int t) { return active && (!CAUSAL || t <= qtile); };
  auto load_ds = [&](int t, float (&r)[16]) {
    const float* tile = dS_head + ds_pair(qtile, t, nt, CAUSAL) * kDsTile;
#pragma unroll
    for (int st = 0; st < 16; ++st) r[st] = tile[(8 * (st >> 2) + (st & 3)) * kTile];
  };

  constexpr bool kSwz = kKtSwizzle<DP, CAUSAL>;
  TileCopy<DP, VEC> kc;
  kc.load(K, Kv.st, 0, T, d, tid);
  kc.template store_t<kLdt, kSwz>(kts[0], tid);
  float dsr[16];
  if (has_work(0)) load_ds(0, dsr);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int cur = t & 1;
    const bool has_next = t + 1 < ntiles;
    if (has_next) kc.load(K, Kv.st, (t + 1) * kTile, T, d, tid);
    float nxt[16];
    if (has_next && has_work(t + 1)) load_ds(t + 1, nxt);
    if (has_work(t)) {
      const float* kt = kts[cur];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          // K^T[b*32 + lr][keys 8g + 4h .. +3]: one 128-bit read feeds 4 steps
          const int kc_col = b * 32 + lr;
          const f32x4 kf = *reinterpret_cast<const f32x4*>(kt + kc_col * kLdt + vt_swz<kSwz>(kc_col, 8 * g + 4 * h));
#pragma unroll
          for (int e = 0; e < 4; ++e) dq[b] = mfma32(kf[e], dsr[4 * g + e], dq[b]);
        }
      }
    }
    if (has_next) {
      kc.template store_t<kLdt, kSwz>(kts[cur ^ 1], tid);
#pragma unroll
      for (int st = 0; st < 16; ++st) dsr[st] = nxt[st];
    }
    __syncthreads();
  }

  if (qi < T) {
    float* qrow = dQv.head(bh, H) + (int64_t)qi * dQv.st;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dd = b * 32 + 8 * g + 4 * h;
        if (dd >= d) continue;
        f32x4 v = {dq[b][4 * g] * scale, dq[b][4 * g + 1] * scale, dq[b][4 * g + 2] * scale,
                   dq[b][4 * g + 3] * scale};
        store4<VEC>(qrow + dd, v, d - dd);
      }
    }
  }
}

// dQ from the stored dS tiles over 64-query workgroups, for the grids that
// take the paired dK/dV kernel: four waves as 2 query tiles x 2 key phases.
// Per iteration the workgroup stages key tiles t and t + 1 by DMA
// (FaDmaTile64, double-buffered); wave (a, p) takes key tile t + p for query
// tile a, so the two phases of a query tile split its key range and the
// longest work item is half that of a 128-query workgroup.  dQ^T += K^T dS^T
// reads K columns with 32-bit conflict-free reads (the layout of the dK/dV
// pair kernel's dO^T P product); each wave's dS tile of the next pair is
// loaded into registers during the current one.  At the end the two phases
// of a query tile add their dQ accumulators through LDS, each phase
// finishing half of the column blocks (a sum of two terms; deterministic).  Requires d == DP == 64 and
// 16-byte aligned rows.
template <int DP, bool CAUSAL>
__global__ void __launch_bounds__(kFaThreads, 4)
flash_bwd_dq_ds_pair_kernel(FaIn Kv, const float* __restrict__ dS, FaOut dQv, int T, int H, int nqb, int BH,
                            float scale) {
  static_assert(DP == 64, "the paired dQ kernel is built for head dim 64");
  constexpr int NB = DP / 32;
  constexpr int kQueries = 2 * kTile;  // queries per workgroup
  using Tile = FaDmaTile64;
  __shared__ __attribute__((aligned(16))) float ks[2][2][Tile::kFloats];  // key tiles t, t+1 of a stage
  static_assert(2 * NB * 16 * kWave <= 4 * Tile::kFloats, "phase hand-over fits in the staging buffers");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform to the compiler
  const int lr = lane & 31, h = lane >> 5;
  const int qt_local = wave & 1;  // query tile of this wave
  const int phase = wave >> 1;    // key tile t + phase of each staged pair
  const int qb = CAUSAL ? nqb - 1 - (int)(blockIdx.x / BH) : (int)(blockIdx.x / BH);  // longest first
  const int bh = blockIdx.x % BH;
  const float* __restrict__ K = Kv.head(bh, H);
  const int q0 = qb * kQueries + qt_local * kTile;
  const int qi = q0 + lr;
  const int qtile = q0 / kTile;
  const int nt = (T + kTile - 1) / kTile;
  const bool active = q0 < T;  // tiles past the end were never stored
  const float* __restrict__ dS_head = dS + (int64_t)bh * ds_pairs(nt, CAUSAL) * kDsTile + 4 * h * kTile + lr;

  f32x16 dq[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) dq[b] = zero16();

  const int kv_end = CAUSAL ? min(T, qb * kQueries + kQueries) : T;
  const int ntiles = (kv_end + kTile - 1) / kTile;
  auto has_work = [&](int t) { return active && t < ntiles && (!CAUSAL || t <= qtile); };
  // Lane (lr, h) of step st needs dS^T[key acc_row(st, h)][query lr] of the
  // key-major stored tile.
  auto load_ds = [&](int t, float (&r)[16]) {
    const float* tile = dS_head + ds_pair(qtile, t, nt, CAUSAL) * kDsTile;
#pragma unroll
    for (int st = 0; st < 16; ++st) r[st] = tile[(8 * (st >> 2) + (st & 3)) * kTile];
  };
  const Tile::Src ksrc = Tile::src(K, Kv.st, wave, lane);
  auto issue_tiles = [&](int t, int buf) {
#pragma unroll
    for (int p = 0; p < 2; ++p) Tile::issue(ksrc, (t + p) * kTile, T, ks[buf][p], wave, lane);
  };
  // Lane offset of the K column reads for st % 4 == 0 (st % 4 == k: XOR k << 2).
  const int col_off = Tile::lane_off(0, lr, h);

  issue_tiles(0, 0);
  float dsr[16];
  if (has_work(phase)) load_ds(phase, dsr);
  wait_vm_lgkm0<0>();
  ring_barrier();

  for (int t = 0; t < ntiles; t += 2) {
    const int cur = (t >> 1) & 1;
    if (t + 2 < ntiles) issue_tiles(t + 2, cur ^ 1);
    const bool next_work = has_work(t + 2 + phase);
    float nxt[16];
    if (next_work) load_ds(t + 2 + phase, nxt);
    if (has_work(t + phase)) {
      const float* kt = ks[cur][phase];
      // Lane (lr, h) of step st reads K row acc_row(st, h), column 32 b + lr.
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int st = 0; st < 16; ++st) {
          const int off = Tile::ct_off(st, b) + (col_off ^ ((st & 3) << 2));
          dq[b] = mfma32(kt[off], dsr[st], dq[b]);
        }
      }
    }
    if (next_work) {
#pragma unroll
      for (int st = 0; st < 16; ++st) dsr[st] = nxt[st];
    }
    // This wave's DMAs and dS loads for the next pair have landed, and
    // (after the barrier) every wave's have and every read of this pair is
    // done.
    wait_vm_lgkm0<0>();
    ring_barrier();
  }

  // The two phases of a query tile exchange halves of their dQ accumulators
  // through the staging buffers (every wave is past the loop's last barrier
  // and no DMA is in flight), lane-major so the writes and reads are
  // conflict free: phase p adds and stores the column blocks b % 2 == p and
  // hands the others over.  Each sum has two terms, so it is the same in
  // either order.
  static_assert(NB % 2 == 0, "the column blocks of dQ split evenly over the two phases");
  float* hq = &ks[0][0][0] + qt_local * (NB * 16 * kWave);
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (b % 2 == phase) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) hq[(b * 16 + r) * kWave + lane] = dq[b][r];
  }
  __syncthreads();
  if (qi >= T) return;
  float* qrow = dQv.head(bh, H) + (int64_t)qi * dQv.st;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (b % 2 != phase) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[b][r] += hq[(b * 16 + r) * kWave + lane];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int dd = b * 32 + 8 * g + 4 * h;
      f32x4 v = {dq[b][4 * g] * scale, dq[b][4 * g + 1] * scale, dq[b][4 * g + 2] * scale,
                 dq[b][4 * g + 3] * scale};
      *reinterpret_cast<f32x4*>(qrow + dd) = v;
    }
  }
}

// ------------------------------------------------------------ dispatching

int pad_dim(int64_t d) { return d <= 32 ? 32 : (d <= 64 ? 64 : 128); }

template <template <int, bool, bool> class Launcher, typename... Args>
int dispatch_fa(int dp, bool causal, bool vec, Args... args) {
#define AAR_FA_CASE(DPV)                                                      \
  if (dp == DPV) {                                                            \
    if (causal) {                                                             \
      return vec ? Launcher<DPV, true, true>::run(args...)                    \
                 : Launcher<DPV, true, false>::run(args...);                  \
    }                                                                         \
    return vec ? Launcher<DPV, false, true>::run(args...)                     \
               : Launcher<DPV, false, false>::run(args...);                   \
  }
  AAR_FA_CASE(32)
  AAR_FA_CASE(64)
  AAR_FA_CASE(128)
#undef AAR_FA_CASE
  return AAR_EUNSUPPORTED;
}

struct FwdArgs {
  FaIn q, k, v;
  FaOut o;
  float* lse;
  int T, d, H, BH;
  float scale;
  void* ws;  // split partials when non-null and large enough
  size_t ws_bytes;
  int query_block;  // queries per workgroup: 64 (paired kernel) or 128
  hipStream_t st;
};

// Blocks the causal forward splits: nqb/2 (the longest) when the grid fills at
// most half of the resident workgroup slots (`slots` = CUs x workgroups per
// CU), or one full round with at least 8 query blocks.  Measured on MI355X,
// d = 64, forward + combine against the unsplit forward: grids of 32-384
// workgroups 0.53-0.87x the time, 768 workgroups 0.94x at T = 1024 and 0.86x
// at T = 4096 but 1.06x at T = 512 (4 blocks of 4-16 key tiles, where the
// combine pass costs more than the balance gains).  With more than one round
// the dispatcher already balances the blocks.
int fa_fwd_split_blocks(int64_t bh, int64_t nqb, int64_t slots) {
  const int64_t grid = bh * nqb;
  if (nqb < 2 || nqb + nqb / 2 > kFaMaxItems || grid > std::min(slots, kFaSplitMaxGrid)) return 0;
  if (2 * grid > slots && nqb < 8) return 0;
  return (int)(nqb / 2);
}

// Workspace of a split with S = nqb/2: partial rows (256-byte aligned), then
// their log2-sum-exps.  Depends on the shape only, so it can be sized without
// a device; grids above kFaSplitMaxGrid workgroups (more than any MI355X
// holds at once) never split and need none.
size_t fa_fwd_part_o_bytes(int64_t bh, int64_t T, int64_t d) {
  const int64_t nqb = (T + kBlock - 1) / kBlock;
  if (nqb < 2 || nqb + nqb / 2 > kFaMaxItems || bh * nqb > kFaSplitMaxGrid) return 0;
  const int64_t rows = bh * (nqb / 2) * 2 * kBlock;
  return ((size_t)rows * pad_dim(d) * sizeof(float) + 255) / 256 * 256;
}
size_t fa_fwd_split_bytes(int64_t bh, int64_t T, int64_t d) {
  const size_t ob = fa_fwd_part_o_bytes(bh, T, d);
  if (ob == 0) return 0;
  const int64_t nqb = (T + kBlock - 1) / kBlock;
  return ob + (size_t)(bh * (nqb / 2) * 2 * kBlock) * sizeof(float);
}

// Work items of one head, longest first (see FaSplit).
void fa_fwd_items(FaSplit& sp, int T, int nqb) {
  int len[kFaMaxItems], n = 0;
  for (int qb = nqb - 1; qb >= 0; --qb) {
    const int nt = (std::min(T, qb * kBlock + kBlock) + kTile - 1) / kTile;
    if (qb >= nqb - sp.S) {
      sp.item[n] = (uint16_t)(qb << 2 | 1), len[n++] = nt / 2;
      sp.item[n] = (uint16_t)(qb << 2 | 2), len[n++] = nt - nt / 2;
    } else {
      sp.item[n] = (uint16_t)(qb << 2), len[n++] = nt;
    }
  }
  for (int i = 1; i < n; ++i)  // stable insertion sort, descending length
    for (int j = i; j > 0 && len[j] > len[j - 1]; --j) {
      std::swap(len[j], len[j - 1]);
      std::swap(sp.item[j], sp.item[j - 1]);
    }
}

// Workgroups of the causal forward resident on one CU (register-limited).
template <int DP, bool VEC>
int fa_fwd_resident() {
  static const int n = [] {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, flash_fwd_kernel<DP, true, VEC, true>, kFaThreads, 0) !=
        hipSuccess) {
      b = 1;
    }
    return b > 0 ? b : 1;
  }();
  return n;
}

// Queries per forward workgroup.  The paired 64-query kernel (two key phases
// per query tile, K and V staged by DMA) halves the longest chain of key
// tiles of the 128-query kernel and has no staging registers; the 128-query
// kernel shares each staged key tile among four query tiles.  Measured on
// MI355X (causal, d = 64; R = 128-query grid / resident 128-query
// workgroups), the paired kernel takes 0.81-0.86x the time at R <= 1
// (T = 256..4096), 0.91-0.93x at R = 2 and 0.98x at R = 4 for T <= 1024, but
// 1.01x at R = 4, T = 4096 and at R = 8, T = 256.  So: paired up to two
// rounds, and up to four for T <= 1024.  It is built for causal d = 64
// exactly, with 128-bit operands; other shapes take 128.  `forced` (64 or
// 128, from a caller's per-call plan; 0 = none) overrides the choice for
// the shapes that can take either.
int fa_fwd_query_block(int64_t bh, int64_t T, int64_t d, bool causal, bool vec, int forced = 0) {
  if (!causal || d != 64 || !vec) return kBlock;
  if (forced) return forced;
  const int64_t slots = (int64_t)device_cu_count() * fa_fwd_resident<64, true>();
  const int64_t grid = bh * ((T + kBlock - 1) / kBlock);
  return (grid <= 2 * slots || (T <= 1024 && grid <= 4 * slots)) ? 64 : kBlock;
}

template <int DP, bool C, bool VEC>
struct FwdLaunch {
  static int run(const FwdArgs& a) {
    if constexpr (C && VEC && DP == 64) {
      const int64_t nqb64 = (a.T + 2 * kTile - 1) / (2 * kTile);
      // (a dispatch holds the grid as a 32-bit work-item count)
      if (a.query_block == 64 && nqb64 * a.BH * kFaThreads <= (int64_t)UINT32_MAX) {
        if (a.T <= 1024) {
          flash_fwd_pair_kernel<DP, C, 1><<<dim3((unsigned)(nqb64 * a.BH)), dim3(kFaThreads), 0, a.st>>>(
              a.q, a.k, a.v, a.o, a.lse, a.T, a.H, (int)nqb64, a.BH, a.scale * kLog2e);
        } else {
          flash_fwd_pair_kernel<DP, C, 2><<<dim3((unsigned)(nqb64 * a.BH)), dim3(kFaThreads), 0, a.st>>>(
              a.q, a.k, a.v, a.o, a.lse, a.T, a.H, (int)nqb64, a.BH, a.scale * kLog2e);
        }
        return launch_status();
      }
    }
    const int nqb = (a.T + kBlock - 1) / kBlock;
    FaSplit sp{};
    if (C && a.ws && aligned16(a.ws) && a.ws_bytes >= fa_fwd_split_bytes(a.BH, a.T, a.d)) {
      sp.S = fa_fwd_split_blocks(a.BH, nqb, (int64_t)device_cu_count() * fa_fwd_resident<DP, VEC>());
    }
    if (sp.S > 0) {
      fa_fwd_items(sp, a.T, nqb);
      sp.part_o = static_cast<float*>(a.ws);
      sp.part_l = reinterpret_cast<float*>(static_cast<char*>(a.ws) + fa_fwd_part_o_bytes(a.BH, a.T, a.d));
    }
    // The unsplit instance keeps the key loop free of the split's tile offsets
    // (with them the T = 4096 causal forward ran 4 % slower).
    if (sp.S > 0) {
      flash_fwd_kernel<DP, C, VEC, true><<<dim3((unsigned)((nqb + sp.S) * a.BH)), dim3(kFaThreads), 0, a.st>>>(
          a.q, a.k, a.v, a.o, a.lse, a.T, a.d, a.H, nqb, a.BH, a.scale * kLog2e, sp);
    } else {
      flash_fwd_kernel<DP, C, VEC, false><<<dim3((unsigned)(nqb * a.BH)), dim3(kFaThreads), 0, a.st>>>(
          a.q, a.k, a.v, a.o, a.lse, a.T, a.d, a.H, nqb, a.BH, a.scale * kLog2e, sp);
    }
    int rc = launch_status();
    if (rc != AAR_OK || sp.S == 0) return rc;
    const int64_t lanes = (int64_t)a.BH * sp.S * kBlock * (DP / 4);
    flash_fwd_combine_kernel<DP, VEC><<<dim3((unsigned)ceil_div(lanes, (int64_t)256)), dim3(256), 0, a.st>>>(
        sp, a.o, a.lse, a.T, a.d, a.H, nqb, a.BH);
    return launch_status();
  }
};

struct BwdArgs {
  FaIn q, k, v, dout;
  const float *lse, *D;
  FaOut dq, dk, dv;
  float* dS;  // stored-dS path when non-null
  int T, d, H, BH;
  float scale;
  int key_block;  // keys per dK/dV workgroup: 64 (paired kernel) or 128
  hipStream_t st;
};

// Workgroups of a dK/dV kernel resident on one CU at once.
template <int DP, bool C, bool VEC, bool PAIR>
int fa_dkdv_resident() {
  static const int n = [] {
    int b = 0;
    hipError_t e;
    if constexpr (PAIR) {
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, flash_bwd_dkdv_pair_kernel<DP, C, true>, kFaThreads, 0);
    } else {
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, flash_bwd_dkdv_kernel<DP, C, VEC, true>, kFaThreads,
                                                       0);
    }
    if (e != hipSuccess) b = 1;
    return b > 0 ? b : 1;
  }();
  return n;
}

// Keys per dK/dV workgroup.  128-key workgroups hold four key tiles that
// share each staged query tile; when their grid is at most two rounds of
// resident workgroups (short sequences, few heads) its longest items set the
// time, and the paired 64-key kernel (half the longest item) is used instead.
// The paired kernel stages its tiles by DMA in a layout built for d = 64
// exactly, with 128-bit operands; other shapes take 128-key workgroups.
// `forced` (64 or 128, from a caller's per-call plan; 0 = none) overrides
// the choice for the shapes that can take either.
int fa_bwd_key_block(int64_t bh, int64_t T, int64_t d, bool causal, bool vec, int forced = 0) {
  if (d != 64 || !vec) return 128;
  if (forced) return forced;
  const int resident =
      causal ? fa_dkdv_resident<64, true, true, false>() : fa_dkdv_resident<64, false, true, false>();
  const int64_t slots = (int64_t)device_cu_count() * resident;
  const int64_t grid = bh * ((T + kBlock - 1) / kBlock);
  return grid <= 2 * slots ? 64 : 128;
}

template <int DP, bool C, bool VEC>
struct BwdLaunch {
  static int run(const BwdArgs& a) {
    if constexpr (DP == 64 && VEC) {
      const int64_t nb2 = (a.T + 2 * kTile - 1) / (2 * kTile);
      // (a dispatch holds the grid as a 32-bit work-item count)
      if (a.key_block == 64 && a.d == DP && nb2 * a.BH * kFaThreads <= (int64_t)UINT32_MAX) {
        if (a.dS) {
          flash_bwd_dkdv_pair_kernel<DP, C, true><<<dim3((unsigned)(nb2 * a.BH)), dim3(kFaThreads), 0, a.st>>>(
              a.q, a.k, a.v, a.dout, a.lse, a.D, a.dk, a.dv, a.dS, a.T, a.d, a.H, (int)nb2, a.BH, a.scale,
              a.scale * kLog2e);
        } else {
          flash_bwd_dkdv_pair_kernel<DP, C, false><<<dim3((unsigned)(nb2 * a.BH)), dim3(kFaThreads), 0, a.st>>>(
              a.q, a.k, a.v, a.dout, a.lse, a.D, a.dk, a.dv, nullptr, a.T, a.d, a.H, (int)nb2, a.BH, a.scale,
              a.scale * kLog2e);
        }
        const int rc = launch_status();
        if (rc != AAR_OK) return rc;
        return run_dq(a);
      }
    }
    const int nb = (a.T + kBlock - 1) / kBlock;
    if (a.dS) {
      flash_bwd_dkdv_kernel<DP, C, VEC, true><<<dim3((unsigned)(nb * a.BH)), dim3(kFaThreads), 0, a.st>>>(
          a.q, a.k, a.v, a.dout, a.lse, a.D, a.dk, a.dv, a.dS, a.T, a.d, a.H, nb, a.BH, a.scale,
          a.scale * kLog2e);
    } else {
      flash_bwd_dkdv_kernel<DP, C, VEC, false><<<dim3((unsigned)(nb * a.BH)), dim3(kFaThreads), 0, a.st>>>(
          a.q, a.k, a.v, a.dout, a.lse, a.D, a.dk, a.dv, nullptr, a.T, a.d, a.H, nb, a.BH, a.scale,
          a.scale * kLog2e);
    }
    const int rc = launch_status();
    if (rc != AAR_OK) return rc;
    return run_dq(a);
  }

  // The dQ pass (128-query workgroups), from the stored dS tiles or by
  // recomputing P and dP.
  static int run_dq(const BwdArgs& a) {
    const int nb = (a.T + kBlock - 1) / kBlock;
    if constexpr (DP == 64 && VEC) {
      const int64_t nb2 = (a.T + 2 * kTile - 1) / (2 * kTile);
      if (a.dS && a.key_block == 64 && a.d == DP && nb2 * a.BH * kFaThreads <= (int64_t)UINT32_MAX) {
        flash_bwd_dq_ds_pair_kernel<DP, C><<<dim3((unsigned)(nb2 * a.BH)), dim3(kFaThreads), 0, a.st>>>(
            a.k, a.dS, a.dq, a.T, a.H, (int)nb2, a.BH, a.scale);
        return launch_status();
      }
    }
    if (a.dS) {
      flash_bwd_dq_ds_kernel<DP, C, VEC><<<dim3((unsigned)(nb * a.BH)), dim3(kFaThreads), 0, a.st>>>(
          a.k, a.dS, a.dq, a.T, a.d, a.H, nb, a.BH, a.scale);
    } else {
      flash_bwd_dq_kernel<DP, C, VEC><<<dim3((unsigned)(nb * a.BH)), dim3(kFaThreads), 0, a.st>>>(
          a.q, a.k, a.v, a.dout, a.lse, a.D, a.dq, a.T, a.d, a.H, nb, a.BH, a.scale, a.scale * kLog2e);
    }
    return launch_status();
  }
};

// 128-bit accesses need 16-byte aligned head rows: aligned bases, d and all
// strides multiples of 4.
bool fa_vec_ok(int64_t d, std::initializer_list<const void*> ptrs, const int64_t* strides, int nstrides) {
  if (d % 4 != 0) return false;
  for (const void* p : ptrs)
    if (!aligned16(p)) return false;
  for (int i = 0; i < nstrides; ++i)
    if (strides[i] % 4 != 0) return false;
  return true;
}

FaIn fa_in(const float* p, const int64_t* s) { return FaIn{p, s[0], s[1], s[2]}; }
FaOut fa_out(float* p, const int64_t* s) { return FaOut{p, s[0], s[1], s[2]}; }

bool fa_shape_ok(int64_t bh, int64_t T, int64_t d) {
  return bh > 0 && T > 0 && d > 0 && d <= 128 && T <= (1 << 24) && bh <= (1 << 24) &&
         bh * ((T + kBlock - 1) / kBlock) * kFaThreads <= (int64_t)UINT32_MAX;  // 32-bit grid work-items
}

}  // namespace
}  // namespace aar

using namespace aar;

extern "C" size_t aar_flash_fwd_workspace_bytes(int64_t bh, int64_t T, int64_t d, int causal) {
  if (!causal || bh <= 0 || T <= 0 || d <= 0 || d > 128 || bh > (1 << 24) || T > (1 << 24)) return 0;
  return fa_fwd_split_bytes(bh, T, d);
}

extern "C" int aar_flash_fwd_strided_plan_f32(const float* q, const float* k, const float* v, float* o,
                                              float* lse, int64_t B, int64_t H, int64_t T, int64_t d,
                                              const int64_t* strides, int causal, float scale, int query_block,
                                              void* workspace, size_t workspace_bytes, void* stream) {
  if (query_block != 0 && query_block != 64 && query_block != 128) return AAR_EINVAL;
  if (B < 0 || H < 0 || T < 0 || d <= 0) return AAR_EINVAL;
  if (d > 128) return AAR_EINVAL;
  if (B == 0 || H == 0 || T == 0) return AAR_OK;
  if (!q || !k || !v || !o || !lse || !strides) return AAR_EINVAL;
  if (!fa_shape_ok(B * H, T, d) || H > INT32_MAX) return AAR_EUNSUPPORTED;
  const bool vec = fa_vec_ok(d, {q, k, v, o}, strides, 12);
  FwdArgs a{fa_in(q, strides),      fa_in(k, strides + 3), fa_in(v, strides + 6), fa_out(o, strides + 9),
            lse,                    (int)T,                (int)d,                (int)H,
            (int)(B * H),           scale,                 workspace,             workspace_bytes,
            fa_fwd_query_block(B * H, T, d, causal != 0, vec, query_block), as_stream(stream)};
  return dispatch_fa<FwdLaunch>(pad_dim(d), causal != 0, vec, a);
}

extern "C" int aar_flash_fwd_strided_f32(const float* q, const float* k, const float* v, float* o, float* lse,
                                         int64_t B, int64_t H, int64_t T, int64_t d, const int64_t* strides,
                                         int causal, float scale, void* workspace, size_t workspace_bytes,
                                         void* stream) {
  return aar_flash_fwd_strided_plan_f32(q, k, v, o, lse, B, H, T, d, strides, causal, scale, 0, workspace,
                                        workspace_bytes, stream);
}

extern "C" int aar_flash_fwd_f32(const float* q, const float* k, const float* v, float* o, float* lse,
                                 int64_t bh, int64_t T, int64_t d, int causal, float scale,
                                 void* stream) {
  if (bh < 0 || T < 0 || d <= 0) return AAR_EINVAL;
  const int64_t c[3] = {bh * T * d, T * d, d};  // [1, bh, T, d] contiguous
  const int64_t strides[12] = {c[0], c[1], c[2], c[0], c[1], c[2], c[0], c[1], c[2], c[0], c[1], c[2]};
  return aar_flash_fwd_strided_f32(q, k, v, o, lse, 1, bh, T, d, strides, causal, scale, nullptr, 0, stream);
}

extern "C" size_t aar_flash_bwd_workspace_bytes(int64_t bh, int64_t T, int64_t d) {
  (void)d;
  if (bh <= 0 || T <= 0) return 0;
  return (size_t)bh * (size_t)T * sizeof(float);
}

// D rows, padded to 256 bytes, then the dS tiles.
static size_t fa_d_bytes(int64_t bh, int64_t T) {
  return ((size_t)bh * (size_t)T * sizeof(float) + 255) / 256 * 256;
}

extern "C" size_t aar_flash_bwd_fast_workspace_bytes(int64_t bh, int64_t T, int64_t d, int causal) {
  (void)d;
  if (bh <= 0 || T <= 0) return 0;
  const int64_t nt = (T + kTile - 1) / kTile;
  // Sizes past 2^62 bytes cannot be allocated: saturate instead of wrapping.
  const double bytes = (double)bh * (double)ds_pairs(nt, causal != 0) * kDsTile * sizeof(float);
  if (bytes > 4.0e18) return SIZE_MAX;
  return fa_d_bytes(bh, T) + (size_t)bh * (size_t)ds_pairs(nt, causal != 0) * kDsTile * sizeof(float);
}

extern "C" int aar_flash_bwd_strided_plan_f32(const float* q, const float* k, const float* v, const float* o,
                                              const float* lse, const float* dout, float* dq, float* dk,
                                              float* dv, int64_t B, int64_t H, int64_t T, int64_t d,
                                              const int64_t* strides, int causal, float scale, int key_block,
                                              void* workspace, size_t workspace_bytes, void* stream) {
  if (key_block != 0 && key_block != 64 && key_block != 128) return AAR_EINVAL;
  if (B < 0 || H < 0 || T < 0 || d <= 0) return AAR_EINVAL;
  if (d > 128) return AAR_EINVAL;
  if (B == 0 || H == 0 || T == 0) return AAR_OK;
  if (!q || !k || !v || !o || !lse || !dout || !dq || !dk || !dv || !strides) return AAR_EINVAL;
  if (!fa_shape_ok(B * H, T, d) || H > INT32_MAX) return AAR_EUNSUPPORTED;
  const int64_t bh = B * H;
  if (!workspace || workspace_bytes < aar_flash_bwd_workspace_bytes(bh, T, d)) return AAR_EWORKSPACE;
  hipStream_t st = as_stream(stream);
  float* D = static_cast<float*>(workspace);
  const int64_t rows = bh * T;
  const bool dot_vec = fa_vec_ok(d, {o, dout}, strides + 9, 6);
  // four rows per 16-lane group where they never straddle two heads
  if (dot_vec && T % 4 == 0) {
    flash_bwd_dot_kernel<true, 4><<<dim3((unsigned)ceil_div(rows / 4 * 16, (int64_t)256)), dim3(256), 0, st>>>(
        fa_in(dout, strides + 12), fa_in(o, strides + 9), D, rows, (int)T, (int)H, (int)d);
  } else {
    auto dot_kernel = dot_vec ? flash_bwd_dot_kernel<true, 1> : flash_bwd_dot_kernel<false, 1>;
    dot_kernel<<<dim3((unsigned)ceil_div(rows * 16, (int64_t)256)), dim3(256), 0, st>>>(
        fa_in(dout, strides + 12), fa_in(o, strides + 9), D, rows, (int)T, (int)H, (int)d);
  }
  int rc = launch_status();
  if (rc != AAR_OK) return rc;
  const bool vec = fa_vec_ok(d, {q, k, v, dout, dq, dk, dv}, strides, 24);
  float* dS = workspace_bytes >= aar_flash_bwd_fast_workspace_bytes(bh, T, d, causal) && aligned16(workspace)
                  ? reinterpret_cast<float*>(static_cast<char*>(workspace) + fa_d_bytes(bh, T))
                  : nullptr;
  BwdArgs a{fa_in(q, strides),          fa_in(k, strides + 3),      fa_in(v, strides + 6),
            fa_in(dout, strides + 12),  lse,                        D,
            fa_out(dq, strides + 15),   fa_out(dk, strides + 18),   fa_out(dv, strides + 21),
            dS,                         (int)T,                     (int)d,
            (int)H,                     (int)bh,                    scale,
            fa_bwd_key_block(bh, T, d, causal != 0, vec, key_block),  st};
  return dispatch_fa<BwdLaunch>(pad_dim(d), causal != 0, vec, a);
}

extern "C" int aar_flash_bwd_strided_f32(const float* q, const float* k, const float* v, const float* o,
                                         const float* lse, const float* dout, float* dq, float* dk, float* dv,
                                         int64_t B, int64_t H, int64_t T, int64_t d, const int64_t* strides,
                                         int causal, float scale, void* workspace, size_t workspace_bytes,
                                         void* stream) {
  return aar_flash_bwd_strided_plan_f32(q, k, v, o, lse, dout, dq, dk, dv, B, H, T, d, strides, causal, scale, 0,
                                        workspace, workspace_bytes, stream);
}

extern "C" int aar_flash_bwd_f32(const float* q, const float* k, const float* v, const float* o,
                                 const float* lse, const float* dout, float* dq, float* dk, float* dv,
                                 int64_t bh, int64_t T, int64_t d, int causal, float scale,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  if (bh < 0 || T < 0 || d <= 0) return AAR_EINVAL;
  int64_t strides[24];
  for (int i = 0; i < 8; ++i) {
    strides[3 * i] = bh * T * d;
    strides[3 * i + 1] = T * d;
    strides[3 * i + 2] = d;
  }
  return aar_flash_bwd_strided_f32(q, k, v, o, lse, dout, dq, dk, dv, 1, bh, T, d, strides, causal, scale,
                                   workspace, workspace_bytes, stream);
}

extern "C" int aar_flash_fwd_plan(int64_t bh, int64_t T, int64_t d, int causal, int vec, size_t workspace_bytes,
                                  int* split_blocks) {
  if (!split_blocks || bh <= 0 || T <= 0 || d <= 0) return AAR_EINVAL;
  if (d > 128) return AAR_EINVAL;
  if (!fa_shape_ok(bh, T, d)) return AAR_EUNSUPPORTED;
  *split_blocks = 0;
  if (!causal || workspace_bytes < fa_fwd_split_bytes(bh, T, d) || fa_fwd_split_bytes(bh, T, d) == 0) return AAR_OK;
  const int64_t nqb = (T + kBlock - 1) / kBlock;
  const int dp = pad_dim(d);
  int resident = 1;
#define AAR_RES(DPV) \
  if (dp == DPV) resident = vec ? fa_fwd_resident<DPV, true>() : fa_fwd_resident<DPV, false>();
  AAR_RES(32)
  AAR_RES(64)
  AAR_RES(128)
#undef AAR_RES
  *split_blocks = fa_fwd_split_blocks(bh, nqb, (int64_t)device_cu_count() * resident);
  return AAR_OK;
}

extern "C" int aar_flash_bwd_plan(int64_t bh, int64_t T, int64_t d, int causal, int vec, int* key_block) {
  if (!key_block || bh <= 0 || T <= 0 || d <= 0) return AAR_EINVAL;
  if (d > 128) return AAR_EINVAL;
  if (!fa_shape_ok(bh, T, d)) return AAR_EUNSUPPORTED;
  *key_block = fa_bwd_key_block(bh, T, d, causal != 0, vec != 0);
  return AAR_OK;
}

extern "C" int aar_flash_fwd_query_block(int64_t bh, int64_t T, int64_t d, int causal, int vec, int* query_block) {
  if (!query_block || bh <= 0 || T <= 0 || d <= 0) return AAR_EINVAL;
  if (d > 128) return AAR_EINVAL;
  if (!fa_shape_ok(bh, T, d)) return AAR_EUNSUPPORTED;
  *query_block = fa_fwd_query_block(bh, T, d, causal != 0, vec != 0);
  return AAR_OK;
}
