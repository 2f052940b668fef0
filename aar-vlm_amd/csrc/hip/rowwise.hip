// Row-wise fp32 kernels over the last dim: softmax fwd/bwd and layernorm
// fwd (with or without stats) / bwd.  Reference semantics:
//   softmax_cpu / softmax_backward_cpu   cppsrc/ops/softmax.cpp:15-55
//   layernorm_cpu / _with_stats / _bwd   cppsrc/ops/layernorm.cpp:20-134
//
// HBM-bound design:
//  * A row is held in VGPRs for the whole op, so x (and g, y) cross HBM once:
//    softmax fwd moves 8*cols bytes per row, bwd 12*cols, layernorm fwd
//    8*cols (+8 for stats), bwd 12*cols (+8).
//  * Each row is owned by W waves (W = 1 up to 2048 columns, else 4); a lane
//    holds NV slots of 4 consecutive floats (one 128-bit load each) laid out
//    so every slot is a contiguous 1 KB segment across the wave.
//  * Reductions are wave64 DPP/ds_swizzle butterflies; with W = 4 the four
//    wave partials meet in LDS and are summed in a fixed order.
//  * Softmax and layernorm forward launch a grid that covers the rows once.
//    Layernorm backward's workgroups are persistent (a few per CU) and stride
//    over rows, so gamma stays in registers and dgamma/dbeta accumulate per
//    lane in registers; each workgroup writes one partial row to a workspace
//    and a fixed-order tree sums the partials.  No float atomics: the result
//    is bit-reproducible on a given device.
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>
#include <mutex>

#include "common.hpp"

namespace aar {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// One lane's share of a row: NV slots of 4 floats (VEC: 128-bit accesses, the
// row must be 16-byte aligned with cols % 4 == 0) or NV single floats.
template <int NV, int W, bool VEC>
struct RowSlots {
  static constexpr int kElem = VEC ? 4 : 1;
  static constexpr int kN = NV * kElem;
  float v[kN];

  // Column of element e (0..kElem-1) of slot i for lane `lane` of wave `wr`.
  __device__ __forceinline__ static int col(int i, int e, int wr, int lane) {
    return ((i * W + wr) * kWave + lane) * kElem + e;
  }

  // STREAM: the data is touched once (nontemporal hint, keeps it from
  // displacing reused lines such as gamma/beta).
  template <bool STREAM = true>
  __device__ __forceinline__ void load(const float* __restrict__ row, int cols, int wr, int lane) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c0 = col(i, 0, wr, lane);
      if (VEC) {
        f32x4 t = {0.f, 0.f, 0.f, 0.f};
        if (c0 < cols) {
          const f32x4* src = reinterpret_cast<const f32x4*>(row + c0);
          t = STREAM ? __builtin_nontemporal_load(src) : *src;
        }
        v[4 * i + 0] = t[0];
        v[4 * i + 1] = t[1];
        v[4 * i + 2] = t[2];
        v[4 * i + 3] = t[3];
      } else {
        v[i] = c0 < cols ? row[c0] : 0.f;
      }
    }
  }

  __device__ __forceinline__ void store(float* __restrict__ row, int cols, int wr, int lane) const {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c0 = col(i, 0, wr, lane);
      if (c0 >= cols) continue;
      if (VEC) {
        f32x4 t = {v[4 * i + 0], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
        __builtin_nontemporal_store(t, reinterpret_cast<f32x4*>(row + c0));
      } else {
        row[c0] = v[i];
      }
    }
  }

  __device__ __forceinline__ bool valid(int k, int cols, int wr, int lane) const {
    return col(k / kElem, k % kElem, wr, lane) < cols;
  }
};

// Row-group reduction: full wave reduction, then (W > 1) a fixed-order sum of
// the W wave partials through LDS.  `slot` selects a private LDS cell set; all
// waves of the workgroup must call this uniformly.
template <int W, bool MAX, int NW = kWaves>
__device__ __forceinline__ float group_reduce(float v, float* red, int slot, int grp, int wr,
                                              int lane) {
  v = MAX ? wave_max(v) : wave_sum(v);
  if (W == 1) return v;
  float* cell = red + (slot * NW + grp * W);
  if (lane == 0) cell[wr] = v;
  __syncthreads();
  float r = cell[0];
#pragma unroll
  for (int i = 1; i < W; ++i) r = MAX ? fmaxf(r, cell[i]) : r + cell[i];
  return r;
}

// Rows each row group handles per iteration: their loads are all issued
// before the first reduction, so several KB per wave are in flight (a single
// small row leaves HBM latency exposed).
template <int NV, int W>
struct RowsPerIter {
  static_assert(W == 1 || NV <= 8, "row-group size");
  static constexpr int value = W == 1 && NV <= 4 ? 2 : 1;
};

inline int rows_per_iter(int nv, int w) { return w == 1 && nv <= 4 ? 2 : 1; }

// Workgroups to cover the rows once, capped at `per_cu` workgroups per CU.
// Softmax and layernorm forward use a covering grid (one pass per
// workgroup, no row loop), which streams HBM faster on MI355X than a
// persistent grid: the dispatcher walks the workgroups in address order, so
// the in-flight rows form one compact window.  Layernorm backward keeps a
// persistent grid because each workgroup emits one dgamma/dbeta partial row.
constexpr int kCoverPerCu = 1 << 12;
// Layernorm forward over rows of several waves (W > 1: one row per workgroup
// and iteration) loads its gamma/beta slots once per workgroup: a covering
// grid reloads them for every row (as many L2 bytes as the row's HBM bytes),
// so those plans cap the grid at 64 workgroups per CU and loop over 4+ rows.
// Measured at 4096 columns: 5.74 -> 6.05 TB/s (cap 128: 5.99, 32: 5.91).
constexpr int kLnFwdWidePerCu = 64;
inline int rows_grid(int64_t rows, int nv, int W, int per_cu) {
  const int64_t per_wg_iter = (int64_t)(kWaves / W) * rows_per_iter(nv, W);
  const int64_t need = ceil_div(rows, per_wg_iter);
  const int64_t cap = (int64_t)device_cu_count() * per_cu;
  return (int)(need < cap ? need : cap);
}

// First row of row group `grp` in iteration `it`; the group's rows are
// row0 .. row0 + U - 1.
__device__ __forceinline__ int64_t group_row0(int64_t it, int per_iter, int grp, int U) {
  return ((it * gridDim.x + blockIdx.x) * per_iter + grp) * U;
}

// Rows wider than the register plans take one workgroup each; a dispatch
// holds each grid extent as a 32-bit work-item count.
inline bool wide_grid_ok(int64_t rows) { return rows * kThreads <= (int64_t)UINT32_MAX; }

// LDS cells used by group_reduce: 2 parities x U rows (at most 8) x 2
// reductions x 4 waves.  (W == 1 row groups reduce within the wave and use
// no cells.)
constexpr int kMaxRowsPerIter = 8;
constexpr int kRedCells = 2 * kMaxRowsPerIter * 2 * kWaves;

// ------------------------------------------------------------------ softmax

template <int NV, int W, bool VEC>
__global__ void __launch_bounds__(kThreads)
softmax_fwd_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t rows, int cols) {
  constexpr int U = RowsPerIter<NV, W>::value;
  __shared__ float red[kRedCells];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = wave / W, wr = wave % W;
  constexpr int per_iter = kWaves / W;
  const int64_t iters = ceil_div(rows, (int64_t)gridDim.x * per_iter * U);
  using RS = RowSlots<NV, W, VEC>;
  for (int64_t it = 0; it < iters; ++it) {
    const int64_t row0 = group_row0(it, per_iter, grp, U);
    RS s[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (row0 + u < rows) s[u].load(x + (row0 + u) * cols, cols, wr, lane);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = row0 + u < rows;
      float mx = -INFINITY;
#pragma unroll
      for (int k = 0; k < RS::kN; ++k)
        if (live && s[u].valid(k, cols, wr, lane)) mx = fmaxf(mx, s[u].v[k]);
      mx = group_reduce<W, true>(mx, red, (((int)(it & 1) * U + u) * 2 + 0), grp, wr, lane);
      float sum = 0.f;
#pragma unroll
      for (int k = 0; k < RS::kN; ++k) {
        const float e = (live && s[u].valid(k, cols, wr, lane)) ? expf(s[u].v[k] - mx) : 0.f;
        s[u].v[k] = e;
        sum += e;
      }
      sum = group_reduce<W, false>(sum, red, (((int)(it & 1) * U + u) * 2 + 1), grp, wr, lane);
      const float inv = 1.0f / sum;
#pragma unroll
      for (int k = 0; k < RS::kN; ++k) s[u].v[k] *= inv;
      if (live) s[u].store(y + (row0 + u) * cols, cols, wr, lane);
    }
  }
}

template <int NV, int W, bool VEC>
__global__ void __launch_bounds__(kThreads)
softmax_bwd_kernel(const float* __restrict__ g, const float* __restrict__ y, float* __restrict__ dx,
                   int64_t rows, int cols) {
  constexpr int U = RowsPerIter<NV, W>::value;
  __shared__ float red[kRedCells];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = wave / W, wr = wave % W;
  constexpr int per_iter = kWaves / W;
  const int64_t iters = ceil_div(rows, (int64_t)gridDim.x * per_iter * U);
  using RS = RowSlots<NV, W, VEC>;
  for (int64_t it = 0; it < iters; ++it) {
    const int64_t row0 = group_row0(it, per_iter, grp, U);
    RS sg[U], sy[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (row0 + u < rows) {
        sg[u].load(g + (row0 + u) * cols, cols, wr, lane);
        sy[u].load(y + (row0 + u) * cols, cols, wr, lane);
      } else {
#pragma unroll
        for (int k = 0; k < RS::kN; ++k) sg[u].v[k] = sy[u].v[k] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float dot = 0.f;
#pragma unroll
      for (int k = 0; k < RS::kN; ++k) dot += sg[u].v[k] * sy[u].v[k];  // padding slots are zero
      dot = group_reduce<W, false>(dot, red, (((int)(it & 1) * U + u) * 2), grp, wr, lane);
#pragma unroll
      for (int k = 0; k < RS::kN; ++k) sg[u].v[k] = sy[u].v[k] * (sg[u].v[k] - dot);
      if (row0 + u < rows) sg[u].store(dx + (row0 + u) * cols, cols, wr, lane);
    }
  }
}

// ---------------------------------------------------------------- layernorm

template <int NV, int W, bool VEC, bool STATS>
__global__ void __launch_bounds__(kThreads)
layernorm_fwd_kernel(const float* __restrict__ x, const float* __restrict__ w,
                     const float* __restrict__ b, float* __restrict__ y, float* __restrict__ mean,
                     float* __restrict__ rstd, int64_t rows, int cols, float eps) {
  constexpr int U = RowsPerIter<NV, W>::value;
  __shared__ float red[kRedCells];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = wave / W, wr = wave % W;
  constexpr int per_iter = kWaves / W;
  const int64_t iters = ceil_div(rows, (int64_t)gridDim.x * per_iter * U);
  using RS = RowSlots<NV, W, VEC>;
  __shared__ float stat[2][2][per_iter * U];
  RS sw, sb;
  sw.template load<false>(w, cols, wr, lane);
  sb.template load<false>(b, cols, wr, lane);
  const float inv_d = 1.0f / (float)cols;
  for (int64_t it = 0; it < iters; ++it) {
    const int64_t row0 = group_row0(it, per_iter, grp, U);
    RS s[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (row0 + u < rows) {
        s[u].load(x + (row0 + u) * cols, cols, wr, lane);
      } else {
#pragma unroll
        for (int k = 0; k < RS::kN; ++k) s[u].v[k] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t row = row0 + u;
      float sum = 0.f;
#pragma unroll
      for (int k = 0; k < RS::kN; ++k) sum += s[u].v[k];
      sum = group_reduce<W, false>(sum, red, (((int)(it & 1) * U + u) * 2 + 0), grp, wr, lane);
      const float mu = sum * inv_d;
      float sq = 0.f;
#pragma unroll
      for (int k = 0; k < RS::kN; ++k) {
        const float dlt = s[u].valid(k, cols, wr, lane) ? s[u].v[k] - mu : 0.f;
        sq += dlt * dlt;
      }
      sq = group_reduce<W, false>(sq, red, (((int)(it & 1) * U + u) * 2 + 1), grp, wr, lane);
      const float var = sq * inv_d;
      const float r = 1.0f / sqrtf(var + eps);
#pragma unroll
      for (int k = 0; k < RS::kN; ++k) s[u].v[k] = (s[u].v[k] - mu) * r * sw.v[k] + sb.v[k];
      if (row < rows) s[u].store(y + row * cols, cols, wr, lane);
      if (STATS && wr == 0 && lane == 0) {
        stat[it & 1][0][grp * U + u] = mu;
        stat[it & 1][1][grp * U + u] = r;
      }
    }
    if (STATS) {
      // The workgroup's rows of this iteration are consecutive: write their
      // statistics as one contiguous run per array instead of scattered
      // single floats.  (Parity-buffered, so one barrier per iteration.)
      __syncthreads();
      const int64_t base = group_row0(it, per_iter, 0, U);
      const int t = threadIdx.x;
      if (t < per_iter * U && base + t < rows) {
        mean[base + t] = stat[it & 1][0][t];
        rstd[base + t] = stat[it & 1][1][t];
      }
    }
  }
}

// Layernorm-backward shape per row plan (NV slots per lane, W waves per row):
//  * waves per workgroup: 8 for rows spread over 4 waves with up to 4 slots
//    per lane (measured faster on MI355X than four 4-wave workgroups per
//    CU), else 4 (16-wave workgroups, which would cut the partial rows 4x,
//    measured slower);
//  * rows per row group and iteration (all loads issued before the first
//    reduction);
//  * minimum waves per SIMD the register allocation must allow;
//  * next-rows prefetch (two row sets in flight per wave): measured slower
//    than the occupancy it costs, so off;
//  * resident waves per CU the persistent grid is sized for.
constexpr int ln_bwd_waves(int nv, int w) { return (w > 1 && nv <= 4) ? 8 : 4; }
constexpr int ln_bwd_rows(int nv, int w) { return w == 1 && nv <= 4 ? 2 : 1; }
constexpr int ln_bwd_min_waves(int nv, int w, bool acc = false) {
  // (the accumulating 768-column instance holds an addend row besides the two
  // rows in flight: at 4 waves per SIMD it spilled 25 VGPRs)
  return w == 1 && nv == 3 ? (acc ? 3 : 4) : 1;
}
constexpr bool ln_bwd_prefetch(int, int) { return false; }
constexpr int kLnBwdWavesPerCu = 16;

// Rows U of row group `grp` starting at row0: gy and x slots, mean and rstd
// (rows past the end read as zeros and are never stored).
template <int U, typename RS>
__device__ __forceinline__ void ln_bwd_load(RS (&sg)[U], RS (&sx)[U], float (&mu)[U], float (&r)[U],
                                            const float* __restrict__ gy, const float* __restrict__ x,
                                            const float* __restrict__ mean, const float* __restrict__ rstd,
                                            int64_t row0, int64_t rows, int cols, int wr, int lane) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (row0 + u < rows) {
      sg[u].load(gy + (row0 + u) * cols, cols, wr, lane);
      sx[u].load(x + (row0 + u) * cols, cols, wr, lane);
      mu[u] = mean[row0 + u];
      r[u] = rstd[row0 + u];
    } else {
#pragma unroll
      for (int k = 0; k < RS::kN; ++k) sg[u].v[k] = sx[u].v[k] = 0.f;
      mu[u] = 0.f;
      r[u] = 0.f;
    }
  }
}

// Stage 1 of layernorm backward: dx per row, plus per-workgroup partial
// column sums of gy*xhat (dgamma) and gy (dbeta) written to
// part[blockIdx.x][2][cols].  Workgroups of NW waves are persistent (as many
// as fit on the device at once, at most 16 waves per CU) and stride over the
// rows.  PF: the next iteration's rows are loaded before the current ones
// are reduced, so each wave keeps two row sets in flight.  ACC: dx is added
// onto `addend` (dx = addend + value, the fp32 addition of a gradient
// fan-in); the addend row is loaded once the row's reductions are done, so
// it costs no registers while gy and x are held.  EARLY (narrow rows, NV <=
// 2, without PF): the addend rows are loaded with gy and x instead, so a row
// waits for one memory round trip, not two; the host takes it for grids
// below the resident cap (short inputs: 16384 x 384, 27.2 -> 23.5 us), where
// each workgroup runs only a few row iterations (at 65536 rows, persistent
// workgroups, it measured 75.0 -> 77.5 us).
template <int NV, int W, bool VEC, int NW, bool PF, bool ACC, bool EARLY = false>
__global__ void __launch_bounds__(NW * 64, ln_bwd_min_waves(NV, W, ACC))
layernorm_bwd_kernel(const float* __restrict__ gy, const float* __restrict__ x,
                     const float* __restrict__ w, const float* __restrict__ mean,
                     const float* __restrict__ rstd, const float* addend, float* dx,
                     float* __restrict__ part, int64_t rows, int cols) {
  constexpr int U = ln_bwd_rows(NV, W);
  constexpr int per_iter = NW / W;
  __shared__ float red[2 * kMaxRowsPerIter * 2 * NW];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = wave / W, wr = wave % W;
  const int64_t iters = ceil_div(rows, (int64_t)gridDim.x * per_iter * U);
  using RS = RowSlots<NV, W, VEC>;
  RS sw, dwacc, dbacc;
  sw.template load<false>(w, cols, wr, lane);
#pragma unroll
  for (int k = 0; k < RS::kN; ++k) {
    dwacc.v[k] = 0.f;
    dbacc.v[k] = 0.f;
  }
  const float inv_d = 1.0f / (float)cols;
  RS sg[U], sx[U];
  float mu[U], r[U];
  constexpr bool kEarlyAddend = ACC && EARLY && !PF && NV <= 2;
  RS sa_early[kEarlyAddend ? U : 1];
  if (PF) ln_bwd_load<U>(sg, sx, mu, r, gy, x, mean, rstd, group_row0(0, per_iter, grp, U), rows, cols, wr, lane);
  for (int64_t it = 0; it < iters; ++it) {
    const int64_t row0 = group_row0(it, per_iter, grp, U);
    if (!PF) ln_bwd_load<U>(sg, sx, mu, r, gy, x, mean, rstd, row0, rows, cols, wr, lane);
    if constexpr (kEarlyAddend) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (row0 + u < rows) sa_early[u].load(addend + (row0 + u) * cols, cols, wr, lane);
    }
    RS ng[U], nx[U];
    float nmu[U], nr[U];
    if (PF && it + 1 < iters) {
      ln_bwd_load<U>(ng, nx, nmu, nr, gy, x, mean, rstd, group_row0(it + 1, per_iter, grp, U), rows, cols, wr,
                     lane);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float sum_g = 0.f, sum_gn = 0.f;
#pragma unroll
      for (int k = 0; k < RS::kN; ++k) {
        const float n = (sx[u].v[k] - mu[u]) * r[u];
        const float gg = sg[u].v[k] * sw.v[k];
        sum_g += gg;
        sum_gn += gg * n;
        dwacc.v[k] += sg[u].v[k] * n;
        dbacc.v[k] += sg[u].v[k];
        sx[u].v[k] = n;  // keep xhat
      }
      sum_g = group_reduce<W, false, NW>(sum_g, red, (((int)(it & 1) * U + u) * 2 + 0), grp, wr, lane);
      sum_gn = group_reduce<W, false, NW>(sum_gn, red, (((int)(it & 1) * U + u) * 2 + 1), grp, wr, lane);
      RS sa;
      if constexpr (kEarlyAddend) {
        sa = sa_early[u];
      } else if (ACC) {
        // (the empty asm keeps the compiler from hoisting these loads above the
        // reductions, where they would hold registers beside gy and x)
        asm volatile("" ::: "memory");
        if (row0 + u < rows) sa.load(addend + (row0 + u) * cols, cols, wr, lane);
      }
#pragma unroll
      for (int k = 0; k < RS::kN; ++k) {
        const float gg = sg[u].v[k] * sw.v[k];
        sg[u].v[k] = r[u] * (gg - sum_g * inv_d - sx[u].v[k] * sum_gn * inv_d);
      }
      if (ACC) {
        // a separately rounded addition (no fma with the product above), as
        // the add of a gradient fan-in performs it
#pragma clang fp contract(off)
#pragma unroll
        for (int k = 0; k < RS::kN; ++k) sg[u].v[k] = sa.v[k] + sg[u].v[k];
      }
      if (row0 + u < rows) sg[u].store(dx + (row0 + u) * cols, cols, wr, lane);
    }
    if (PF) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        sg[u] = ng[u];
        sx[u] = nx[u];
        mu[u] = nmu[u];
        r[u] = nr[u];
      }
    }
  }
  // Combine the row groups of this workgroup in a fixed order: group 0 seeds
  // the LDS accumulator, groups 1.. add in turn, then group 0's waves write
  // the workgroup's partial row.
  if (per_iter == 1) {
    float* pw = part + (int64_t)blockIdx.x * 2 * cols;
    dwacc.store(pw, cols, wr, lane);
    dbacc.store(pw + cols, cols, wr, lane);
    return;
  }
  __shared__ float stage[2][RS::kN * kWave * W];
#pragma unroll 1
  for (int gi = 0; gi < per_iter; ++gi) {
    if (grp == gi) {
#pragma unroll
      for (int k = 0; k < RS::kN; ++k) {
        const int o = (k * W + wr) * kWave + lane;
        stage[0][o] = gi == 0 ? dwacc.v[k] : stage[0][o] + dwacc.v[k];
        stage[1][o] = gi == 0 ? dbacc.v[k] : stage[1][o] + dbacc.v[k];
      }
    }
    __syncthreads();
  }
  if (grp == 0) {
#pragma unroll
    for (int k = 0; k < RS::kN; ++k) {
      const int o = (k * W + wr) * kWave + lane;
      dwacc.v[k] = stage[0][o];
      dbacc.v[k] = stage[1][o];
    }
    float* pw = part + (int64_t)blockIdx.x * 2 * cols;
    dwacc.store(pw, cols, wr, lane);
    dbacc.store(pw + cols, cols, wr, lane);
  }
}

// Stage 2 of layernorm backward: dw[c] and db[c] from the partial rows
// part[p][0..2C) (dgamma in [0,C), dbeta in [C,2C)).  A workgroup of
// kRedThreads threads owns V consecutive columns of the 2C (V = 4: one
// 128-bit load per partial row, when C % 4 == 0 and the partials are 16-byte
// aligned; else V = 1), so the grid has 2C / V workgroups and every load of a
// thread is issued before the first add.  Thread t sums parts t, t + 256, ...
// in that order; the 256 sums of a column then meet in a fixed tree (a wave
// butterfly, then the four waves in order through LDS).  Deterministic.
//
// Workgroups are dealt round-robin over the 8 XCDs (hardware id b runs on
// XCD b % 8).  Ids are remapped so each XCD owns one contiguous run of column
// blocks: the 128-byte lines of a partial row are then fetched into one XCD's
// L2 instead of up to eight.
constexpr int kRedThreads = 256;
constexpr int kXcds = 8;

__device__ __forceinline__ int xcd_contiguous_block(int b, int nblk) {
  const int q = nblk / kXcds, r = nblk % kXcds, x = b % kXcds;
  return x * q + min(x, r) + b / kXcds;
}

template <int V>
__global__ void __launch_bounds__(kRedThreads)
layernorm_bwd_reduce_kernel(const float* __restrict__ part, float* __restrict__ dw, float* __restrict__ db,
                            int nparts, int cols) {
  __shared__ float acc[kRedThreads / kWave][V];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t ncol2 = 2 * (int64_t)cols;
  const int64_t nblk = ncol2 / V;
  // More blocks than one grid holds (over 2^16 of them) loop with the grid's stride.
  for (int64_t blk = xcd_contiguous_block(blockIdx.x, gridDim.x); blk < nblk; blk += gridDim.x) {
    const int64_t c0 = blk * V;
    float s[V];
#pragma unroll
    for (int v = 0; v < V; ++v) s[v] = 0.f;
#pragma unroll 4
    for (int p = threadIdx.x; p < nparts; p += kRedThreads) {
      const float* src = part + (int64_t)p * ncol2 + c0;
      if constexpr (V == 4) {
        const f32x4 t = *reinterpret_cast<const f32x4*>(src);
#pragma unroll
        for (int v = 0; v < 4; ++v) s[v] += t[v];
      } else {
        s[0] += *src;
      }
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const float w = wave_sum(s[v]);
      if (lane == 0) acc[wave][v] = w;
    }
    __syncthreads();
    if (threadIdx.x < V) {
      const int v = threadIdx.x;
      float t = acc[0][v];
#pragma unroll
      for (int i = 1; i < kRedThreads / kWave; ++i) t += acc[i][v];
      const int64_t c = c0 + v;
      if (c < cols) {
        dw[c] = t;
      } else {
        db[c - cols] = t;
      }
    }
    __syncthreads();
  }
}

// ------------------------------------------------------- generic wide rows
// Rows wider than the register-resident kernels cover: one workgroup per row,
// three passes over the row (re-reads hit L2).

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < kWaves; ++i) r += red[i];
  return r;
}

__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < kWaves; ++i) r = fmaxf(r, red[i]);
  return r;
}

__global__ void __launch_bounds__(kThreads)
softmax_fwd_wide_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t cols) {
  __shared__ float red[kWaves];
  const float* xr = x + (int64_t)blockIdx.x * cols;
  float* yr = y + (int64_t)blockIdx.x * cols;
  float mx = -INFINITY;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) mx = fmaxf(mx, xr[c]);
  mx = block_max(mx, red);
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
    const float e = expf(xr[c] - mx);
    yr[c] = e;
    s += e;
  }
  s = block_sum(s, red);
  const float inv = 1.0f / s;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) yr[c] *= inv;
}

__global__ void __launch_bounds__(kThreads)
softmax_bwd_wide_kernel(const float* __restrict__ g, const float* __restrict__ y,
                        float* __restrict__ dx, int64_t cols) {
  __shared__ float red[kWaves];
  const int64_t off = (int64_t)blockIdx.x * cols;
  float dot = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) dot += g[off + c] * y[off + c];
  dot = block_sum(dot, red);
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) dx[off + c] = y[off + c] * (g[off + c] - dot);
}

__global__ void __launch_bounds__(kThreads)
layernorm_fwd_wide_kernel(const float* __restrict__ x, const float* __restrict__ w,
                          const float* __restrict__ b, float* __restrict__ y,
                          float* __restrict__ mean, float* __restrict__ rstd, int64_t cols,
                          float eps) {
  __shared__ float red[kWaves];
  const int64_t off = (int64_t)blockIdx.x * cols;
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) s += x[off + c];
  const float mu = block_sum(s, red) / (float)cols;
  float q = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
    const float d = x[off + c] - mu;
    q += d * d;
  }
  const float var = block_sum(q, red) / (float)cols;
  const float r = 1.0f / sqrtf(var + eps);
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) y[off + c] = (x[off + c] - mu) * r * w[c] + b[c];
  if (mean && threadIdx.x == 0) {
    mean[blockIdx.x] = mu;
    rstd[blockIdx.x] = r;
  }
}

// One workgroup per row for dx; dgamma/dbeta partials: workgroup p covers rows
// p, p + gridDim.x, ... and accumulates per column in a strided loop.
__global__ void __launch_bounds__(kThreads)
layernorm_bwd_wide_kernel(const float* __restrict__ gy, const float* __restrict__ x,
                          const float* __restrict__ w, const float* __restrict__ mean,
                          const float* __restrict__ rstd, const float* addend, float* dx, int64_t cols) {
  __shared__ float red[kWaves];
  const int64_t off = (int64_t)blockIdx.x * cols;
  const float mu = mean[blockIdx.x], r = rstd[blockIdx.x];
  float sg = 0.f, sgn = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
    const float n = (x[off + c] - mu) * r;
    const float gg = gy[off + c] * w[c];
    sg += gg;
    sgn += gg * n;
  }
  sg = block_sum(sg, red);
  sgn = block_sum(sgn, red);
  const float inv_d = 1.0f / (float)cols;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
    const float n = (x[off + c] - mu) * r;
    const float gg = gy[off + c] * w[c];
    const float v = r * (gg - sg * inv_d - n * sgn * inv_d);
    if (addend) {
#pragma clang fp contract(off)
      dx[off + c] = addend[off + c] + v;  // separately rounded, as the fan-in's add
    } else {
      dx[off + c] = v;
    }
  }
}

__global__ void __launch_bounds__(kThreads)
layernorm_bwd_wide_cols_kernel(const float* __restrict__ gy, const float* __restrict__ x,
                               const float* __restrict__ mean, const float* __restrict__ rstd,
                               float* __restrict__ part, int64_t rows, int64_t cols) {
  // part[blockIdx.y][2][cols]: rows blockIdx.y, blockIdx.y + gridDim.y, ...
  const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (c >= cols) return;
  float a = 0.f, b = 0.f;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const float g = gy[r * cols + c];
    a += g * ((x[r * cols + c] - mean[r]) * rstd[r]);
    b += g;
  }
  part[(int64_t)blockIdx.y * 2 * cols + c] = a;
  part[(int64_t)blockIdx.y * 2 * cols + cols + c] = b;
}

// ------------------------------------------------------------ dispatching

struct RowPlan {
  int nv;   // slots per lane: 1, 2, 3, 4 or 8 (0 = use the wide kernels)
  int w;    // waves per row: 1 or 4
  bool vec;
};

RowPlan plan_rows(int64_t cols, bool vec) {
  const int64_t units = vec ? cols / 4 : cols;  // slots needed per row
  RowPlan p{0, 1, vec};
  for (int w : {1, 4}) {
    for (int nv : {1, 2, 3, 4, 8}) {
      if (units <= (int64_t)nv * kWave * w) {
        if (w == 4 && (nv < 2 || nv == 3)) continue;
        p.nv = nv;
        p.w = w;
        return p;
      }
    }
  }
  return p;
}

#define AAR_ROW_DISPATCH(PLAN, LAUNCH)                 \
  do {                                                  \
    if ((PLAN).vec) {                                   \
      if ((PLAN).w == 1) {                              \
        switch ((PLAN).nv) {                            \
          case 1: LAUNCH(1, 1, true); break;            \
          case 2: LAUNCH(2, 1, true); break;            \
          case 3: LAUNCH(3, 1, true); break;            \
          case 4: LAUNCH(4, 1, true); break;            \
          default: LAUNCH(8, 1, true); break;           \
        }                                               \
      } else {                                          \
        switch ((PLAN).nv) {                            \
          case 2: LAUNCH(2, 4, true); break;            \
          case 4: LAUNCH(4, 4, true); break;            \
          default: LAUNCH(8, 4, true); break;           \
        }                                               \
      }                                                 \
    } else {                                            \
      if ((PLAN).w == 1) {                              \
        switch ((PLAN).nv) {                            \
          case 1: LAUNCH(1, 1, false); break;           \
          case 2: LAUNCH(2, 1, false); break;           \
          case 3: LAUNCH(3, 1, false); break;           \
          case 4: LAUNCH(4, 1, false); break;           \
          default: LAUNCH(8, 1, false); break;          \
        }                                               \
      } else {                                          \
        switch ((PLAN).nv) {                            \
          case 2: LAUNCH(2, 4, false); break;           \
          case 4: LAUNCH(4, 4, false); break;           \
          default: LAUNCH(8, 4, false); break;          \
        }                                               \
      }                                                 \
    }                                                   \
  } while (0)

// Workgroups of a layernorm-backward instance resident on one CU at once
// (register- and LDS-limited), from the runtime's occupancy calculator.
template <int NV, int W, bool V>
int ln_bwd_resident() {
  static const int n = [] {
    int b = 0;
    constexpr int nw = ln_bwd_waves(NV, W);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &b, layernorm_bwd_kernel<NV, W, V, nw, ln_bwd_prefetch(NV, W), false>, nw * kWave, 0) != hipSuccess) {
      b = 1;
    }
    return b > 0 ? b : 1;
  }();
  return n;
}

// Number of dgamma/dbeta partial rows = persistent workgroups of the
// backward kernel: as many as are resident at once, at most
// kLnBwdWavesPerCu waves per CU, so no workgroup waits for a second round.
int ln_bwd_parts_for(int64_t rows, const RowPlan& p, bool* below_cap = nullptr) {
  const int64_t cus = device_cu_count();
  int64_t cap, pass;
  if (p.nv == 0) {
    cap = cus * 4;
    pass = 1;
  } else {
    const int nw = ln_bwd_waves(p.nv, p.w);
    int resident = 1;
#define R(NV, W, V) resident = ln_bwd_resident<NV, W, V>()
    AAR_ROW_DISPATCH(p, R);
#undef R
    cap = cus * std::min(resident, kLnBwdWavesPerCu / nw);
    // at least 32 rows per workgroup: below the cap (short inputs) fewer,
    // longer workgroups write fewer partial rows (16384 x 384: 20.8 -> 20.2 us,
    // x 768: 35.7 -> 33.4 us; 64 rows was slower again)
    pass = std::max<int64_t>((int64_t)(nw / p.w) * ln_bwd_rows(p.nv, p.w), 32);
  }
  const int64_t need = ceil_div(rows, pass);
  if (below_cap) *below_cap = need < cap;
  return (int)(need < cap ? need : cap);
}
// Workspace sizing does not know the pointers' alignment: cover both plans.
int ln_bwd_parts_max(int64_t rows, int64_t cols) {
  const int a = ln_bwd_parts_for(rows, plan_rows(cols, true));
  const int b = ln_bwd_parts_for(rows, plan_rows(cols, false));
  return a > b ? a : b;
}

}  // namespace
}  // namespace aar

using namespace aar;

extern "C" int aar_softmax_fwd_f32(const float* x, float* y, int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols <= 0) return AAR_EINVAL;
  if (rows == 0) return AAR_OK;
  if (!x || !y || cols > INT32_MAX) return AAR_EINVAL;
  hipStream_t st = as_stream(stream);
  const RowPlan p = plan_rows(cols, cols % 4 == 0 && aligned16(x) && aligned16(y));
  if (p.nv == 0) {
    if (!wide_grid_ok(rows)) return AAR_EUNSUPPORTED;
    softmax_fwd_wide_kernel<<<dim3((unsigned)rows), dim3(kThreads), 0, st>>>(x, y, cols);
    return launch_status();
  }
  const int grid = rows_grid(rows, p.nv, p.w, kCoverPerCu);
#define L(NV, W, V) softmax_fwd_kernel<NV, W, V><<<dim3(grid), dim3(kThreads), 0, st>>>(x, y, rows, (int)cols)
  AAR_ROW_DISPATCH(p, L);
#undef L
  return launch_status();
}

extern "C" int aar_softmax_bwd_f32(const float* g, const float* y, float* dx, int64_t rows, int64_t cols,
                                   void* stream) {
  if (rows < 0 || cols <= 0) return AAR_EINVAL;
  if (rows == 0) return AAR_OK;
  if (!g || !y || !dx || cols > INT32_MAX) return AAR_EINVAL;
  hipStream_t st = as_stream(stream);
  const RowPlan p = plan_rows(cols, cols % 4 == 0 && aligned16(g) && aligned16(y) && aligned16(dx));
  if (p.nv == 0) {
    if (!wide_grid_ok(rows)) return AAR_EUNSUPPORTED;
    softmax_bwd_wide_kernel<<<dim3((unsigned)rows), dim3(kThreads), 0, st>>>(g, y, dx, cols);
    return launch_status();
  }
  const int grid = rows_grid(rows, p.nv, p.w, kCoverPerCu);
#define L(NV, W, V) \
  softmax_bwd_kernel<NV, W, V><<<dim3(grid), dim3(kThreads), 0, st>>>(g, y, dx, rows, (int)cols)
  AAR_ROW_DISPATCH(p, L);
#undef L
  return launch_status();
}

extern "C" int aar_layernorm_fwd_f32(const float* x, const float* w, const float* b, float* y,
                                     float* mean, float* rstd, int64_t rows, int64_t cols, float eps,
                                     void* stream) {
  if (rows < 0 || cols <= 0 || !(eps > 0.f)) return AAR_EINVAL;
  if (rows == 0) return AAR_OK;
  if (!x || !w || !b || !y || cols > INT32_MAX) return AAR_EINVAL;
  const bool stats = mean && rstd;
  hipStream_t st = as_stream(stream);
  const bool vec = cols % 4 == 0 && aligned16(x) && aligned16(y) && aligned16(w) && aligned16(b);
  const RowPlan p = plan_rows(cols, vec);
  if (p.nv == 0) {
    if (!wide_grid_ok(rows)) return AAR_EUNSUPPORTED;
    layernorm_fwd_wide_kernel<<<dim3((unsigned)rows), dim3(kThreads), 0, st>>>(
        x, w, b, y, stats ? mean : nullptr, stats ? rstd : nullptr, cols, eps);
    return launch_status();
  }
  const int grid = rows_grid(rows, p.nv, p.w, p.w > 1 ? kLnFwdWidePerCu : kCoverPerCu);
  if (stats) {
#define L(NV, W, V)                                                                              \
  layernorm_fwd_kernel<NV, W, V, true><<<dim3(grid), dim3(kThreads), 0, st>>>(x, w, b, y, mean, \
                                                                              rstd, rows,       \
                                                                              (int)cols, eps)
    AAR_ROW_DISPATCH(p, L);
#undef L
  } else {
#define L(NV, W, V)                                                                    \
  layernorm_fwd_kernel<NV, W, V, false><<<dim3(grid), dim3(kThreads), 0, st>>>(       \
      x, w, b, y, nullptr, nullptr, rows, (int)cols, eps)
    AAR_ROW_DISPATCH(p, L);
#undef L
  }
  return launch_status();
}

extern "C" size_t aar_layernorm_bwd_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  const int64_t parts = ln_bwd_parts_max(rows, cols);
  return (size_t)parts * 2 * (size_t)cols * sizeof(float);
}

namespace aar {
namespace {

// 128-bit load path: 16-byte aligned rows and partials.
bool ln_bwd_vec(const void* gy, const void* x, const void* w, const void* dx, const void* ws, int64_t cols) {
  return cols % 4 == 0 && aligned16(gy) && aligned16(x) && aligned16(w) && aligned16(dx) && aligned16(ws);
}

// Workspace the plan for these operands needs (partial rows).
size_t ln_bwd_need_bytes(int64_t rows, int64_t cols, bool vec) {
  return (size_t)ln_bwd_parts_for(rows, plan_rows(cols, vec)) * 2 * (size_t)cols * sizeof(float);
}

int layernorm_bwd_run(const float* gy, const float* x, const float* w, const float* mean, const float* rstd,
                      const float* addend, float* dx, float* dw, float* db, int64_t rows, int64_t cols,
                      void* workspace, size_t workspace_bytes, void* stream) {
  if (rows < 0 || cols <= 0) return AAR_EINVAL;
  if (!dw || !db || cols > INT32_MAX) return AAR_EINVAL;
  hipStream_t st = as_stream(stream);
  if (rows == 0) {
    int rc = aar_memset_zero(dw, cols * sizeof(float), stream);
    if (rc == AAR_OK) rc = aar_memset_zero(db, cols * sizeof(float), stream);
    return rc;
  }
  if (!gy || !x || !w || !mean || !rstd || !dx) return AAR_EINVAL;
  const bool vec = ln_bwd_vec(gy, x, w, dx, workspace, cols) && (!addend || aligned16(addend));
  const RowPlan p = plan_rows(cols, vec);
  bool short_grid = false;
  const int parts = ln_bwd_parts_for(rows, p, &short_grid);
  const size_t need = (size_t)parts * 2 * (size_t)cols * sizeof(float);
  if (!workspace || workspace_bytes < need) return AAR_EWORKSPACE;
  float* part = static_cast<float*>(workspace);
  int rc;
  if (p.nv == 0) {
    if (!wide_grid_ok(rows)) return AAR_EUNSUPPORTED;
    layernorm_bwd_wide_kernel<<<dim3((unsigned)rows), dim3(kThreads), 0, st>>>(gy, x, w, mean, rstd,
                                                                                addend, dx, cols);
    rc = launch_status();
    if (rc != AAR_OK) return rc;
    layernorm_bwd_wide_cols_kernel<<<dim3((unsigned)ceil_div(cols, kThreads), (unsigned)parts),
                                     dim3(kThreads), 0, st>>>(gy, x, mean, rstd, part, rows, cols);
  } else {
    if (addend && short_grid) {
#define L(NV, W, V)                                                                                  \
  layernorm_bwd_kernel<NV, W, V, ln_bwd_waves(NV, W), ln_bwd_prefetch(NV, W), true, true>                \
      <<<dim3(parts), dim3(ln_bwd_waves(NV, W) * kWave), 0, st>>>(gy, x, w, mean, rstd, addend, dx, part, \
                                                                 rows, (int)cols)
      AAR_ROW_DISPATCH(p, L);
#undef L
    } else if (addend) {
#define L(NV, W, V)                                                                                  \
  layernorm_bwd_kernel<NV, W, V, ln_bwd_waves(NV, W), ln_bwd_prefetch(NV, W), true>                      \
      <<<dim3(parts), dim3(ln_bwd_waves(NV, W) * kWave), 0, st>>>(gy, x, w, mean, rstd, addend, dx, part, \
                                                                 rows, (int)cols)
      AAR_ROW_DISPATCH(p, L);
#undef L
    } else {
#define L(NV, W, V)                                                                                  \
  layernorm_bwd_kernel<NV, W, V, ln_bwd_waves(NV, W), ln_bwd_prefetch(NV, W), false>                     \
      <<<dim3(parts), dim3(ln_bwd_waves(NV, W) * kWave), 0, st>>>(gy, x, w, mean, rstd, nullptr, dx, part, \
                                                                 rows, (int)cols)
      AAR_ROW_DISPATCH(p, L);
#undef L
    }
  }
  rc = launch_status();
  if (rc != AAR_OK) return rc;
  // Reduce grid: one workgroup per V columns of the 2C, at most 2^16.
  const int64_t red_blocks = 2 * cols / ((cols % 4 == 0 && aligned16(part)) ? 4 : 1);
  const unsigned red_grid = (unsigned)std::min<int64_t>(red_blocks, int64_t(1) << 16);
  if (cols % 4 == 0 && aligned16(part)) {
    layernorm_bwd_reduce_kernel<4><<<dim3(red_grid), dim3(kRedThreads), 0, st>>>(part, dw, db, parts, (int)cols);
  } else {
    layernorm_bwd_reduce_kernel<1><<<dim3(red_grid), dim3(kRedThreads), 0, st>>>(part, dw, db, parts, (int)cols);
  }
  return launch_status();
}

// Static scratch of the no-allocation entry point: one copy per GPU, held
// until the process ends.  Host code never passes `scratch` itself to a
// kernel (on the host the name is a stand-in, not a device address); it uses
// the per-device address hipGetSymbolAddress returns.
constexpr size_t kLnBwdScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kLnBwdScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch, looked up once per device
// with that device current.
int scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return AAR_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return static_cast<int>(e);
    if (!p) return AAR_EUNSUPPORTED;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return AAR_OK;
}

// Any 16-byte aligned address: stands for the scratch buffer in the
// alignment test of the plan (the buffer itself is 256-byte aligned).
inline const void* scratch_align_probe() { return reinterpret_cast<const void*>(uintptr_t(256)); }

}  // namespace
}  // namespace aar

extern "C" int aar_layernorm_bwd_f32(const float* gy, const float* x, const float* w,
                                     const float* mean, const float* rstd, float* dx, float* dw,
                                     float* db, int64_t rows, int64_t cols, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  return layernorm_bwd_run(gy, x, w, mean, rstd, nullptr, dx, dw, db, rows, cols, workspace, workspace_bytes,
                           stream);
}

extern "C" int aar_layernorm_bwd_acc_f32(const float* gy, const float* x, const float* w, const float* mean,
                                         const float* rstd, const float* dx_addend, float* dx, float* dw,
                                         float* db, int64_t rows, int64_t cols, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  if (rows > 0 && !dx_addend) return AAR_EINVAL;
  return layernorm_bwd_run(gy, x, w, mean, rstd, dx_addend, dx, dw, db, rows, cols, workspace, workspace_bytes,
                           stream);
}

extern "C" size_t aar_layernorm_bwd_noalloc_max_bytes(void) { return kLnBwdScratchBytes; }

extern "C" int aar_layernorm_bwd_noalloc_f32(const float* gy, const float* x, const float* w,
                                             const float* mean, const float* rstd, float* dx, float* dw,
                                             float* db, int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols <= 0 || cols > INT32_MAX) return AAR_EINVAL;
  // The buffer is 256-byte aligned, so the plan follows the operands' alignment.
  if (rows > 0 && ln_bwd_need_bytes(rows, cols, ln_bwd_vec(gy, x, w, dx, scratch_align_probe(), cols)) >
                      kLnBwdScratchBytes) {
    return AAR_ESCRATCH;
  }
  void* ws = nullptr;
  const int rc = scratch_ptr(&ws);
  if (rc != AAR_OK) return rc;
  return layernorm_bwd_run(gy, x, w, mean, rstd, nullptr, dx, dw, db, rows, cols, ws, kLnBwdScratchBytes, stream);
}
