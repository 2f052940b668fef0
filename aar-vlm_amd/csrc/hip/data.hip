// Token-window batches for the language-model training loop, gathered on the
// device from a token stream resident in HBM.  Reference semantics:
//   TokenWindowDataset.__getitem__, default_collate
//                         python/shakespeare/scripts/data.py:38-53
//   to_device_batch       python/shakespeare/scripts/train.py:99-102
// x[b][t] = tokens[starts[b] + t], y[b][t] = tokens[starts[b] + t + 1].
// The stream is int64 little-endian on disk (prepare.py:44-47), which is the
// device's own layout, so a token file uploads once without conversion and a
// training step moves 16*B*T bytes of (x, y) plus B window starts, instead of
// a host-side gather, collate and copy per batch.
#include <hip/hip_runtime.h>

#include "common.hpp"

namespace aar {
namespace {

// One thread per (b, t); neighbouring threads read neighbouring tokens, and
// the y read of one thread is the x read of the next (an L2 hit).  A window
// that does not fit the stream writes zeros and raises *err; nothing outside
// the stream is read.
__global__ void __launch_bounds__(256)
token_windows_kernel(const int64_t* __restrict__ tok, int64_t n_tok, const int64_t* __restrict__ starts,
                     int64_t T, int64_t total, int64_t* __restrict__ x, int64_t* __restrict__ y,
                     int* __restrict__ err) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t b = i / T, t = i - b * T;
    const int64_t s = starts[b];
    if (s >= 0 && s <= n_tok - T - 1) {
      x[i] = tok[s + t];
      y[i] = tok[s + t + 1];
    } else {
      x[i] = 0;
      y[i] = 0;
      if (t == 0 && err) *err = 1;
    }
  }
}

}  // namespace
}  // namespace aar

using namespace aar;

extern "C" int aar_token_windows_i64(const int64_t* tokens, int64_t n_tokens, const int64_t* starts,
                                     int64_t batch, int64_t seq_len, int64_t* x, int64_t* y, int* err,
                                     void* stream) {
  if (n_tokens < 0 || batch < 0 || seq_len <= 0) return AAR_EINVAL;
  if (batch == 0) return AAR_OK;
  if (!tokens || !starts || !x || !y) return AAR_EINVAL;
  const int64_t total = batch * seq_len;
  int64_t g = (total + 255) / 256;
  if (g > (int64_t(1) << 20)) g = int64_t(1) << 20;
  token_windows_kernel<<<dim3((unsigned)g), dim3(256), 0, as_stream(stream)>>>(tokens, n_tokens, starts, seq_len,
                                                                              total, x, y, err);
  return launch_status();
}
