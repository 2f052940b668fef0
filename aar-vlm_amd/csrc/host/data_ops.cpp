// Token-window batches on the device (the data side of the training loop).
// Semantics of the reference's host pipeline:
//   TokenWindowDataset.__getitem__ / default_collate   python/shakespeare/scripts/data.py:38-53
//   to_device_batch                                    python/shakespeare/scripts/train.py:99-102
#include <vector>

#include "aar_hip.h"
#include "ops.hpp"

namespace aar {

std::tuple<Tensor, Tensor> token_windows(const Tensor& tokens, const Tensor& starts, int64_t seq_len) {
  if (tokens.dtype != DType::Int64 || starts.dtype != DType::Int64) {
    throw std::invalid_argument("token_windows: tokens and starts must be Int64");
  }
  if (tokens.shape.size() != 1 || starts.shape.size() != 1) {
    throw std::invalid_argument("token_windows: tokens and starts must be 1D");
  }
  if (seq_len <= 0) throw std::invalid_argument("token_windows: seq_len must be positive");
  if (tokens.device == Device::CPU) throw_cpu_compute("token_windows");
  if (!tokens.is_contiguous()) throw std::invalid_argument("token_windows: tokens must be contiguous");
  const int64_t n = tokens.shape[0], batch = starts.shape[0];
  Tensor dev_starts = starts;
  if (starts.device == Device::CPU) {
    // Starts drawn on the host are checked here, as the reference's slicing
    // would fail on the host; device starts are checked by the kernel.
    std::vector<int64_t> host(batch);
    const int64_t* src = static_cast<const int64_t*>(starts.data());
    const int64_t st = starts.strides.empty() ? 1 : starts.strides[0];
    for (int64_t b = 0; b < batch; ++b) {
      host[b] = src[b * st];
      if (host[b] < 0 || host[b] > n - seq_len - 1) {
        throw std::out_of_range("token_windows: window start out of range");
      }
    }
    dev_starts = Tensor::empty({batch}, DType::Int64, Device::CUDA);
    copy_bytes(dev_starts.data(), Device::CUDA, host.data(), Device::CPU, host.size() * sizeof(int64_t));
  } else if (!starts.is_contiguous()) {
    throw std::invalid_argument("token_windows: starts must be contiguous");
  }
  Tensor x = Tensor::empty({batch, seq_len}, DType::Int64, Device::CUDA);
  Tensor y = Tensor::empty({batch, seq_len}, DType::Int64, Device::CUDA);
  check_status(aar_token_windows_i64(static_cast<const int64_t*>(tokens.data()), n,
                                     static_cast<const int64_t*>(dev_starts.data()), batch, seq_len,
                                     static_cast<int64_t*>(x.data()), static_cast<int64_t*>(y.data()),
                                     device_error_word(kErrTokenWindow), current_stream()),
               "token_windows");
  return {x, y};
}

}  // namespace aar
