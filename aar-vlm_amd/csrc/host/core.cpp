// Tensor, Storage, allocators and device plumbing of aargrad._core.
// Reference behaviour: cppsrc/core/tensor.cpp:1-141 (factories, to(), grad slot),
// cppsrc/core/cuda_allocator.cpp:8-22, cppsrc/core/cuda_copy.cu:11-37,
// cppsrc/core/cuda_check.hpp:8-17 (error taxonomy).
//
// The device allocator differs from the reference's bare cudaMalloc/cudaFree:
// it caches freed blocks by rounded size.  All device work is ordered on one
// stream, so a block released by the host can be handed to the next op at
// once; host-visible reads synchronise through device->host copies.
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <unordered_map>

#include "aar_hip.h"
#include "tensor.hpp"

namespace aar {

size_t dtype_size(DType dtype) {
  switch (dtype) {
    case DType::Fp32: return 4;
    case DType::Fp16: return 2;
    case DType::Bf16: return 2;
    case DType::Int64: return 8;
  }
  throw std::runtime_error("Unsupported dtype");
}

const char* dtype_name(DType dtype) {
  switch (dtype) {
    case DType::Fp32: return "Fp32";
    case DType::Fp16: return "Fp16";
    case DType::Bf16: return "Bf16";
    case DType::Int64: return "Int64";
  }
  return "?";
}

void check_status(int status, const char* what) {
  if (status == AAR_OK) return;
  std::string msg = std::string(what) + ": " + aar_error_string(status);
  if (status == AAR_EINVAL || status == AAR_EUNSUPPORTED) throw std::invalid_argument(msg);
  if (status == AAR_ENOMEM) throw std::bad_alloc();
  throw std::runtime_error("HIP error: " + msg);
}

void* current_stream() { return nullptr; }

[[noreturn]] void throw_cpu_compute(const char* op) {
  throw std::runtime_error(std::string(op) +
                           ": this aargrad build computes on the MI355X GPU only; move the "
                           "tensors to Device.CUDA");
}

[[noreturn]] void throw_not_on_device(const char* op) {
  throw std::runtime_error(std::string(op) + ": not provided on Device.CUDA by this aargrad build");
}

// ---------------------------------------------------------------- allocators

namespace {

class CpuAllocator final : public Allocator {
 public:
  void* alloc(size_t bytes) override {
    if (bytes == 0) return nullptr;
    const size_t rounded = (bytes + 63) / 64 * 64;
    void* p = std::aligned_alloc(64, rounded);
    if (!p) throw std::bad_alloc();
    return p;
  }
  void free(void* ptr) noexcept override { std::free(ptr); }
  Device device() const noexcept override { return Device::CPU; }
};

class DeviceCachingAllocator final : public Allocator {
 public:
  void* alloc(size_t bytes) override {
    if (bytes == 0) return nullptr;
    const size_t r = round(bytes);
    {
      std::lock_guard<std::mutex> lock(mu_);
      auto it = free_.find(r);
      if (it != free_.end() && !it->second.empty()) {
        void* p = it->second.back();
        it->second.pop_back();
        live_[p] = r;
        cached_ -= r;
        in_use_ += r;
        return p;
      }
    }
    void* p = nullptr;
    int rc = aar_malloc(&p, r);
    if (rc == AAR_ENOMEM) {
      release_cached();
      rc = aar_malloc(&p, r);
    }
    if (rc == AAR_ENOMEM) throw std::bad_alloc();
    check_status(rc, "device allocation");
    std::lock_guard<std::mutex> lock(mu_);
    live_[p] = r;
    in_use_ += r;
    return p;
  }

  void free(void* ptr) noexcept override {
    if (!ptr) return;
    std::lock_guard<std::mutex> lock(mu_);
    auto it = live_.find(ptr);
    if (it == live_.end()) return;
    const size_t r = it->second;
    live_.erase(it);
    free_[r].push_back(ptr);
    in_use_ -= r;
    cached_ += r;
  }

  Device device() const noexcept override { return Device::CUDA; }

  void release_cached() {
    std::lock_guard<std::mutex> lock(mu_);
    for (auto& kv : free_)
      for (void* p : kv.second) aar_free(p);
    free_.clear();
    cached_ = 0;
  }

  size_t in_use() {
    std::lock_guard<std::mutex> lock(mu_);
    return in_use_;
  }
  size_t cached() {
    std::lock_guard<std::mutex> lock(mu_);
    return cached_;
  }

 private:
  // 512-byte granularity below 1 MiB, 2 MiB above.
  static size_t round(size_t n) {
    if (n <= (1u << 20)) return (n + 511) / 512 * 512;
    const size_t g = 2u << 20;
    return (n + g - 1) / g * g;
  }

  std::mutex mu_;
  std::unordered_map<size_t, std::vector<void*>> free_;
  std::unordered_map<void*, size_t> live_;
  size_t in_use_ = 0;
  size_t cached_ = 0;
};

// Leaked on purpose: device memory must not be released from a static
// destructor that may run after the HIP runtime has been torn down.
DeviceCachingAllocator* g_device_alloc = new DeviceCachingAllocator();

}  // namespace

Allocator* cpu_allocator() {
  static CpuAllocator inst;
  return &inst;
}

Allocator* device_allocator() { return g_device_alloc; }
void device_empty_cache() { g_device_alloc->release_cached(); }
size_t device_bytes_in_use() { return g_device_alloc->in_use(); }
size_t device_bytes_cached() { return g_device_alloc->cached(); }

namespace {
Allocator* allocator_for(Device device) {
  return device == Device::CPU ? cpu_allocator() : device_allocator();
}
}  // namespace

Storage::Storage(size_t nbytes, Allocator* allocator) : nbytes_(nbytes), allocator_(allocator) {
  data_ = allocator_->alloc(nbytes);
}

Storage::~Storage() {
  if (data_) allocator_->free(data_);
}

Workspace::Workspace(size_t bytes) {
  if (bytes) storage = std::make_shared<Storage>(bytes, device_allocator());
}

// --------------------------------------------------------------- transfers

namespace {
std::mutex g_err_mu;
int* g_err_words = nullptr;  // kErrSlots ints on the device, zeroed once
}  // namespace

int* device_error_word(DeviceErrorSlot slot) {
  std::lock_guard<std::mutex> lock(g_err_mu);
  if (!g_err_words) {
    void* p = device_allocator()->alloc(256);  // held for the life of the process
    check_status(aar_memset_zero(p, 256, current_stream()), "device error word");
    g_err_words = static_cast<int*>(p);
  }
  return g_err_words + slot;
}

void check_device_errors() {
  int* words;
  {
    std::lock_guard<std::mutex> lock(g_err_mu);
    words = g_err_words;
  }
  if (!words) return;
  int host[kErrSlots] = {};
  check_status(aar_memcpy(host, words, sizeof(host), 2, current_stream()), "device error word");
  if (host[kErrEmbeddingId] || host[kErrCrossEntropyTarget] || host[kErrTokenWindow]) {
    check_status(aar_memset_zero(words, sizeof(host), current_stream()), "device error word");
    if (host[kErrEmbeddingId]) throw std::out_of_range("embedding: id out of range [0, vocab_size)");
    if (host[kErrCrossEntropyTarget]) throw std::out_of_range("cross_entropy: target out of range [0, V)");
    throw std::out_of_range("token_windows: window start out of range");
  }
}

void copy_bytes(void* dst, Device dst_device, const void* src, Device src_device, size_t nbytes) {
  if (nbytes == 0) return;
  if (dst_device == Device::CPU && src_device == Device::CPU) {
    std::memcpy(dst, src, nbytes);
    return;
  }
  int kind = 3;
  if (src_device == Device::CPU) kind = 1;
  else if (dst_device == Device::CPU) kind = 2;
  check_status(aar_memcpy(dst, src, nbytes, kind, current_stream()), "copy_bytes");
  if (kind == 2) check_device_errors();
}

void zero_bytes(void* p, Device device, size_t nbytes) {
  if (nbytes == 0) return;
  if (device == Device::CPU) {
    std::memset(p, 0, nbytes);
    return;
  }
  check_status(aar_memset_zero(p, nbytes, current_stream()), "zero_bytes");
}

void device_synchronize() {
  check_status(aar_synchronize(), "cuda_synchronize");
  check_device_errors();
}

// ------------------------------------------------------------------ tensor

std::vector<int64_t> compute_contiguous_strides(const std::vector<int64_t>& shape) {
  std::vector<int64_t> strides(shape.size());
  int64_t s = 1;
  for (int i = static_cast<int>(shape.size()) - 1; i >= 0; --i) {
    strides[i] = s;
    s *= shape[i];
  }
  return strides;
}

Tensor::Tensor(std::vector<int64_t> shape_, DType dtype_, Device device_)
    : shape(std::move(shape_)),
      strides(compute_contiguous_strides(shape)),
      storage_offset(0),
      dtype(dtype_),
      device(device_) {}

size_t Tensor::numel() const {
  size_t n = 1;
  for (int64_t d : shape) n *= static_cast<size_t>(d);
  return n;
}

size_t Tensor::nbytes() const { return numel() * dtype_size(dtype); }

bool Tensor::is_contiguous() const {
  if (storage_offset != 0) return false;
  if (strides.size() != shape.size()) return false;
  const auto expected = compute_contiguous_strides(shape);
  for (size_t i = 0; i < strides.size(); ++i)
    if (strides[i] != expected[i]) return false;
  return true;
}

Tensor Tensor::empty(std::vector<int64_t> shape, DType dtype, Device device) {
  for (int64_t d : shape)
    if (d < 0) throw std::invalid_argument("Tensor: negative dimension");
  Tensor t(std::move(shape), dtype, device);
  if (t.numel() > 0) t.storage = std::make_shared<Storage>(t.nbytes(), allocator_for(device));
  return t;
}

Tensor Tensor::zeros(std::vector<int64_t> shape, DType dtype, Device device) {
  Tensor t = empty(std::move(shape), dtype, device);
  if (t.storage) zero_bytes(t.storage->data(), device, t.storage->nbytes());
  return t;
}

Tensor Tensor::ones(std::vector<int64_t> shape, DType dtype, Device device) {
  // fp32 on the device: a fill kernel on the current stream.  The upload the
  // other dtypes take (a host fill, as the reference does, tensor.cpp:78-87)
  // synchronizes the stream; for backward()'s seed gradient that drained the
  // queue between a training step's forward and backward.
  if (device == Device::CUDA && dtype == DType::Fp32) {
    Tensor t = empty(std::move(shape), dtype, device);
    if (t.storage) {
      check_status(aar_fill_f32(static_cast<float*>(t.storage->data()), 1.0f, static_cast<int64_t>(t.numel()),
                                current_stream()),
                   "ones");
    }
    return t;
  }
  Tensor cpu = empty(shape, dtype, Device::CPU);
  if (cpu.storage) {
    const size_t n = cpu.numel();
    switch (dtype) {
      case DType::Fp32: {
        float* p = static_cast<float*>(cpu.storage->data());
        for (size_t i = 0; i < n; ++i) p[i] = 1.0f;
        break;
      }
      case DType::Int64: {
        int64_t* p = static_cast<int64_t*>(cpu.storage->data());
        for (size_t i = 0; i < n; ++i) p[i] = 1;
        break;
      }
      case DType::Fp16: {
        uint16_t* p = static_cast<uint16_t*>(cpu.storage->data());
        for (size_t i = 0; i < n; ++i) p[i] = 0x3C00;
        break;
      }
      case DType::Bf16: {
        uint16_t* p = static_cast<uint16_t*>(cpu.storage->data());
        for (size_t i = 0; i < n; ++i) p[i] = 0x3F80;
        break;
      }
    }
  }
  if (device == Device::CPU) return cpu;
  return cpu.to(device);
}

Tensor Tensor::to(Device target) const {
  if (target == device) return *this;
  if (!is_contiguous()) {
    throw std::runtime_error("Tensor::to: source must be contiguous; call contiguous() first");
  }
  Tensor out = Tensor::empty(shape, dtype, target);
  if (out.storage) copy_bytes(out.storage->data(), target, data(), device, nbytes());
  return out;
}

void* Tensor::data() {
  if (!storage) return nullptr;
  return static_cast<char*>(storage->data()) + static_cast<size_t>(storage_offset) * dtype_size(dtype);
}

const void* Tensor::data() const {
  if (!storage) return nullptr;
  return static_cast<const char*>(storage->data()) +
         static_cast<size_t>(storage_offset) * dtype_size(dtype);
}

Tensor& Tensor::set_requires_grad(bool req) {
  if (req && !is_leaf()) throw std::runtime_error("set_requires_grad: cannot set on non-leaf tensor");
  requires_grad = req;
  if (req && !grad_slot) grad_slot = std::make_shared<std::shared_ptr<Tensor>>();
  return *this;
}

std::shared_ptr<Tensor> Tensor::grad() const { return grad_slot ? *grad_slot : nullptr; }

void Tensor::zero_grad() {
  if (grad_slot) *grad_slot = nullptr;
}

void Tensor::backward() {
  if (numel() != 1) {
    throw std::runtime_error("backward(): grad implicitly created only for scalar outputs");
  }
  Tensor g = Tensor::ones(shape, dtype, device);
  run_backward(*this, g);
}

void Tensor::backward(const Tensor& grad_output) {
  if (grad_output.shape != shape) throw std::runtime_error("backward(grad_output): shape mismatch");
  if (grad_output.device != device) throw std::runtime_error("backward(grad_output): device mismatch");
  run_backward(*this, grad_output);
}

void Function::record_input(const Tensor& t) {
  Input edge;
  edge.needs_grad = t.requires_grad;
  if (t.requires_grad) {
    if (t.grad_fn) edge.grad_fn = t.grad_fn;
    else edge.leaf = t;
  }
  inputs.push_back(std::move(edge));
}

}  // namespace aar
