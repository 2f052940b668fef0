// Host-side value types of aargrad._core for the MI355X backend: dtype and
// device enums, storage with an owning allocator, the strided Tensor, and the
// autograd Function tape.  Semantics follow the reference core:
//   Tensor / compute_contiguous_strides   cppsrc/core/tensor.hpp:14-48, tensor.cpp:18-141
//   Storage / Allocator                   cppsrc/core/storage.hpp:9-29, allocator.hpp:8-23
//   Function / record_input               cppsrc/autograd/function.hpp:9-24, function.cpp:4-15
// Device memory comes from a caching allocator over the C ABI (aar_malloc);
// every device computation is a call into include/aar_hip.h.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace aar {

enum class DType : uint8_t { Fp32, Fp16, Bf16, Int64 };
// CUDA keeps the reference's enum name (scripts use ag.Device.CUDA); here it
// denotes the HIP GPU.
enum class Device : uint8_t { CPU, CUDA };

size_t dtype_size(DType dtype);
const char* dtype_name(DType dtype);

class Allocator {
 public:
  virtual ~Allocator() = default;
  virtual void* alloc(size_t bytes) = 0;
  virtual void free(void* ptr) noexcept = 0;
  virtual Device device() const noexcept = 0;
};

Allocator* cpu_allocator();
Allocator* device_allocator();

// Release every cached (currently unused) device block back to the driver.
void device_empty_cache();
// Bytes currently handed out / held in the cache by the device allocator.
size_t device_bytes_in_use();
size_t device_bytes_cached();

class Storage {
 public:
  Storage(size_t nbytes, Allocator* allocator);
  ~Storage();
  Storage(const Storage&) = delete;
  Storage& operator=(const Storage&) = delete;

  void* data() noexcept { return data_; }
  const void* data() const noexcept { return data_; }
  size_t nbytes() const noexcept { return nbytes_; }

 private:
  void* data_ = nullptr;
  size_t nbytes_ = 0;
  Allocator* allocator_ = nullptr;
};

class Function;

struct Tensor {
  std::vector<int64_t> shape;
  std::vector<int64_t> strides;
  int64_t storage_offset = 0;
  DType dtype = DType::Fp32;
  Device device = Device::CPU;
  std::shared_ptr<Storage> storage;

  bool requires_grad = false;
  std::shared_ptr<Function> grad_fn;
  std::shared_ptr<std::shared_ptr<Tensor>> grad_slot;

  Tensor() = default;
  Tensor(std::vector<int64_t> shape, DType dtype, Device device = Device::CPU);

  static Tensor empty(std::vector<int64_t> shape, DType dtype, Device device = Device::CPU);
  static Tensor zeros(std::vector<int64_t> shape, DType dtype, Device device = Device::CPU);
  static Tensor ones(std::vector<int64_t> shape, DType dtype, Device device = Device::CPU);

  size_t numel() const;
  size_t nbytes() const;
  bool is_contiguous() const;

  void* data();
  const void* data() const;

  Tensor to(Device target) const;

  Tensor& set_requires_grad(bool req);
  bool is_leaf() const { return grad_fn == nullptr; }
  std::shared_ptr<Tensor> grad() const;
  void zero_grad();
  void backward();
  void backward(const Tensor& grad_output);
};

std::vector<int64_t> compute_contiguous_strides(const std::vector<int64_t>& shape);

class Function {
 public:
  struct Input {
    std::shared_ptr<Function> grad_fn;
    Tensor leaf;
    bool needs_grad = false;
  };
  std::vector<Input> inputs;

  virtual ~Function() = default;
  virtual std::vector<Tensor> backward(const Tensor& grad_output) = 0;
  virtual const char* name() const { return "Function"; }
  void record_input(const Tensor& t);

  // Gradient fan-in folded into the producing kernel.  When the engine holds
  // a gradient for input k already (`held[k]`, null when none) and the
  // function fuses fan-ins (`fuses_fan_in`), it calls backward_into, which
  // may return held[k] + its own gradient for input k in one pass and set
  // summed[k]: the engine then takes that tensor as the new held gradient in
  // place of add_grads(held, new).  The sum must be that fp32 addition bit for
  // bit.  The default fuses nothing.
  virtual bool fuses_fan_in() const { return false; }
  virtual std::vector<Tensor> backward_into(const Tensor& grad_output, const std::vector<const Tensor*>& held,
                                            std::vector<bool>& summed) {
    (void)held;
    summed.assign(inputs.size(), false);
    return backward(grad_output);
  }
};

void run_backward(const Tensor& root, const Tensor& grad_output);

// ----------------------------------------------------------- device plumbing

// Translate a C-ABI status into the reference's exception taxonomy:
// invalid argument -> std::invalid_argument, out of memory -> std::bad_alloc,
// anything else -> std::runtime_error("HIP error: ...").
void check_status(int status, const char* what);

// The stream every op of this module is ordered on (the null stream).
void* current_stream();

void copy_bytes(void* dst, Device dst_device, const void* src, Device src_device, size_t nbytes);

// Deferred device-side errors.  Kernels that cannot throw (an embedding id,
// a cross-entropy target or a token window out of range) set a word here; the host raises
// std::out_of_range at its next synchronisation point (a device-to-host copy
// or cuda_synchronize), the way the reference raises on its CPU path.
enum DeviceErrorSlot { kErrEmbeddingId = 0, kErrCrossEntropyTarget = 1, kErrTokenWindow = 2, kErrSlots = 3 };
int* device_error_word(DeviceErrorSlot slot);
void check_device_errors();
void zero_bytes(void* p, Device device, size_t nbytes);
void device_synchronize();

// Device scratch for one call, returned to the cache when the handle dies.
struct Workspace {
  std::shared_ptr<Storage> storage;
  explicit Workspace(size_t bytes);
  void* data() const { return storage ? storage->data() : nullptr; }
  size_t bytes() const { return storage ? storage->nbytes() : 0; }
};

// Errors for compute requested on the host: this build computes on the GPU only.
[[noreturn]] void throw_cpu_compute(const char* op);
[[noreturn]] void throw_not_on_device(const char* op);

// ------------------------------------------------------------ shape helpers
Tensor make_view(const Tensor& src, std::vector<int64_t> shape, std::vector<int64_t> strides,
                 int64_t storage_offset);
void copy_strided_to_contiguous(const Tensor& src, Tensor& dst);

}  // namespace aar
