// Device runtime behind the C ABI: allocation, copies, zero-fill, sync,
// events, device properties and error text.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "common.hpp"

namespace aar {

namespace {

// Grid-stride zero fill, 16 bytes per lane where alignment allows.
__global__ void fill_zero_kernel(unsigned char* __restrict__ p, size_t bytes) {
  const size_t tid = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const uintptr_t base = reinterpret_cast<uintptr_t>(p);
  const size_t head = (16 - (base & 15)) & 15;
  const size_t lead = head < bytes ? head : bytes;
  if (tid < lead) p[tid] = 0;
  const size_t body = (bytes - lead) / 16;
  uint4* q = reinterpret_cast<uint4*>(p + lead);
  for (size_t i = tid; i < body; i += stride) q[i] = make_uint4(0, 0, 0, 0);
  const size_t tail_start = lead + body * 16;
  for (size_t i = tail_start + tid; i < bytes; i += stride) p[i] = 0;
}

std::mutex g_cu_mutex;
std::vector<int> g_cu_counts;

}  // namespace

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lock(g_cu_mutex);
  if ((int)g_cu_counts.size() <= dev) g_cu_counts.resize(dev + 1, 0);
  if (g_cu_counts[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_cu_counts[dev] = n;
  }
  return g_cu_counts[dev];
}

}  // namespace aar

using namespace aar;

extern "C" {

const char* aar_error_string(int status) {
  switch (status) {
    case AAR_OK: return "ok";
    case AAR_EINVAL: return "aar: invalid argument";
    case AAR_EWORKSPACE: return "aar: workspace missing or too small";
    case AAR_EUNSUPPORTED: return "aar: shape not supported by the gfx950 kernels";
    case AAR_ENOMEM: return "aar: out of device memory";
    case AAR_ESCRATCH: return "aar: problem needs more than the no-allocation entry point's static scratch";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "aar: unknown error";
}

int aar_device_count(int* count) {
  if (!count) return AAR_EINVAL;
  *count = 0;
  hipError_t e = hipGetDeviceCount(count);
  if (e != hipSuccess) {
    *count = 0;
    return static_cast<int>(e);
  }
  return AAR_OK;
}

int aar_device_info(int* cu_count, int* clock_khz, int* lds_bytes_per_cu, char* arch_name,
                    int arch_name_len) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (cu_count) *cu_count = prop.multiProcessorCount;
  if (clock_khz) *clock_khz = prop.clockRate;
  if (lds_bytes_per_cu) *lds_bytes_per_cu = static_cast<int>(prop.maxSharedMemoryPerMultiProcessor);
  if (arch_name && arch_name_len > 0) {
    strncpy(arch_name, prop.gcnArchName, arch_name_len - 1);
    arch_name[arch_name_len - 1] = '\0';
  }
  return AAR_OK;
}

int aar_malloc(void** ptr, size_t bytes) {
  if (!ptr) return AAR_EINVAL;
  *ptr = nullptr;
  if (bytes == 0) return AAR_OK;
  hipError_t e = hipMalloc(ptr, bytes);
  if (e != hipSuccess) {
    *ptr = nullptr;
    (void)hipGetLastError();
    return e == hipErrorOutOfMemory ? AAR_ENOMEM : static_cast<int>(e);
  }
  return AAR_OK;
}

int aar_free(void* ptr) {
  if (!ptr) return AAR_OK;
  hipError_t e = hipFree(ptr);
  return e == hipSuccess ? AAR_OK : static_cast<int>(e);
}

int aar_memcpy(void* dst, const void* src, size_t bytes, int kind, void* stream) {
  if (bytes == 0) return AAR_OK;
  if (!dst || !src) return AAR_EINVAL;
  hipError_t e;
  switch (kind) {
    case 1:
      e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream));
      if (e == hipSuccess) e = hipStreamSynchronize(as_stream(stream));
      break;
    case 2:
      e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream));
      if (e == hipSuccess) e = hipStreamSynchronize(as_stream(stream));
      break;
    case 3:
      e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream));
      break;
    default:
      return AAR_EINVAL;
  }
  return e == hipSuccess ? AAR_OK : static_cast<int>(e);
}

int aar_memset_zero(void* ptr, size_t bytes, void* stream) {
  if (bytes == 0) return AAR_OK;
  if (!ptr) return AAR_EINVAL;
  const size_t work = (bytes + 15) / 16;
  size_t blocks = (work + 255) / 256;
  const size_t cap = static_cast<size_t>(device_cu_count()) * 8;
  if (blocks > cap) blocks = cap;
  if (blocks == 0) blocks = 1;
  fill_zero_kernel<<<dim3((unsigned)blocks), dim3(256), 0, as_stream(stream)>>>(
      static_cast<unsigned char*>(ptr), bytes);
  return launch_status();
}

int aar_synchronize(void) {
  hipError_t e = hipDeviceSynchronize();
  return e == hipSuccess ? AAR_OK : static_cast<int>(e);
}

int aar_stream_synchronize(void* stream) {
  hipError_t e = hipStreamSynchronize(as_stream(stream));
  return e == hipSuccess ? AAR_OK : static_cast<int>(e);
}

int aar_event_create(void** event) {
  if (!event) return AAR_EINVAL;
  hipEvent_t ev = nullptr;
  hipError_t e = hipEventCreate(&ev);
  *event = ev;
  return e == hipSuccess ? AAR_OK : static_cast<int>(e);
}

int aar_event_destroy(void* event) {
  if (!event) return AAR_OK;
  hipError_t e = hipEventDestroy(reinterpret_cast<hipEvent_t>(event));
  return e == hipSuccess ? AAR_OK : static_cast<int>(e);
}

int aar_event_record(void* event, void* stream) {
  if (!event) return AAR_EINVAL;
  hipError_t e = hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_stream(stream));
  return e == hipSuccess ? AAR_OK : static_cast<int>(e);
}

int aar_event_elapsed_ms(float* ms, void* start, void* stop) {
  if (!ms || !start || !stop) return AAR_EINVAL;
  hipError_t e = hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop));
  if (e != hipSuccess) return static_cast<int>(e);
  e = hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop));
  return e == hipSuccess ? AAR_OK : static_cast<int>(e);
}

}  // extern "C"
