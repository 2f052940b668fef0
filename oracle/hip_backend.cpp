// hip_backend.cpp -- the reference-side glue of the MI355X backend.
//
// The reference (AARONKANG04/aar-vlm, cppsrc/) reaches a device through a
// fixed set of C++ functions: the *_cuda entry points that its ops/*.cpp
// files declare and call when a tensor lives on Device::CUDA (for example
// matmul_cuda at cppsrc/ops/matmul.cpp:10-12, flash_attention_forward_cuda at
// cppsrc/ops/flash_attention.cpp:15-22), the device allocator
// (cppsrc/core/cuda_allocator.hpp:6-13) and the byte copies
// (cppsrc/core/cuda_copy.hpp:8-12).  A maintainer adopting libaar_hip.so adds
// this file as cppsrc/ops/hip_backend.cpp in place of every *.cu file and
// every *_cuda_stub.cpp: each entry point becomes one aar_* call of the
// plain-C ABI in include/aar_hip.h, with the same output shapes and the same
// exception types as the reference's CUDA files.
//
// In this repository the file is TEST INFRASTRUCTURE: oracle/Makefile
// compiles it against the reference's headers, together with the reference's
// CPU sources and ref_driver.cpp, into oracle/_ref/libaar_glue.so, linked
// with --no-undefined against libaar_hip.so.  It is never part of the
// package.
#include <cmath>
#include <cstring>
#include <limits>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "aar_hip.h"
#include "core/allocator.hpp"
#include "core/cuda_allocator.hpp"
#include "core/cuda_copy.hpp"
#include "core/tensor.hpp"

namespace vlm {
namespace {

// Status -> the exception the reference throws for the same condition.
void check(int s, const char* what) {
  if (s == AAR_OK) return;
  if (s == AAR_ENOMEM) throw std::bad_alloc();
  const std::string msg = std::string(what) + ": " + aar_error_string(s);
  if (s == AAR_EINVAL || s == AAR_EUNSUPPORTED) throw std::invalid_argument(msg);
  throw std::runtime_error("HIP error: " + msg);
}

const float* f(const Tensor& t) { return static_cast<const float*>(t.data()); }
float* f(Tensor& t) { return static_cast<float*>(t.data()); }
const int64_t* ids(const Tensor& t) { return static_cast<const int64_t*>(t.data()); }
int64_t n_of(const Tensor& t) { return static_cast<int64_t>(t.numel()); }
int64_t last(const Tensor& t) { return t.shape.empty() ? 1 : t.shape.back(); }
int64_t rows_of(const Tensor& t) {
  const int64_t c = last(t);
  return c ? n_of(t) / c : 0;
}

Tensor device_empty(std::vector<int64_t> shape) { return Tensor::empty(std::move(shape), DType::Fp32, Device::CUDA); }

// Device scratch of at least `bytes` (an empty tensor for 0 bytes).
Tensor scratch(size_t bytes) {
  return bytes ? device_empty({static_cast<int64_t>((bytes + 3) / 4)}) : Tensor();
}
void* ptr(Tensor& ws) { return ws.storage ? ws.data() : nullptr; }

// `t` itself when dense row-major, else a dense device copy.
Tensor dense(const Tensor& t) {
  if (t.is_contiguous()) return t;
  Tensor out = device_empty(t.shape);
  const std::vector<int64_t> cs = compute_contiguous_strides(t.shape);
  check(aar_strided_copy_f32(f(t), f(out), static_cast<int>(t.shape.size()), t.shape.data(), t.strides.data(),
                             cs.data(), nullptr),
        "contiguous");
  return out;
}

class HipAllocator final : public Allocator {
 public:
  void* alloc(size_t nbytes, size_t /*alignment*/) override {
    if (nbytes == 0) return nullptr;
    void* p = nullptr;
    check(aar_malloc(&p, nbytes), "alloc");
    return p;
  }
  void free(void* p) noexcept override {
    if (p) aar_free(p);
  }
  Device device() const noexcept override { return Device::CUDA; }
};

Tensor gemm(int op, const Tensor& a, const Tensor& b, int64_t M, int64_t N, int64_t K) {
  Tensor c = device_empty({M, N});
  if (M == 0 || N == 0) return c;
  const Tensor ad = dense(a), bd = dense(b);
  const size_t wsb = aar_gemm_f32_workspace_bytes(op, M, N, K);
  Tensor ws = scratch(wsb);
  check(aar_gemm_f32(op, M, N, K, f(ad), f(bd), f(c), ptr(ws), wsb, nullptr), "matmul");
  return c;
}

// Batched product over the leading dims of rank >= 3 operands.
Tensor batched(int op, const Tensor& a, const Tensor& b) {
  const size_t nd = a.shape.size();
  const int64_t r = a.shape[nd - 2], c = a.shape[nd - 1];
  const int64_t M = op == AAR_GEMM_TN ? c : r, K = op == AAR_GEMM_TN ? r : c;
  const int64_t N = op == AAR_GEMM_NT ? b.shape[nd - 2] : b.shape[nd - 1];
  std::vector<int64_t> shape(a.shape.begin(), a.shape.end() - 2);
  int64_t batch = 1;
  for (int64_t s : shape) batch *= s;
  shape.push_back(M);
  shape.push_back(N);
  Tensor out = device_empty(shape);
  if (batch == 0 || M == 0 || N == 0) return out;
  const Tensor ad = dense(a), bd = dense(b);
  const int64_t lda = c, ldb = b.shape[nd - 1];
  check(aar_gemm_f32_batched(op, batch, M, N, K, f(ad), lda, r * c, f(bd), ldb, b.shape[nd - 2] * ldb, f(out), N,
                             M * N, nullptr),
        "bmm");
  return out;
}

Tensor unary(int (*fn)(const float*, float*, int64_t, void*), const Tensor& x, const char* what) {
  Tensor out = device_empty(x.shape);
  if (n_of(x)) check(fn(f(x), f(out), n_of(x), nullptr), what);
  return out;
}

Tensor binary(int (*fn)(const float*, const float*, float*, int64_t, void*), const Tensor& a, const Tensor& b,
              const char* what) {
  Tensor out = device_empty(a.shape);
  if (n_of(a)) check(fn(f(a), f(b), f(out), n_of(a), nullptr), what);
  return out;
}

Tensor causal_mask(const Tensor& x, float fill) {
  Tensor out = device_empty(x.shape);
  const int64_t T = last(x);
  if (n_of(x)) check(aar_causal_mask_f32(f(x), f(out), n_of(x) / (T * T), T, fill, nullptr), "causal_mask");
  return out;
}

}  // namespace

// ------------------------------------------------------------ allocator, copies
Allocator* cuda_allocator() {
  static HipAllocator instance;
  return &instance;
}

void copy_bytes(void* dst, Device dst_device, const void* src, Device src_device, size_t nbytes) {
  if (nbytes == 0) return;
  if (dst_device == Device::CPU && src_device == Device::CPU) {
    std::memcpy(dst, src, nbytes);
    return;
  }
  const int kind = src_device == Device::CPU ? 1 : (dst_device == Device::CPU ? 2 : 3);
  check(aar_memcpy(dst, src, nbytes, kind, nullptr), "copy_bytes");
}

void zero_bytes(void* p, Device device, size_t nbytes) {
  if (nbytes == 0) return;
  if (device == Device::CPU) {
    std::memset(p, 0, nbytes);
    return;
  }
  check(aar_memset_zero(p, nbytes, nullptr), "zero_bytes");
}

// ------------------------------------------------------------ GEMM (cppsrc/ops/matmul.cpp:10-12)
Tensor matmul_cuda(const Tensor& a, const Tensor& b) {
  return gemm(AAR_GEMM_NN, a, b, a.shape[0], b.shape[1], a.shape[1]);
}
Tensor matmul_a_bt_cuda(const Tensor& a, const Tensor& b) {
  return gemm(AAR_GEMM_NT, a, b, a.shape[0], b.shape[0], a.shape[1]);
}
Tensor matmul_at_b_cuda(const Tensor& a, const Tensor& b) {
  return gemm(AAR_GEMM_TN, a, b, a.shape[1], b.shape[1], a.shape[0]);
}

// ------------------------------------------------------------ batched GEMM (cppsrc/ops/bmm.cpp:10-12)
Tensor bmm_cuda(const Tensor& a, const Tensor& b) { return batched(AAR_GEMM_NN, a, b); }
Tensor bmm_a_bt_cuda(const Tensor& a, const Tensor& b) { return batched(AAR_GEMM_NT, a, b); }
Tensor bmm_at_b_cuda(const Tensor& a, const Tensor& b) { return batched(AAR_GEMM_TN, a, b); }

// ------------------------------------------------------------ softmax (cppsrc/ops/softmax.cpp:11-12)
Tensor softmax_cuda(const Tensor& x) {
  Tensor y = device_empty(x.shape);
  if (n_of(x)) check(aar_softmax_fwd_f32(f(x), f(y), rows_of(x), last(x), nullptr), "softmax");
  return y;
}
Tensor softmax_backward_cuda(const Tensor& g, const Tensor& y) {
  Tensor dx = device_empty(g.shape);
  if (n_of(g)) check(aar_softmax_bwd_f32(f(g), f(y), f(dx), rows_of(g), last(g), nullptr), "softmax backward");
  return dx;
}

// ------------------------------------------------------------ layernorm (cppsrc/ops/layernorm.cpp:12-17)
Tensor layernorm_cuda(const Tensor& x, const Tensor& w, const Tensor& b, float eps) {
  Tensor y = device_empty(x.shape);
  if (n_of(x))
    check(aar_layernorm_fwd_f32(f(x), f(w), f(b), f(y), nullptr, nullptr, rows_of(x), last(x), eps, nullptr),
          "layernorm");
  return y;
}
void layernorm_with_stats_cuda(const Tensor& x, const Tensor& w, const Tensor& b, float eps, Tensor& y, Tensor& mean,
                               Tensor& rstd) {
  if (n_of(x))
    check(aar_layernorm_fwd_f32(f(x), f(w), f(b), f(y), f(mean), f(rstd), rows_of(x), last(x), eps, nullptr),
          "layernorm");
}
void layernorm_backward_cuda(const Tensor& gy, const Tensor& x, const Tensor& w, const Tensor& mean,
                             const Tensor& rstd, Tensor& dx, Tensor& dw, Tensor& db) {
  const int64_t R = rows_of(x), C = last(x);
  if (R == 0 || C == 0) return;
  const size_t wsb = aar_layernorm_bwd_workspace_bytes(R, C);
  Tensor ws = scratch(wsb);
  check(aar_layernorm_bwd_f32(f(gy), f(x), f(w), f(mean), f(rstd), f(dx), f(dw), f(db), R, C, ptr(ws), wsb,
                              nullptr),
        "layernorm backward");
}

// ------------------------------------------------------------ flash attention (cppsrc/ops/flash_attention.cpp:15-22)
void flash_attention_forward_cuda(const Tensor& q, const Tensor& k, const Tensor& v, Tensor& out, Tensor& lse,
                                  bool causal, float scale) {
  const int64_t d = last(q), T = q.shape[q.shape.size() - 2];
  if (d > 128) throw std::invalid_argument("flash_attention: d_head exceeds D_MAX (128)");
  if (n_of(q) == 0) return;
  const int64_t bh = n_of(q) / (T * d);
  const int64_t st[12] = {bh * T * d, T * d, d, bh * T * d, T * d, d, bh * T * d, T * d, d, bh * T * d, T * d, d};
  const size_t wsb = aar_flash_fwd_workspace_bytes(bh, T, d, causal);
  Tensor ws = scratch(wsb);
  check(aar_flash_fwd_strided_f32(f(q), f(k), f(v), f(out), f(lse), 1, bh, T, d, st, causal, scale, ptr(ws), wsb,
                                  nullptr),
        "flash_attention");
}
void flash_attention_backward_cuda(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& o,
                                   const Tensor& lse, const Tensor& go, Tensor& dq, Tensor& dk, Tensor& dv,
                                   bool causal, float scale) {
  const int64_t d = last(q), T = q.shape[q.shape.size() - 2];
  if (d > 128) throw std::invalid_argument("flash_attention: d_head exceeds D_MAX (128)");
  if (n_of(q) == 0) return;
  const int64_t bh = n_of(q) / (T * d);
  const Tensor god = dense(go);
  // The larger workspace keeps the dS tiles for the dQ pass; past 16 GiB the
  // minimum (dQ recomputes them) is used instead.
  size_t wsb = aar_flash_bwd_fast_workspace_bytes(bh, T, d, causal);
  if (wsb > (size_t(16) << 30)) wsb = aar_flash_bwd_workspace_bytes(bh, T, d);
  Tensor ws = scratch(wsb);
  check(aar_flash_bwd_f32(f(q), f(k), f(v), f(o), f(lse), f(god), f(dq), f(dk), f(dv), bh, T, d, causal, scale,
                          ptr(ws), wsb, nullptr),
        "flash_attention backward");
}

// ------------------------------------------------------------ elementwise (cppsrc/ops/elementwise.cpp:13-26)
Tensor add_cuda(const Tensor& a, const Tensor& b) { return binary(aar_add_f32, a, b, "add"); }
Tensor sub_cuda(const Tensor& a, const Tensor& b) { return binary(aar_sub_f32, a, b, "sub"); }
Tensor mul_cuda(const Tensor& a, const Tensor& b) { return binary(aar_mul_f32, a, b, "mul"); }
Tensor relu_backward_cuda(const Tensor& g, const Tensor& x) { return binary(aar_relu_bwd_f32, g, x, "relu backward"); }
Tensor gelu_backward_cuda(const Tensor& g, const Tensor& x) { return binary(aar_gelu_bwd_f32, g, x, "gelu backward"); }
Tensor relu_cuda(const Tensor& a) { return unary(aar_relu_f32, a, "relu"); }
Tensor neg_cuda(const Tensor& a) { return unary(aar_neg_f32, a, "neg"); }
Tensor gelu_cuda(const Tensor& a) { return unary(aar_gelu_f32, a, "gelu"); }
Tensor scale_cuda(const Tensor& x, float alpha) {
  Tensor out = device_empty(x.shape);
  if (n_of(x)) check(aar_scale_f32(f(x), f(out), alpha, n_of(x), nullptr), "scale");
  return out;
}
void fill_cuda(Tensor& out, float v) {
  if (n_of(out)) check(aar_fill_f32(f(out), v, n_of(out), nullptr), "fill");
}
void scaled_add_inplace_cuda(Tensor& dst, const Tensor& src, float alpha) {
  if (n_of(dst)) check(aar_scaled_add_f32(f(dst), f(src), alpha, n_of(dst), nullptr), "scaled_add_inplace");
}
Tensor sum_all_cuda(const Tensor& a) {
  Tensor out = device_empty({});
  const size_t wsb = aar_sum_workspace_bytes(n_of(a));
  Tensor ws = scratch(wsb);
  check(aar_sum_f32(f(a), f(out), n_of(a), ptr(ws), wsb, nullptr), "sum_all");
  return out;
}
Tensor add_bias_cuda(const Tensor& x, const Tensor& bias) {
  Tensor out = device_empty(x.shape);
  if (n_of(x)) check(aar_add_bias_f32(f(x), f(bias), f(out), rows_of(x), last(x), nullptr), "add_bias");
  return out;
}
Tensor bias_grad_cuda(const Tensor& g, int64_t D) {
  Tensor db = device_empty({D});
  if (D == 0) return db;
  const int64_t R = n_of(g) / D;
  if (R == 0) {
    zero_bytes(db.data(), Device::CUDA, db.nbytes());
    return db;
  }
  const size_t wsb = aar_colsum_workspace_bytes(R, D);
  Tensor ws = scratch(wsb);
  check(aar_colsum_f32(f(g), f(db), R, D, ptr(ws), wsb, nullptr), "bias_grad");
  return db;
}

// ------------------------------------------------------------ embedding (cppsrc/ops/embedding.cpp:9-11)
Tensor embedding_cuda(const Tensor& weight, const Tensor& id) {
  const int64_t V = weight.shape[0], D = weight.shape[1];
  std::vector<int64_t> shape = id.shape;
  shape.push_back(D);
  Tensor out = device_empty(shape);
  if (n_of(id) && D) check(aar_embedding_fwd_f32(f(weight), ids(id), f(out), n_of(id), V, D, nullptr, nullptr),
                           "embedding");
  return out;
}
Tensor embedding_backward_cuda(const Tensor& g, const Tensor& id, int64_t vocab) {
  const int64_t D = last(g), N = n_of(id);
  Tensor dw = device_empty({vocab, D});
  if (N == 0 || D == 0 || vocab == 0) {
    zero_bytes(dw.data(), Device::CUDA, dw.nbytes());
    return dw;
  }
  const size_t wsb = aar_embedding_bwd_workspace_bytes(N, vocab, D);
  Tensor ws = scratch(wsb);
  check(aar_embedding_bwd_f32(f(g), ids(id), f(dw), N, vocab, D, ptr(ws), wsb, nullptr), "embedding backward");
  return dw;
}

// ------------------------------------------------------------ cross entropy (cppsrc/ops/cross_entropy.cpp:12-15)
Tensor cross_entropy_cuda(const Tensor& logits, const Tensor& targets, int64_t ignore_index) {
  const int64_t N = logits.shape[0], V = logits.shape[1];
  Tensor loss = device_empty({});
  const size_t wsb = aar_cross_entropy_workspace_bytes(N);
  Tensor ws = scratch(wsb);
  check(aar_cross_entropy_fwd_f32(f(logits), ids(targets), f(loss), N, V, ignore_index, nullptr, ptr(ws), wsb,
                                  nullptr),
        "cross_entropy");
  return loss;
}
Tensor cross_entropy_backward_cuda(const Tensor& grad_output, const Tensor& logits, const Tensor& targets,
                                   int64_t ignore_index) {
  const int64_t N = logits.shape[0], V = logits.shape[1];
  Tensor dl = device_empty({N, V});
  const size_t wsb = aar_cross_entropy_workspace_bytes(N);
  Tensor ws = scratch(wsb);
  check(aar_cross_entropy_bwd_f32(f(grad_output), f(logits), ids(targets), f(dl), N, V, ignore_index, ptr(ws), wsb,
                                  nullptr),
        "cross_entropy backward");
  return dl;
}

// ------------------------------------------------------------ dropout, AdamW, causal mask
void dropout_cuda(const Tensor& x, float p, uint64_t seed, Tensor& out, Tensor& mask) {
  if (n_of(x)) check(aar_dropout_f32(f(x), f(out), f(mask), n_of(x), p, seed, nullptr), "dropout");
}
void adamw_step_cuda(Tensor& param, const Tensor& grad, Tensor& m, Tensor& v, float lr, float beta1, float beta2,
                     float eps, float weight_decay, float bias_correction1, float bias_correction2) {
  if (n_of(param))
    check(aar_adamw_f32(f(param), f(grad), f(m), f(v), n_of(param), lr, beta1, beta2, eps, weight_decay,
                        bias_correction1, bias_correction2, nullptr),
          "adamw_step");
}
Tensor apply_causal_mask_cuda(const Tensor& x) { return causal_mask(x, -std::numeric_limits<float>::infinity()); }
Tensor causal_mask_backward_cuda(const Tensor& g) { return causal_mask(g, 0.0f); }

// ------------------------------------------------------------ strided copies (cppsrc/ops/shape.cpp:11-12)
void contiguous_cuda(const Tensor& src, Tensor& dst) {
  if (n_of(src) == 0) return;
  const std::vector<int64_t> cs = compute_contiguous_strides(src.shape);
  check(aar_strided_copy_f32(f(src), f(dst), static_cast<int>(src.shape.size()), src.shape.data(),
                             src.strides.data(), cs.data(), nullptr),
        "contiguous");
}
void copy_contiguous_into_strided_cuda(const Tensor& src, Tensor& dst) {
  if (n_of(src) == 0) return;
  const std::vector<int64_t> cs = compute_contiguous_strides(src.shape);
  check(aar_strided_copy_f32(f(src), f(dst), static_cast<int>(src.shape.size()), src.shape.data(), cs.data(),
                             dst.strides.data(), nullptr),
        "copy_contiguous_into_strided");
}

}  // namespace vlm
