// Ops of the GPT training step around the hot path: elementwise family,
// bias add, sum_all, embedding, cross entropy, SGD / AdamW updates.
// Validation messages, exception types and autograd Functions follow:
//   cppsrc/ops/elementwise.cpp:29-42 (check_binary), :182-197 (check_bias),
//     :225-300 (Functions), :315-474 (public ops)
//   cppsrc/ops/embedding.cpp:63-104
//   cppsrc/ops/cross_entropy.cpp:103-152
//   cppsrc/ops/adamw.cpp:11-20, :47-75
// Device arithmetic runs in the kernels of csrc/hip/nn_ops.hip through the C
// ABI; every reduction there is fixed-order, so results are reproducible.
#include <cmath>
#include <cstring>

#include "aar_hip.h"
#include "ops.hpp"

namespace aar {

namespace {

const float* fp(const Tensor& t) { return static_cast<const float*>(t.data()); }
float* fp(Tensor& t) { return static_cast<float*>(t.data()); }
const int64_t* ip(const Tensor& t) { return static_cast<const int64_t*>(t.data()); }

Tensor as_contig(const Tensor& t) { return t.is_contiguous() ? t : contiguous(t); }

void check_binary(const Tensor& a, const Tensor& b, const char* op) {
  if (a.shape != b.shape) throw std::invalid_argument(std::string(op) + ": shape mismatch");
  if (a.dtype != b.dtype) throw std::invalid_argument(std::string(op) + ": dtype mismatch");
  if (a.device != b.device) throw std::invalid_argument(std::string(op) + ": device mismatch");
  if (a.dtype != DType::Fp32) throw std::invalid_argument(std::string(op) + ": only Fp32 supported");
}

int64_t n_of(const Tensor& t) { return static_cast<int64_t>(t.numel()); }

// ---------------------------------------------------------- device legs

Tensor sub_dev(const Tensor& a, const Tensor& b) {
  if (a.device == Device::CPU) throw_cpu_compute("sub");
  Tensor out = Tensor::empty(a.shape, a.dtype, a.device);
  check_status(aar_sub_f32(fp(a), fp(b), fp(out), n_of(a), current_stream()), "sub");
  return out;
}

Tensor mul_dev(const Tensor& a, const Tensor& b) {
  if (a.device == Device::CPU) throw_cpu_compute("mul");
  Tensor out = Tensor::empty(a.shape, a.dtype, a.device);
  check_status(aar_mul_f32(fp(a), fp(b), fp(out), n_of(a), current_stream()), "mul");
  return out;
}

Tensor scale_dev(const Tensor& x, float alpha) {
  if (x.device == Device::CPU) throw_cpu_compute("scale");
  Tensor out = Tensor::empty(x.shape, x.dtype, x.device);
  check_status(aar_scale_f32(fp(x), fp(out), alpha, n_of(x), current_stream()), "scale");
  return out;
}

Tensor neg_dev(const Tensor& x) {
  if (x.device == Device::CPU) throw_cpu_compute("neg");
  Tensor out = Tensor::empty(x.shape, x.dtype, x.device);
  check_status(aar_neg_f32(fp(x), fp(out), n_of(x), current_stream()), "neg");
  return out;
}

Tensor relu_dev(const Tensor& x) {
  if (x.device == Device::CPU) throw_cpu_compute("relu");
  Tensor out = Tensor::empty(x.shape, x.dtype, x.device);
  check_status(aar_relu_f32(fp(x), fp(out), n_of(x), current_stream()), "relu");
  return out;
}

Tensor relu_bwd_dev(const Tensor& g, const Tensor& x) {
  Tensor gc = as_contig(g);
  Tensor out = Tensor::empty(gc.shape, gc.dtype, gc.device);
  check_status(aar_relu_bwd_f32(fp(gc), fp(x), fp(out), n_of(gc), current_stream()), "relu backward");
  return out;
}

Tensor gelu_dev(const Tensor& x) {
  if (x.device == Device::CPU) throw_cpu_compute("gelu");
  Tensor out = Tensor::empty(x.shape, x.dtype, x.device);
  check_status(aar_gelu_f32(fp(x), fp(out), n_of(x), current_stream()), "gelu");
  return out;
}

Tensor gelu_bwd_dev(const Tensor& g, const Tensor& x) {
  Tensor gc = as_contig(g);
  Tensor out = Tensor::empty(gc.shape, gc.dtype, gc.device);
  check_status(aar_gelu_bwd_f32(fp(gc), fp(x), fp(out), n_of(gc), current_stream()), "gelu backward");
  return out;
}

Tensor add_bias_dev(const Tensor& x, const Tensor& b) {
  if (x.device == Device::CPU) throw_cpu_compute("add_bias");
  Tensor out = Tensor::empty(x.shape, x.dtype, x.device);
  const int64_t D = b.shape[0];
  if (D == 0) return out;  // no columns: nothing to add
  check_status(aar_add_bias_f32(fp(x), fp(b), fp(out), n_of(x) / D, D, current_stream()), "add_bias");
  return out;
}

Tensor bias_grad_dev(const Tensor& g, int64_t D) {
  Tensor gc = as_contig(g);
  Tensor db = Tensor::empty({D}, gc.dtype, gc.device);
  if (D == 0) return db;  // no columns: nothing to sum
  const int64_t rows = n_of(gc) / D;
  Workspace ws(aar_colsum_workspace_bytes(rows, D));
  check_status(aar_colsum_f32(fp(gc), fp(db), rows, D, ws.data(), ws.bytes(), current_stream()), "bias_grad");
  return db;
}

Tensor sum_all_dev(const Tensor& a) {
  if (a.device == Device::CPU) throw_cpu_compute("sum_all");
  Tensor out = Tensor::empty({}, a.dtype, a.device);
  Workspace ws(aar_sum_workspace_bytes(n_of(a)));
  check_status(aar_sum_f32(fp(a), fp(out), n_of(a), ws.data(), ws.bytes(), current_stream()), "sum_all");
  return out;
}

// ------------------------------------------------------------- Functions

class SubFunction : public Function {
 public:
  std::vector<Tensor> backward(const Tensor& g) override { return {g, neg_dev(as_contig(g))}; }
  const char* name() const override { return "SubFunction"; }
};

class MulFunction : public Function {
 public:
  Tensor saved_a, saved_b;
  std::vector<Tensor> backward(const Tensor& g) override {
    Tensor gc = as_contig(g);
    return {mul_dev(gc, saved_b), mul_dev(gc, saved_a)};
  }
  const char* name() const override { return "MulFunction"; }
};

class ScaleFunction : public Function {
 public:
  float alpha = 1.0f;
  std::vector<Tensor> backward(const Tensor& g) override { return {scale_dev(as_contig(g), alpha)}; }
  const char* name() const override { return "ScaleFunction"; }
};

class ReluFunction : public Function {
 public:
  Tensor saved_x;
  std::vector<Tensor> backward(const Tensor& g) override { return {relu_bwd_dev(g, saved_x)}; }
  const char* name() const override { return "ReluFunction"; }
};

class GeluFunction : public Function {
 public:
  Tensor saved_x;
  std::vector<Tensor> backward(const Tensor& g) override { return {gelu_bwd_dev(g, saved_x)}; }
  const char* name() const override { return "GeluFunction"; }
};

class AddBiasFunction : public Function {
 public:
  int64_t bias_size = 0;
  std::vector<Tensor> backward(const Tensor& g) override { return {g, bias_grad_dev(g, bias_size)}; }
  const char* name() const override { return "AddBiasFunction"; }
};

// d(sum)/dx = broadcast of the scalar grad; the scalar is read on the device
// (no host round trip, unlike the reference's copy to the host).
class SumAllFunction : public Function {
 public:
  std::vector<int64_t> input_shape;
  std::vector<Tensor> backward(const Tensor& g) override {
    Tensor out = Tensor::empty(input_shape, DType::Fp32, Device::CUDA);
    Tensor gc = as_contig(g);
    // out = 0 * out + 1 * broadcast(g): fill from the device scalar via add_bias
    // with a 1-column view (rows = numel, cols = 1).
    Tensor zero = Tensor::zeros(input_shape, DType::Fp32, Device::CUDA);
    check_status(aar_add_bias_f32(fp(zero), fp(gc), fp(out), n_of(out), 1, current_stream()),
                 "sum_all backward");
    return {out};
  }
  const char* name() const override { return "SumAllFunction"; }
};

class EmbeddingFunction : public Function {
 public:
  Tensor saved_ids;
  int64_t vocab_size = 0;
  std::vector<Tensor> backward(const Tensor& g) override {
    Tensor gc = as_contig(g);
    const int64_t D = gc.shape.back();
    const int64_t n = n_of(saved_ids);
    Tensor dW = Tensor::empty({vocab_size, D}, DType::Fp32, Device::CUDA);
    Workspace ws(aar_embedding_bwd_workspace_bytes(n, vocab_size, D));
    check_status(aar_embedding_bwd_f32(fp(gc), ip(saved_ids), fp(dW), n, vocab_size, D, ws.data(), ws.bytes(),
                                       current_stream()),
                 "embedding backward");
    return {dW};
  }
  const char* name() const override { return "EmbeddingFunction"; }
};

// add(embedding(w1, ids1), embedding(w2, ids2)) as one node: the gradient of
// each table is the embedding backward of the same g.
class EmbeddingAddFunction : public Function {
 public:
  Tensor saved_ids1, saved_ids2;
  int64_t vocab1 = 0, vocab2 = 0;
  std::vector<Tensor> backward(const Tensor& g) override {
    Tensor gc = as_contig(g);
    const int64_t D = gc.shape.back();
    auto table_grad = [&](const Tensor& ids, int64_t V) {
      const int64_t n = n_of(ids);
      Tensor dW = Tensor::empty({V, D}, DType::Fp32, Device::CUDA);
      Workspace ws(aar_embedding_bwd_workspace_bytes(n, V, D));
      check_status(aar_embedding_bwd_f32(fp(gc), ip(ids), fp(dW), n, V, D, ws.data(), ws.bytes(), current_stream()),
                   "embedding backward");
      return dW;
    };
    return {table_grad(saved_ids1, vocab1), table_grad(saved_ids2, vocab2)};
  }
  const char* name() const override { return "EmbeddingAddFunction"; }
};

class CrossEntropyFunction : public Function {
 public:
  Tensor saved_logits, saved_targets;
  int64_t ignore_index = -100;
  std::vector<Tensor> backward(const Tensor& g) override {
    Tensor gc = as_contig(g);
    const int64_t N = saved_logits.shape[0], V = saved_logits.shape[1];
    Tensor dL = Tensor::empty({N, V}, DType::Fp32, Device::CUDA);
    Workspace ws(aar_cross_entropy_workspace_bytes(N));
    check_status(aar_cross_entropy_bwd_f32(fp(gc), fp(saved_logits), ip(saved_targets), fp(dL), N, V,
                                           ignore_index, ws.data(), ws.bytes(), current_stream()),
                 "cross_entropy backward");
    return {dL};
  }
  const char* name() const override { return "CrossEntropyFunction"; }
};

template <typename Fn>
Tensor attach(std::shared_ptr<Fn> fn, Tensor out) {
  out.requires_grad = true;
  out.grad_fn = std::move(fn);
  return out;
}

}  // namespace

// ======================================================================= API

Tensor sub(const Tensor& a, const Tensor& b) {
  check_binary(a, b, "sub");
  Tensor ac = as_contig(a), bc = as_contig(b);
  if (!ac.requires_grad && !bc.requires_grad) return sub_dev(ac, bc);
  auto fn = std::make_shared<SubFunction>();
  fn->record_input(ac);
  fn->record_input(bc);
  return attach(fn, sub_dev(ac, bc));
}

Tensor mul(const Tensor& a, const Tensor& b) {
  check_binary(a, b, "mul");
  Tensor ac = as_contig(a), bc = as_contig(b);
  if (!ac.requires_grad && !bc.requires_grad) return mul_dev(ac, bc);
  auto fn = std::make_shared<MulFunction>();
  fn->record_input(ac);
  fn->record_input(bc);
  fn->saved_a = ac;
  fn->saved_b = bc;
  return attach(fn, mul_dev(ac, bc));
}

Tensor scale(const Tensor& x, float alpha) {
  if (x.dtype != DType::Fp32) throw std::invalid_argument("scale: only Fp32 supported");
  Tensor xc = as_contig(x);
  if (!xc.requires_grad) return scale_dev(xc, alpha);
  auto fn = std::make_shared<ScaleFunction>();
  fn->record_input(xc);
  fn->alpha = alpha;
  return attach(fn, scale_dev(xc, alpha));
}

Tensor relu(const Tensor& a) {
  if (a.dtype != DType::Fp32) throw std::invalid_argument("relu: only Fp32 supported");
  Tensor ac = as_contig(a);
  if (!ac.requires_grad) return relu_dev(ac);
  auto fn = std::make_shared<ReluFunction>();
  fn->record_input(ac);
  fn->saved_x = ac;
  return attach(fn, relu_dev(ac));
}

Tensor gelu(const Tensor& a) {
  if (a.dtype != DType::Fp32) throw std::invalid_argument("gelu: only Fp32 supported");
  Tensor ac = as_contig(a);
  if (!ac.requires_grad) return gelu_dev(ac);
  auto fn = std::make_shared<GeluFunction>();
  fn->record_input(ac);
  fn->saved_x = ac;
  return attach(fn, gelu_dev(ac));
}

Tensor sum_all(const Tensor& a) {
  if (a.dtype != DType::Fp32) throw std::invalid_argument("sum_all: only Fp32 supported");
  Tensor ac = as_contig(a);
  if (!ac.requires_grad) return sum_all_dev(ac);
  auto fn = std::make_shared<SumAllFunction>();
  fn->record_input(ac);
  fn->input_shape = ac.shape;
  return attach(fn, sum_all_dev(ac));
}

Tensor add_bias(const Tensor& x, const Tensor& bias) {
  if (bias.shape.size() != 1) throw std::invalid_argument("add_bias: bias must be 1-D");
  if (x.shape.empty() || x.shape.back() != bias.shape[0]) {
    throw std::invalid_argument("add_bias: bias size must match x's last dim");
  }
  if (x.dtype != bias.dtype || x.dtype != DType::Fp32) throw std::invalid_argument("add_bias: only Fp32 supported");
  if (x.device != bias.device) throw std::invalid_argument("add_bias: device mismatch");
  Tensor xc = as_contig(x), bc = as_contig(bias);
  if (!xc.requires_grad && !bc.requires_grad) return add_bias_dev(xc, bc);
  auto fn = std::make_shared<AddBiasFunction>();
  fn->record_input(xc);
  fn->record_input(bc);
  fn->bias_size = bc.shape[0];
  return attach(fn, add_bias_dev(xc, bc));
}

namespace {
void check_scaled_add(const Tensor& dst, const Tensor& src) {
  if (dst.shape != src.shape) throw std::invalid_argument("scaled_add_inplace: shape mismatch");
  if (dst.dtype != src.dtype || dst.dtype != DType::Fp32) {
    throw std::invalid_argument("scaled_add_inplace: only Fp32 supported");
  }
  if (dst.device != src.device) throw std::invalid_argument("scaled_add_inplace: device mismatch");
  if (!dst.is_contiguous()) throw std::invalid_argument("scaled_add_inplace: dst must be contiguous");
  if (dst.device == Device::CPU) throw_cpu_compute("scaled_add_inplace");
}
}  // namespace

void scaled_add_inplace(Tensor& dst, const Tensor& src, float alpha) {
  check_scaled_add(dst, src);
  Tensor sc = as_contig(src);
  check_status(aar_scaled_add_f32(fp(dst), fp(sc), alpha, n_of(dst), current_stream()), "scaled_add_inplace");
}

void scaled_add_inplace_multi(std::vector<Tensor>& dsts, const std::vector<Tensor>& srcs, float alpha) {
  if (dsts.size() != srcs.size()) throw std::invalid_argument("scaled_add_inplace: list length mismatch");
  std::vector<Tensor> sc;
  sc.reserve(srcs.size());
  std::vector<float*> d;
  std::vector<const float*> s;
  std::vector<int64_t> n;
  for (size_t i = 0; i < dsts.size(); ++i) {
    check_scaled_add(dsts[i], srcs[i]);
    sc.push_back(as_contig(srcs[i]));
    d.push_back(fp(dsts[i]));
    s.push_back(fp(sc.back()));
    n.push_back(n_of(dsts[i]));
  }
  check_status(aar_scaled_add_multi_f32(static_cast<int>(d.size()), d.data(), s.data(), n.data(), alpha,
                                        current_stream()),
               "scaled_add_inplace");
}

Tensor embedding(const Tensor& weight, const Tensor& ids) {
  if (weight.dtype != DType::Fp32) throw std::invalid_argument("embedding: weight must be Fp32");
  if (ids.dtype != DType::Int64) throw std::invalid_argument("embedding: ids must be Int64");
  if (weight.shape.size() != 2) {
    throw std::invalid_argument("embedding: weight must be 2D (vocab_size, embed_dim)");
  }
  if (weight.device != ids.device) throw std::invalid_argument("embedding: device mismatch");
  Tensor wc = as_contig(weight), ic = as_contig(ids);
  if (wc.device == Device::CPU) throw_cpu_compute("embedding");
  const int64_t V = wc.shape[0], D = wc.shape[1];
  std::vector<int64_t> out_shape = ic.shape;
  out_shape.push_back(D);
  Tensor out = Tensor::empty(out_shape, DType::Fp32, Device::CUDA);
  check_status(aar_embedding_fwd_f32(fp(wc), ip(ic), fp(out), n_of(ic), V, D, device_error_word(kErrEmbeddingId),
                                     current_stream()),
               "embedding");
  if (!wc.requires_grad) return out;
  auto fn = std::make_shared<EmbeddingFunction>();
  fn->record_input(wc);
  fn->saved_ids = ic;
  fn->vocab_size = V;
  return attach(fn, out);
}

// add(embedding(w1, ids1), embedding(w2, ids2)), the token + position
// embeddings of a GPT (python/shakespeare/scripts/model.py:53), as one
// lookup-and-add pass (aar_embedding_add_fwd_f32): the same values, and the
// same gradients for both tables.  Anything the fused pass does not cover
// (other dtypes or ranks, id shapes that differ, host tensors) takes the
// composition, with its checks and messages.
Tensor embedding_add(const Tensor& w1, const Tensor& ids1, const Tensor& w2, const Tensor& ids2) {
  const bool plain = w1.dtype == DType::Fp32 && w2.dtype == DType::Fp32 && ids1.dtype == DType::Int64 &&
                     ids2.dtype == DType::Int64 && w1.shape.size() == 2 && w2.shape.size() == 2 &&
                     w1.shape[1] == w2.shape[1] && ids1.shape == ids2.shape && w1.device == Device::CUDA &&
                     w2.device == Device::CUDA && ids1.device == Device::CUDA && ids2.device == Device::CUDA;
  if (!plain) return add(embedding(w1, ids1), embedding(w2, ids2));
  Tensor wc1 = as_contig(w1), wc2 = as_contig(w2), ic1 = as_contig(ids1), ic2 = as_contig(ids2);
  const int64_t V1 = wc1.shape[0], V2 = wc2.shape[0], D = wc1.shape[1];
  std::vector<int64_t> out_shape = ic1.shape;
  out_shape.push_back(D);
  Tensor out = Tensor::empty(out_shape, DType::Fp32, Device::CUDA);
  check_status(aar_embedding_add_fwd_f32(fp(wc1), ip(ic1), V1, fp(wc2), ip(ic2), V2, fp(out), n_of(ic1), D,
                                         device_error_word(kErrEmbeddingId), current_stream()),
               "embedding");
  if (!wc1.requires_grad && !wc2.requires_grad) return out;
  auto fn = std::make_shared<EmbeddingAddFunction>();
  fn->record_input(wc1);
  fn->record_input(wc2);
  fn->saved_ids1 = ic1;
  fn->saved_ids2 = ic2;
  fn->vocab1 = V1;
  fn->vocab2 = V2;
  return attach(fn, out);
}

Tensor cross_entropy(const Tensor& logits, const Tensor& targets, int64_t ignore_index) {
  if (logits.dtype != DType::Fp32) throw std::invalid_argument("cross_entropy: logits must be Fp32");
  if (targets.dtype != DType::Int64) throw std::invalid_argument("cross_entropy: targets must be Int64");
  if (logits.shape.size() != 2) throw std::invalid_argument("cross_entropy: logits must be 2D (N, V)");
  if (targets.shape.size() != 1 || targets.shape[0] != logits.shape[0]) {
    throw std::invalid_argument("cross_entropy: targets must be 1D matching N");
  }
  if (logits.device != targets.device) throw std::invalid_argument("cross_entropy: device mismatch");
  Tensor lc = as_contig(logits), tc = as_contig(targets);
  if (lc.device == Device::CPU) throw_cpu_compute("cross_entropy");
  const int64_t N = lc.shape[0], V = lc.shape[1];
  Tensor out = Tensor::empty({}, DType::Fp32, Device::CUDA);
  Workspace ws(aar_cross_entropy_workspace_bytes(N));
  check_status(aar_cross_entropy_fwd_f32(fp(lc), ip(tc), fp(out), N, V, ignore_index,
                                         device_error_word(kErrCrossEntropyTarget), ws.data(), ws.bytes(),
                                         current_stream()),
               "cross_entropy");
  if (!lc.requires_grad) return out;
  auto fn = std::make_shared<CrossEntropyFunction>();
  fn->record_input(lc);
  fn->saved_logits = lc;
  fn->saved_targets = tc;
  fn->ignore_index = ignore_index;
  return attach(fn, out);
}

namespace {
void check_adamw(const Tensor& param, const Tensor& grad, const Tensor& m, const Tensor& v) {
  if (param.dtype != DType::Fp32) throw std::invalid_argument("adamw_step: only Fp32 supported");
  auto check_match = [&](const Tensor& b, const char* what) {
    if (param.shape != b.shape) throw std::invalid_argument(std::string("adamw_step: ") + what + " shape mismatch");
    if (param.dtype != b.dtype) throw std::invalid_argument(std::string("adamw_step: ") + what + " dtype mismatch");
    if (param.device != b.device) {
      throw std::invalid_argument(std::string("adamw_step: ") + what + " device mismatch");
    }
  };
  check_match(grad, "grad");
  check_match(m, "m");
  check_match(v, "v");
  if (!param.is_contiguous() || !grad.is_contiguous() || !m.is_contiguous() || !v.is_contiguous()) {
    throw std::invalid_argument("adamw_step: all tensors must be contiguous");
  }
  if (param.device == Device::CPU) throw_cpu_compute("adamw_step");
}
}  // namespace

void adamw_step(Tensor& param, const Tensor& grad, Tensor& m, Tensor& v, float lr, float beta1, float beta2,
                float eps, float weight_decay, float bias_correction1, float bias_correction2) {
  check_adamw(param, grad, m, v);
  check_status(aar_adamw_f32(fp(param), fp(grad), fp(m), fp(v), n_of(param), lr, beta1, beta2, eps, weight_decay,
                             bias_correction1, bias_correction2, current_stream()),
               "adamw_step");
}

void adamw_step_multi(std::vector<Tensor>& params, const std::vector<Tensor>& grads, std::vector<Tensor>& ms,
                      std::vector<Tensor>& vs, float lr, float beta1,
                      float beta2, float eps, float weight_decay, float bias_correction1, float bias_correction2) {
  if (grads.size() != params.size() || ms.size() != params.size() || vs.size() != params.size()) {
    throw std::invalid_argument("adamw_step: list length mismatch");
  }
  std::vector<float*> p, m, v;
  std::vector<const float*> g;
  std::vector<int64_t> n;
  for (size_t i = 0; i < params.size(); ++i) {
    check_adamw(params[i], grads[i], ms[i], vs[i]);
    p.push_back(fp(params[i]));
    g.push_back(fp(grads[i]));
    m.push_back(fp(ms[i]));
    v.push_back(fp(vs[i]));
    n.push_back(n_of(params[i]));
  }
  check_status(aar_adamw_multi_f32(static_cast<int>(p.size()), p.data(), g.data(), m.data(), v.data(), n.data(), lr,
                                   beta1, beta2, eps, weight_decay, bias_correction1, bias_correction2,
                                   current_stream()),
               "adamw_step");
}

}  // namespace aar
