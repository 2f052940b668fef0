// Op layer of aargrad._core: validation, autograd Functions and dispatch to
// the device kernels through the C ABI (include/aar_hip.h).
//
// Validation messages, exception types, contiguity handling, leading-dim
// flattening and the Function graph follow the reference op files:
//   matmul*      cppsrc/ops/matmul.cpp:93-257
//   softmax      cppsrc/ops/softmax.cpp:57-96
//   layernorm    cppsrc/ops/layernorm.cpp:136-227
//   flash        cppsrc/ops/flash_attention.cpp:25-98
//   views        cppsrc/ops/shape.cpp:99-374
//   add          cppsrc/ops/elementwise.cpp:29-42, :225-231, :315-330
// The device half replaces each reference *_cuda function; host tensors are
// accepted by the view ops (metadata plus a host-side layout copy) but every
// arithmetic op raises for Device.CPU: this build computes on the GPU only.
#include "ops.hpp"

#include <cmath>
#include <cstring>

#include <new>
#include <optional>

#include "aar_hip.h"

namespace aar {

namespace {

// Flash backward workspace.  The stored-dS size (the dQ pass then reads the
// dS tiles the dK/dV pass wrote instead of recomputing them) when it stays
// under kFlashDsCap and the allocator can serve it; otherwise the minimum,
// which selects the recompute path.
constexpr size_t kFlashDsCap = size_t(16) << 30;
Workspace flash_bwd_workspace(int64_t bh, int64_t T, int64_t d, bool causal) {
  const size_t fast = aar_flash_bwd_fast_workspace_bytes(bh, T, d, causal ? 1 : 0);
  if (fast <= kFlashDsCap) {
    try {
      return Workspace(fast);
    } catch (const std::bad_alloc&) {
    }
  }
  return Workspace(aar_flash_bwd_workspace_bytes(bh, T, d));
}

// Flash forward workspace: the partials of the causal key-range split when
// the shape may split (none otherwise).
Workspace flash_fwd_workspace(int64_t bh, int64_t T, int64_t d, bool causal) {
  return Workspace(aar_flash_fwd_workspace_bytes(bh, T, d, causal ? 1 : 0));
}

const float* fp(const Tensor& t) { return static_cast<const float*>(t.data()); }
float* fp(Tensor& t) { return static_cast<float*>(t.data()); }

Tensor as_view(const Tensor& src, std::vector<int64_t> new_shape) {
  auto strides = compute_contiguous_strides(new_shape);
  return make_view(src, std::move(new_shape), std::move(strides), src.storage_offset);
}

Tensor as_contig(const Tensor& t) { return t.is_contiguous() ? t : contiguous(t); }

// ------------------------------------------------------------- layout copies

void copy_strided_to_contiguous_host(const Tensor& src, Tensor& dst) {
  const size_t ndim = src.shape.size();
  const size_t total = src.numel();
  if (total == 0) return;
  const size_t es = dtype_size(src.dtype);
  const char* X = static_cast<const char*>(src.data());
  char* Y = static_cast<char*>(dst.data());
  std::vector<int64_t> idx(ndim, 0);
  for (size_t flat = 0; flat < total; ++flat) {
    int64_t off = 0;
    for (size_t d = 0; d < ndim; ++d) off += idx[d] * src.strides[d];
    std::memcpy(Y + flat * es, X + off * (int64_t)es, es);
    for (int d = (int)ndim - 1; d >= 0; --d) {
      if (++idx[d] < src.shape[d]) break;
      idx[d] = 0;
    }
  }
}

void device_strided_copy(const Tensor& src, Tensor& dst, const char* what) {
  if (src.dtype != DType::Fp32) {
    throw std::runtime_error(std::string(what) + ": only Fp32 supported on CUDA");
  }
  if (src.shape.size() > 8) throw std::runtime_error(std::string(what) + ": rank > 8");
  check_status(aar_strided_copy_f32(fp(src), fp(dst), (int)src.shape.size(), src.shape.data(),
                                    src.strides.data(), dst.strides.data(), current_stream()),
               what);
}

void copy_contiguous_into_strided(const Tensor& src, Tensor& dst) {
  if (src.shape != dst.shape) throw std::runtime_error("copy_contiguous_into_strided: shape mismatch");
  if (src.dtype != dst.dtype || src.device != dst.device) {
    throw std::runtime_error("copy_contiguous_into_strided: dtype/device mismatch");
  }
  if (!src.is_contiguous()) {
    throw std::runtime_error("copy_contiguous_into_strided: src must be contiguous");
  }
  if (src.device == Device::CUDA) {
    device_strided_copy(src, dst, "copy_contiguous_into_strided");
    return;
  }
  // host: walk the destination view
  const size_t ndim = src.shape.size();
  const size_t total = src.numel();
  if (total == 0) return;
  const size_t es = dtype_size(src.dtype);
  const char* X = static_cast<const char*>(src.data());
  char* Y = static_cast<char*>(dst.data());
  std::vector<int64_t> idx(ndim, 0);
  for (size_t flat = 0; flat < total; ++flat) {
    int64_t off = 0;
    for (size_t d = 0; d < ndim; ++d) off += idx[d] * dst.strides[d];
    std::memcpy(Y + off * (int64_t)es, X + flat * es, es);
    for (int d = (int)ndim - 1; d >= 0; --d) {
      if (++idx[d] < src.shape[d]) break;
      idx[d] = 0;
    }
  }
}

// Target shape of a reshape: every entry is an extent >= 0, except at most
// one -1 whose extent is whatever makes the element count match.  Entries are
// checked left to right, so the first offending entry picks the message (the
// messages are those of the reference's reshape, cppsrc/ops/shape.cpp:15-44).
std::vector<int64_t> resolve_new_shape(const std::vector<int64_t>& request, size_t numel) {
  const int64_t total = static_cast<int64_t>(numel);
  std::optional<size_t> infer_at;
  int64_t fixed = 1;  // product of the given extents
  for (size_t i = 0; i < request.size(); ++i) {
    const int64_t e = request[i];
    if (e >= 0) {
      fixed *= e;
    } else if (e != -1) {
      throw std::invalid_argument("reshape: negative dim other than -1");
    } else if (infer_at) {
      throw std::invalid_argument("reshape: at most one -1 dim allowed");
    } else {
      infer_at = i;
    }
  }
  if (!infer_at) {
    if (fixed != total) throw std::invalid_argument("reshape: numel mismatch");
    return request;
  }
  if (fixed == 0 || total % fixed != 0) throw std::invalid_argument("reshape: cannot infer -1 dim");
  std::vector<int64_t> shape = request;
  shape[*infer_at] = total / fixed;
  return shape;
}

// ------------------------------------------------------------ view Functions

class ReshapeFunction : public Function {
 public:
  std::vector<int64_t> original_shape;
  std::vector<Tensor> backward(const Tensor& grad_output) override {
    Tensor g = as_contig(grad_output);
    return {make_view(g, original_shape, compute_contiguous_strides(original_shape), g.storage_offset)};
  }
  const char* name() const override { return "ReshapeFunction"; }
};

class TransposeFunction : public Function {
 public:
  int64_t dim_a = 0, dim_b = 0;
  std::vector<Tensor> backward(const Tensor& grad_output) override {
    std::vector<int64_t> sh = grad_output.shape, st = grad_output.strides;
    std::swap(sh[dim_a], sh[dim_b]);
    std::swap(st[dim_a], st[dim_b]);
    return {as_contig(make_view(grad_output, sh, st, grad_output.storage_offset))};
  }
  const char* name() const override { return "TransposeFunction"; }
};

class SliceFunction : public Function {
 public:
  std::vector<int64_t> original_shape;
  int64_t dim = 0, start = 0, end = 0;
  DType dtype = DType::Fp32;
  Device device = Device::CPU;
  std::vector<Tensor> backward(const Tensor& grad_output) override {
    Tensor full = Tensor::zeros(original_shape, dtype, device);
    Tensor slot = make_view(full, grad_output.shape, full.strides,
                            full.storage_offset + start * full.strides[dim]);
    Tensor src = as_contig(grad_output);
    copy_contiguous_into_strided(src, slot);
    return {full};
  }
  const char* name() const override { return "SliceFunction"; }
};

class SqueezeFunction : public Function {
 public:
  int64_t dim = 0, inserted_size_stride = 1;
  std::vector<Tensor> backward(const Tensor& grad_output) override {
    std::vector<int64_t> sh = grad_output.shape, st = grad_output.strides;
    sh.insert(sh.begin() + dim, 1);
    st.insert(st.begin() + dim, inserted_size_stride);
    return {as_contig(make_view(grad_output, sh, st, grad_output.storage_offset))};
  }
  const char* name() const override { return "SqueezeFunction"; }
};

class UnsqueezeFunction : public Function {
 public:
  int64_t dim = 0;
  std::vector<Tensor> backward(const Tensor& grad_output) override {
    std::vector<int64_t> sh = grad_output.shape, st = grad_output.strides;
    sh.erase(sh.begin() + dim);
    st.erase(st.begin() + dim);
    return {as_contig(make_view(grad_output, sh, st, grad_output.storage_offset))};
  }
  const char* name() const override { return "UnsqueezeFunction"; }
};

class ContiguousFunction : public Function {
 public:
  std::vector<Tensor> backward(const Tensor& grad_output) override { return {as_contig(grad_output)}; }
  const char* name() const override { return "ContiguousFunction"; }
};

// ------------------------------------------------------------------ GEMM

Tensor gemm_device(int op, const Tensor& a, const Tensor& b, int64_t M, int64_t N, int64_t K) {
  Tensor out = Tensor::empty({M, N}, DType::Fp32, Device::CUDA);
  if (out.numel() == 0) return out;
  const size_t wsb = aar_gemm_f32_workspace_bytes(op, M, N, K);
  Workspace ws(wsb);
  check_status(aar_gemm_f32(op, M, N, K, fp(a), fp(b), fp(out), ws.data(), ws.bytes(), current_stream()),
               op == AAR_GEMM_NN ? "matmul" : (op == AAR_GEMM_NT ? "matmul_a_bt" : "matmul_at_b"));
  return out;
}

// 2-D kernels (reference matmul_cuda / matmul_a_bt_cuda / matmul_at_b_cuda).
Tensor matmul_2d(const Tensor& a, const Tensor& b) {
  if (a.device == Device::CPU) throw_cpu_compute("matmul");
  return gemm_device(AAR_GEMM_NN, a, b, a.shape[0], b.shape[1], a.shape[1]);
}
Tensor matmul_a_bt_2d(const Tensor& a, const Tensor& b) {
  if (a.device == Device::CPU) throw_cpu_compute("matmul_a_bt");
  return gemm_device(AAR_GEMM_NT, a, b, a.shape[0], b.shape[0], a.shape[1]);
}
Tensor matmul_at_b_2d(const Tensor& a, const Tensor& b) {
  if (a.device == Device::CPU) throw_cpu_compute("matmul_at_b");
  return gemm_device(AAR_GEMM_TN, a, b, a.shape[1], b.shape[1], a.shape[0]);
}

// Product of all dims but the last (the flattened row count, also when the
// last dim is 0).
int64_t lead_rows(const Tensor& a) {
  int64_t m = 1;
  for (size_t i = 0; i + 1 < a.shape.size(); ++i) m *= a.shape[i];
  return m;
}

Tensor matmul_no_grad(const Tensor& a, const Tensor& b) {
  if (a.shape.size() == 2) return matmul_2d(a, b);
  const int64_t K = a.shape.back();
  const int64_t N = b.shape[1];
  const int64_t M_flat = lead_rows(a);
  Tensor out2d = matmul_2d(as_view(a, {M_flat, K}), b);
  std::vector<int64_t> out_shape(a.shape.begin(), a.shape.end() - 1);
  out_shape.push_back(N);
  return as_view(out2d, std::move(out_shape));
}

Tensor matmul_a_bt_no_grad(const Tensor& a, const Tensor& b) {
  if (a.shape.size() == 2) return matmul_a_bt_2d(a, b);
  const int64_t K = a.shape.back();
  const int64_t N = b.shape[0];
  const int64_t M_flat = lead_rows(a);
  Tensor out2d = matmul_a_bt_2d(as_view(a, {M_flat, K}), b);
  std::vector<int64_t> out_shape(a.shape.begin(), a.shape.end() - 1);
  out_shape.push_back(N);
  return as_view(out2d, std::move(out_shape));
}

Tensor matmul_at_b_no_grad(const Tensor& a, const Tensor& b) {
  if (a.shape.size() == 2 && b.shape.size() == 2) return matmul_at_b_2d(a, b);
  const int64_t M = a.shape.back();
  const int64_t N = b.shape.back();
  const int64_t K_flat = lead_rows(a);
  return matmul_at_b_2d(as_view(a, {K_flat, M}), as_view(b, {K_flat, N}));
}

class MatmulFunction : public Function {
 public:
  Tensor saved_a, saved_b;
  std::vector<Tensor> backward(const Tensor& g) override {
    return {matmul_a_bt_no_grad(g, saved_b), matmul_at_b_no_grad(saved_a, g)};
  }
  const char* name() const override { return "MatmulFunction"; }
};

class MatmulABTFunction : public Function {
 public:
  Tensor saved_a, saved_b;
  std::vector<Tensor> backward(const Tensor& g) override {
    return {matmul_no_grad(g, saved_b), matmul_at_b_no_grad(g, saved_a)};
  }
  const char* name() const override { return "MatmulABTFunction"; }
};

class MatmulATBFunction : public Function {
 public:
  Tensor saved_a, saved_b;
  std::vector<Tensor> backward(const Tensor& g) override {
    return {matmul_a_bt_no_grad(saved_b, g), matmul_no_grad(saved_a, g)};
  }
  const char* name() const override { return "MatmulATBFunction"; }
};

template <typename Fn, typename NoGrad>
Tensor with_matmul_grad(const Tensor& ac, const Tensor& bc, NoGrad no_grad) {
  if (!ac.requires_grad && !bc.requires_grad) return no_grad(ac, bc);
  auto fn = std::make_shared<Fn>();
  fn->record_input(ac);
  fn->record_input(bc);
  fn->saved_a = ac;
  fn->saved_b = bc;
  Tensor out = no_grad(ac, bc);
  out.requires_grad = true;
  out.grad_fn = fn;
  return out;
}

// Linear layer y = x W^T + b as one GEMM whose epilogue adds b (the reference
// runs matmul_a_bt and then add_bias: aargrad/nn.py:101-105).  The epilogue
// performs the same single fp32 addition per element as add_bias, so the
// result is bit-identical to the two-op composition.  K > 0 here.
Tensor linear_no_grad(const Tensor& x, const Tensor& w, const Tensor& b) {
  if (x.device == Device::CPU) throw_cpu_compute("linear");
  const int64_t K = x.shape.back();
  const int64_t N = w.shape[0];
  const int64_t M = static_cast<int64_t>(x.numel()) / K;
  Tensor out = Tensor::empty({M, N}, DType::Fp32, Device::CUDA);
  if (out.numel() != 0) {
    Workspace ws(aar_gemm_f32_workspace_bytes(AAR_GEMM_NT, M, N, K));
    check_status(aar_gemm_f32_bias(AAR_GEMM_NT, M, N, K, fp(x), fp(w), fp(b), fp(out), ws.data(), ws.bytes(),
                                   current_stream()),
                 "linear");
  }
  if (x.shape.size() == 2) return out;
  std::vector<int64_t> out_shape(x.shape.begin(), x.shape.end() - 1);
  out_shape.push_back(N);
  return as_view(out, std::move(out_shape));
}

// dx = g W, dW = g^T x (MatmulABTFunction) and db = column sums of g
// (AddBiasFunction), the same kernels as the two-op composition.
// A linear layer's dW = G^T X and db = colsum(G) (G [rows, N], X [rows, K],
// contiguous): one pass of aar_gemm_f32_colsum_a over G where it takes the
// product's plan, else the product and aar_colsum_f32 (the same values).
std::pair<Tensor, Tensor> weight_bias_grads(const Tensor& g2, const Tensor& x2, const char* what) {
  const int64_t rows = g2.shape[0], N = g2.shape[1], K = x2.shape[1];
  Tensor db = Tensor::empty({N}, DType::Fp32, Device::CUDA);
  {
    Tensor dw = Tensor::empty({N, K}, DType::Fp32, Device::CUDA);
    Workspace ws(aar_gemm_f32_colsum_a_workspace_bytes(AAR_GEMM_TN, N, K, rows));
    const int rc = aar_gemm_f32_colsum_a(AAR_GEMM_TN, N, K, rows, fp(g2), fp(x2), fp(dw), fp(db), ws.data(),
                                         ws.bytes(), current_stream());
    if (rc != AAR_EUNSUPPORTED) {
      check_status(rc, what);
      return {dw, db};
    }
  }
  Workspace ws(aar_colsum_workspace_bytes(rows, N));
  check_status(aar_colsum_f32(fp(g2), fp(db), rows, N, ws.data(), ws.bytes(), current_stream()), what);
  return {matmul_at_b_no_grad(g2, x2), db};
}

class LinearFunction : public Function {
 public:
  Tensor saved_x, saved_w;
  std::vector<Tensor> backward(const Tensor& g) override {
    Tensor gc = as_contig(g);
    const int64_t N = saved_w.shape[0], K = saved_w.shape[1];  // linear() routes N == 0 and K == 0 elsewhere
    const int64_t rows = static_cast<int64_t>(saved_x.numel()) / K;
    auto [dw, db] = weight_bias_grads(as_view(gc, {rows, N}), as_view(saved_x, {rows, K}), "linear backward");
    return {matmul_no_grad(gc, saved_w), dw, db};
  }
  const char* name() const override { return "LinearFunction"; }
};

// -------------------------------------------------------------- softmax

Tensor softmax_no_grad(const Tensor& x) {
  if (x.device == Device::CPU) throw_cpu_compute("softmax");
  Tensor out = Tensor::empty(x.shape, x.dtype, x.device);
  const int64_t last = x.shape.back();
  const int64_t outer = static_cast<int64_t>(x.numel()) / last;
  check_status(aar_softmax_fwd_f32(fp(x), fp(out), outer, last, current_stream()), "softmax");
  return out;
}

Tensor softmax_backward_no_grad(const Tensor& g, const Tensor& y) {
  if (g.device == Device::CPU) throw_cpu_compute("softmax backward");
  Tensor gc = as_contig(g);
  Tensor dx = Tensor::empty(gc.shape, gc.dtype, gc.device);
  const int64_t last = gc.shape.back();
  const int64_t outer = static_cast<int64_t>(gc.numel()) / last;
  check_status(aar_softmax_bwd_f32(fp(gc), fp(y), fp(dx), outer, last, current_stream()),
               "softmax backward");
  return dx;
}

class SoftmaxFunction : public Function {
 public:
  Tensor saved_y;
  std::vector<Tensor> backward(const Tensor& g) override { return {softmax_backward_no_grad(g, saved_y)}; }
  const char* name() const override { return "SoftmaxFunction"; }
};

// ------------------------------------------------------------- layernorm

// A layernorm input that also feeds a residual connection (x + f(LN(x)), the
// pre-norm block) has a gradient fan-in: the residual's gradient arrives
// first and the layernorm's is added to it.  The backward takes that held
// gradient into its kernel (dx = held + value, aar_layernorm_bwd_acc_f32),
// the same fp32 sum as add_grads(held, dx) without the separate add pass.
class LayerNormFunction : public Function {
 public:
  Tensor saved_x, saved_w, saved_mean, saved_rstd;
  std::vector<Tensor> backward(const Tensor& grad_y) override { return run(grad_y, nullptr); }
  bool fuses_fan_in() const override { return true; }
  std::vector<Tensor> backward_into(const Tensor& grad_y, const std::vector<const Tensor*>& held,
                                    std::vector<bool>& summed) override {
    summed.assign(inputs.size(), false);
    const Tensor* h = held.empty() ? nullptr : held[0];
    if (h && h->shape == saved_x.shape && h->dtype == DType::Fp32 && h->device == Device::CUDA &&
        h->is_contiguous()) {
      summed[0] = true;
      return run(grad_y, h);
    }
    return run(grad_y, nullptr);
  }
  const char* name() const override { return "LayerNormFunction"; }

 private:
  std::vector<Tensor> run(const Tensor& grad_y, const Tensor* addend) {
    if (saved_x.device == Device::CPU) throw_cpu_compute("layernorm backward");
    Tensor gy = as_contig(grad_y);
    Tensor dx = Tensor::empty(saved_x.shape, saved_x.dtype, saved_x.device);
    Tensor dw = Tensor::empty(saved_w.shape, saved_w.dtype, saved_w.device);
    Tensor db = Tensor::empty(saved_w.shape, saved_w.dtype, saved_w.device);
    const int64_t last = saved_x.shape.back();
    const int64_t outer = static_cast<int64_t>(saved_x.numel()) / last;
    Workspace ws(aar_layernorm_bwd_workspace_bytes(outer, last));
    if (addend) {
      check_status(aar_layernorm_bwd_acc_f32(fp(gy), fp(saved_x), fp(saved_w), fp(saved_mean), fp(saved_rstd),
                                             fp(*addend), fp(dx), fp(dw), fp(db), outer, last, ws.data(),
                                             ws.bytes(), current_stream()),
                   "layernorm backward");
    } else {
      check_status(aar_layernorm_bwd_f32(fp(gy), fp(saved_x), fp(saved_w), fp(saved_mean), fp(saved_rstd),
                                         fp(dx), fp(dw), fp(db), outer, last, ws.data(), ws.bytes(),
                                         current_stream()),
                   "layernorm backward");
    }
    return {dx, dw, db};
  }
};

// ------------------------------------------------------------- attention

// A [B, H, T, d] view as the kernels take it: element (b, h, t, c) at
// data[b*sb + h*sh + t*st + c].  Leading dims of a [..., T, d] tensor fold
// into (B, H) = (prod(shape[:-3]), shape[-3]) when the folded dims are
// uniformly strided; otherwise (or if d is not unit-stride) the tensor is
// made contiguous first.
struct FlashView {
  Tensor t;  // the tensor the pointer refers to (keeps storage alive)
  int64_t s[3];
};

bool fold_strides(const Tensor& t, int64_t out[3]) {
  const size_t r = t.shape.size();
  if (t.strides[r - 1] != 1) return false;
  out[1] = t.strides[r - 3];
  out[2] = t.strides[r - 2];
  // Fold dims [0, r-3) into one batch dim: the non-trivial ones must nest
  // (stride of dim i = stride of the next inner one x its extent).
  int64_t sb = 0, span = 0;
  bool have = false;
  for (size_t i = r - 3; i-- > 0;) {
    if (t.shape[i] == 1) continue;
    if (!have) {
      sb = t.strides[i];
      span = t.shape[i];
      have = true;
      continue;
    }
    if (t.strides[i] != sb * span) return false;
    span *= t.shape[i];
  }
  out[0] = sb;
  return true;
}

FlashView flash_view(const Tensor& t) {
  FlashView v{t, {0, 0, 0}};
  if (!fold_strides(t, v.s)) {
    v.t = contiguous(t);
    fold_strides(v.t, v.s);
  }
  return v;
}

void flash_dims(const Tensor& t, int64_t& B, int64_t& H, int64_t& T, int64_t& d) {
  const size_t r = t.shape.size();
  d = t.shape[r - 1];
  T = t.shape[r - 2];
  H = t.shape[r - 3];
  B = 1;
  for (size_t i = 0; i + 3 < r; ++i) B *= t.shape[i];
}

void put3(int64_t* dst, const int64_t* s) {
  dst[0] = s[0];
  dst[1] = s[1];
  dst[2] = s[2];
}

class FlashAttentionFunction : public Function {
 public:
  FlashView q, k, v;
  Tensor saved_o, saved_lse;
  bool causal = false;
  float scale_factor = 1.0f;
  std::vector<Tensor> backward(const Tensor& grad_output) override {
    FlashView go = flash_view(grad_output);
    const Tensor& shp = q.t;
    Tensor dq = Tensor::empty(shp.shape, shp.dtype, shp.device);
    Tensor dk = Tensor::empty(shp.shape, shp.dtype, shp.device);
    Tensor dv = Tensor::empty(shp.shape, shp.dtype, shp.device);
    int64_t B, H, T, d;
    flash_dims(shp, B, H, T, d);
    int64_t st[24];
    int64_t oc[3], dc[3];
    fold_strides(saved_o, oc);
    fold_strides(dq, dc);
    put3(st, q.s);
    put3(st + 3, k.s);
    put3(st + 6, v.s);
    put3(st + 9, oc);
    put3(st + 12, go.s);
    put3(st + 15, dc);
    put3(st + 18, dc);
    put3(st + 21, dc);
    Workspace ws = flash_bwd_workspace(B * H, T, d, causal);
    check_status(aar_flash_bwd_strided_f32(fp(q.t), fp(k.t), fp(v.t), fp(saved_o), fp(saved_lse), fp(go.t),
                                           fp(dq), fp(dk), fp(dv), B, H, T, d, st, causal ? 1 : 0, scale_factor,
                                           ws.data(), ws.bytes(), current_stream()),
                 "flash_attention backward");
    return {dq, dk, dv};
  }
  const char* name() const override { return "FlashAttentionFunction"; }
};

void flash_check(const Tensor& q, const Tensor& k, const Tensor& v) {
  if (q.dtype != DType::Fp32 || k.dtype != DType::Fp32 || v.dtype != DType::Fp32) {
    throw std::invalid_argument("flash_attention: only Fp32 supported");
  }
  if (q.device != k.device || q.device != v.device) {
    throw std::invalid_argument("flash_attention: device mismatch");
  }
  if (q.shape.size() < 3 || k.shape.size() < 3 || v.shape.size() < 3) {
    throw std::invalid_argument("flash_attention: need at least 3 dims [..., T, d]");
  }
  if (q.shape != k.shape || q.shape != v.shape) {
    throw std::invalid_argument("flash_attention: q, k, v must share shape");
  }
}

// Forward on (possibly strided) views; O and lse are contiguous.
std::tuple<Tensor, Tensor> flash_forward_device(const FlashView& q, const FlashView& k, const FlashView& v,
                                                bool causal, float s) {
  int64_t B, H, T, d;
  flash_dims(q.t, B, H, T, d);
  if (d > 128) throw std::invalid_argument("flash_attention: d_head exceeds D_MAX (128)");
  std::vector<int64_t> lse_shape(q.t.shape.begin(), q.t.shape.end() - 1);
  Tensor out = Tensor::empty(q.t.shape, q.t.dtype, q.t.device);
  Tensor lse = Tensor::empty(lse_shape, q.t.dtype, q.t.device);
  int64_t st[12], oc[3];
  fold_strides(out, oc);
  put3(st, q.s);
  put3(st + 3, k.s);
  put3(st + 6, v.s);
  put3(st + 9, oc);
  Workspace ws = flash_fwd_workspace(B * H, T, d, causal);
  check_status(aar_flash_fwd_strided_f32(fp(q.t), fp(k.t), fp(v.t), fp(out), fp(lse), B, H, T, d, st,
                                         causal ? 1 : 0, s, ws.data(), ws.bytes(), current_stream()),
               "flash_attention");
  return {out, lse};
}

// Fused attention over a packed projection qkv [..., T, 3*D] (q, k, v are
// the column blocks [0, D), [D, 2D), [2D, 3D), each split into H heads of
// d = D/H): O [..., T, D] with O[t][h*d + c] = attention of head h.  The same
// math as flash_attention on the per-head views (nn.py's MultiHeadAttention
// composition, aargrad/nn.py:177-192), without materialising the views: the
// kernels read q/k/v in place, write O in [T, H, d] order and the backward
// writes dq/dk/dv straight into one packed gradient.
class FlashQKVFunction : public Function {
 public:
  Tensor saved_qkv, saved_o, saved_lse;
  int64_t B = 0, H = 0, T = 0, d = 0;
  bool causal = false;
  float scale_factor = 1.0f;
  std::vector<Tensor> backward(const Tensor& grad_output) override {
    Tensor go = as_contig(grad_output);
    Tensor dqkv = Tensor::empty(saved_qkv.shape, saved_qkv.dtype, saved_qkv.device);
    const int64_t D = H * d;
    const int64_t pk[3] = {T * 3 * D, d, 3 * D};  // packed q/k/v/dq/dk/dv
    const int64_t po[3] = {T * D, d, D};          // O and dO
    int64_t st[24];
    for (int i : {0, 1, 2, 5, 6, 7}) put3(st + 3 * i, pk);
    put3(st + 9, po);
    put3(st + 12, po);
    float* g = fp(dqkv);
    const float* x = fp(saved_qkv);
    Workspace ws = flash_bwd_workspace(B * H, T, d, causal);
    check_status(aar_flash_bwd_strided_f32(x, x + D, x + 2 * D, fp(saved_o), fp(saved_lse), fp(go), g, g + D,
                                           g + 2 * D, B, H, T, d, st, causal ? 1 : 0, scale_factor, ws.data(),
                                           ws.bytes(), current_stream()),
                 "flash_attention_qkv backward");
    return {dqkv};
  }
  const char* name() const override { return "FlashQKVFunction"; }
};


// ------------------------------------------------------------------ add

void check_binary(const Tensor& a, const Tensor& b, const char* op) {
  if (a.shape != b.shape) throw std::invalid_argument(std::string(op) + ": shape mismatch");
  if (a.dtype != b.dtype) throw std::invalid_argument(std::string(op) + ": dtype mismatch");
  if (a.device != b.device) throw std::invalid_argument(std::string(op) + ": device mismatch");
  if (a.dtype != DType::Fp32) throw std::invalid_argument(std::string(op) + ": only Fp32 supported");
}

class AddFunction : public Function {
 public:
  std::vector<Tensor> backward(const Tensor& g) override { return {g, g}; }
  const char* name() const override { return "AddFunction"; }
};

Tensor add_no_grad(const Tensor& a, const Tensor& b) {
  if (a.device == Device::CPU) throw_cpu_compute("add");
  Tensor out = Tensor::empty(a.shape, a.dtype, a.device);
  check_status(aar_add_f32(fp(a), fp(b), fp(out), (int64_t)a.numel(), current_stream()), "add");
  return out;
}

}  // namespace

// ======================================================================= API

Tensor make_view(const Tensor& src, std::vector<int64_t> shape, std::vector<int64_t> strides,
                 int64_t storage_offset) {
  Tensor v;
  v.shape = std::move(shape);
  v.strides = std::move(strides);
  v.storage_offset = storage_offset;
  v.dtype = src.dtype;
  v.device = src.device;
  v.storage = src.storage;
  return v;
}

void copy_strided_to_contiguous(const Tensor& src, Tensor& dst) {
  if (src.shape != dst.shape) throw std::runtime_error("copy_strided_to_contiguous: shape mismatch");
  if (src.dtype != dst.dtype || src.device != dst.device) {
    throw std::runtime_error("copy_strided_to_contiguous: dtype/device mismatch");
  }
  if (!dst.is_contiguous()) throw std::runtime_error("copy_strided_to_contiguous: dst must be contiguous");
  if (src.device == Device::CUDA) {
    device_strided_copy(src, dst, "copy_strided_to_contiguous");
    return;
  }
  copy_strided_to_contiguous_host(src, dst);
}

Tensor contiguous(const Tensor& x) {
  if (x.is_contiguous()) return x;
  Tensor out = Tensor::empty(x.shape, x.dtype, x.device);
  copy_strided_to_contiguous(x, out);
  if (!x.requires_grad) return out;
  auto fn = std::make_shared<ContiguousFunction>();
  fn->record_input(x);
  out.requires_grad = true;
  out.grad_fn = fn;
  return out;
}

Tensor reshape(const Tensor& x, std::vector<int64_t> new_shape) {
  auto resolved = resolve_new_shape(new_shape, x.numel());
  Tensor src = as_contig(x);
  Tensor out = make_view(src, resolved, compute_contiguous_strides(resolved), src.storage_offset);
  if (!x.requires_grad) return out;
  auto fn = std::make_shared<ReshapeFunction>();
  fn->record_input(x);
  fn->original_shape = x.shape;
  out.requires_grad = true;
  out.grad_fn = fn;
  return out;
}

Tensor transpose(const Tensor& x, int64_t dim_a, int64_t dim_b) {
  const int64_t ndim = static_cast<int64_t>(x.shape.size());
  if (dim_a < 0 || dim_a >= ndim || dim_b < 0 || dim_b >= ndim) {
    throw std::invalid_argument("transpose: dim out of range");
  }
  std::vector<int64_t> sh = x.shape, st = x.strides;
  std::swap(sh[dim_a], sh[dim_b]);
  std::swap(st[dim_a], st[dim_b]);
  Tensor out = make_view(x, sh, st, x.storage_offset);
  if (!x.requires_grad) return out;
  auto fn = std::make_shared<TransposeFunction>();
  fn->record_input(x);
  fn->dim_a = dim_a;
  fn->dim_b = dim_b;
  out.requires_grad = true;
  out.grad_fn = fn;
  return out;
}

Tensor slice(const Tensor& x, int64_t dim, int64_t start, int64_t end) {
  const int64_t ndim = static_cast<int64_t>(x.shape.size());
  if (dim < 0 || dim >= ndim) throw std::invalid_argument("slice: dim out of range");
  if (start < 0 || end > x.shape[dim] || start >= end) throw std::invalid_argument("slice: invalid range");
  std::vector<int64_t> sh = x.shape;
  sh[dim] = end - start;
  Tensor out = make_view(x, sh, x.strides, x.storage_offset + start * x.strides[dim]);
  if (!x.requires_grad) return out;
  auto fn = std::make_shared<SliceFunction>();
  fn->record_input(x);
  fn->original_shape = x.shape;
  fn->dim = dim;
  fn->start = start;
  fn->end = end;
  fn->dtype = x.dtype;
  fn->device = x.device;
  out.requires_grad = true;
  out.grad_fn = fn;
  return out;
}

Tensor squeeze(const Tensor& x, int64_t dim) {
  const int64_t ndim = static_cast<int64_t>(x.shape.size());
  if (dim < 0 || dim >= ndim) throw std::invalid_argument("squeeze: dim out of range");
  if (x.shape[dim] != 1) throw std::invalid_argument("squeeze: dim size must be 1");
  std::vector<int64_t> sh = x.shape, st = x.strides;
  const int64_t inserted_stride = st[dim];
  sh.erase(sh.begin() + dim);
  st.erase(st.begin() + dim);
  Tensor out = make_view(x, sh, st, x.storage_offset);
  if (!x.requires_grad) return out;
  auto fn = std::make_shared<SqueezeFunction>();
  fn->record_input(x);
  fn->dim = dim;
  fn->inserted_size_stride = inserted_stride;
  out.requires_grad = true;
  out.grad_fn = fn;
  return out;
}

Tensor unsqueeze(const Tensor& x, int64_t dim) {
  const int64_t ndim = static_cast<int64_t>(x.shape.size());
  if (dim < 0 || dim > ndim) throw std::invalid_argument("unsqueeze: dim out of range");
  std::vector<int64_t> sh = x.shape, st = x.strides;
  const int64_t new_stride = (dim < ndim) ? x.strides[dim] * x.shape[dim] : 1;
  sh.insert(sh.begin() + dim, 1);
  st.insert(st.begin() + dim, new_stride);
  Tensor out = make_view(x, sh, st, x.storage_offset);
  if (!x.requires_grad) return out;
  auto fn = std::make_shared<UnsqueezeFunction>();
  fn->record_input(x);
  fn->dim = dim;
  out.requires_grad = true;
  out.grad_fn = fn;
  return out;
}

Tensor matmul(const Tensor& a, const Tensor& b) {
  if (a.shape.size() < 2 || b.shape.size() != 2) {
    throw std::invalid_argument("matmul: LHS rank must be >= 2 and RHS must be 2D");
  }
  if (a.dtype != b.dtype) throw std::invalid_argument("matmul: dtype mismatch");
  if (a.device != b.device) throw std::invalid_argument("matmul: device mismatch");
  if (a.dtype != DType::Fp32) throw std::invalid_argument("matmul: only Fp32 supported");
  if (b.shape[0] != a.shape.back()) throw std::invalid_argument("matmul: inner dimensions mismatch");
  return with_matmul_grad<MatmulFunction>(as_contig(a), as_contig(b), matmul_no_grad);
}

Tensor matmul_a_bt(const Tensor& a, const Tensor& b) {
  if (a.shape.size() < 2 || b.shape.size() != 2) {
    throw std::invalid_argument("matmul_a_bt: LHS rank must be >= 2 and RHS must be 2D");
  }
  if (a.dtype != b.dtype || a.device != b.device) {
    throw std::invalid_argument("matmul_a_bt: dtype/device mismatch");
  }
  if (a.dtype != DType::Fp32) throw std::invalid_argument("matmul_a_bt: only Fp32 supported");
  if (a.shape.back() != b.shape[1]) throw std::invalid_argument("matmul_a_bt: contraction dim mismatch");
  return with_matmul_grad<MatmulABTFunction>(as_contig(a), as_contig(b), matmul_a_bt_no_grad);
}

Tensor linear(const Tensor& x, const Tensor& w, const Tensor& b) {
  // The checks (and messages) of matmul_a_bt followed by those of add_bias.
  if (x.shape.size() < 2 || w.shape.size() != 2) {
    throw std::invalid_argument("matmul_a_bt: LHS rank must be >= 2 and RHS must be 2D");
  }
  if (x.dtype != w.dtype || x.device != w.device) {
    throw std::invalid_argument("matmul_a_bt: dtype/device mismatch");
  }
  if (x.dtype != DType::Fp32) throw std::invalid_argument("matmul_a_bt: only Fp32 supported");
  if (x.shape.back() != w.shape[1]) throw std::invalid_argument("matmul_a_bt: contraction dim mismatch");
  if (b.shape.size() != 1) throw std::invalid_argument("add_bias: bias must be 1-D");
  if (w.shape[0] != b.shape[0]) throw std::invalid_argument("add_bias: bias size must match x's last dim");
  if (b.dtype != DType::Fp32) throw std::invalid_argument("add_bias: only Fp32 supported");
  if (x.device != b.device) throw std::invalid_argument("add_bias: device mismatch");
  // An empty contraction is the bias broadcast, not a product, and a layer
  // with no outputs has nothing to compute: both take the two-op path.
  if (x.shape.back() == 0 || w.shape[0] == 0) return add_bias(matmul_a_bt(x, w), b);
  Tensor xc = as_contig(x), wc = as_contig(w), bc = as_contig(b);
  if (!xc.requires_grad && !wc.requires_grad && !bc.requires_grad) return linear_no_grad(xc, wc, bc);
  auto fn = std::make_shared<LinearFunction>();
  fn->record_input(xc);
  fn->record_input(wc);
  fn->record_input(bc);
  fn->saved_x = xc;
  fn->saved_w = wc;
  Tensor out = linear_no_grad(xc, wc, bc);
  out.requires_grad = true;
  out.grad_fn = fn;
  return out;
}

// The feed-forward composition linear(relu(linear(x, W1, b1)), W2, b2) of the
// GPT block (add_bias(matmul_a_bt(.)) with a relu between, aargrad/nn.py:101-122)
// with bias + relu in the first GEMM's epilogue.  The backward is the
// composition's, its relu mask taken from the saved output h (positive exactly
// where the relu's input is): same values and gradients, bit for bit.
class MlpReluFunction : public Function {
 public:
  Tensor saved_x, saved_w1, saved_w2, saved_h;  // x and h as [rows, features]
  // h > 0 as bits from the first GEMM's epilogue (aar_gemm_f32_bias_relu_bits),
  // or null where that entry point did not take the product's plan
  std::shared_ptr<Workspace> saved_bits;
  std::vector<int64_t> x_shape;
  std::vector<Tensor> backward(const Tensor& g) override {
    const int64_t N2 = saved_w2.shape[0], H = saved_w1.shape[0];
    const int64_t rows = saved_h.shape[0];
    Tensor gc = as_view(as_contig(g), {rows, N2});
    auto [dw2, db2] = weight_bias_grads(gc, saved_h, "mlp backward");
    // dh = relu_backward(g W2): with the mask bits, one GEMM applies the mask
    // in its epilogue (aar_gemm_f32_mask_bits_colsum without column sums),
    // else the plain GEMM and the mask pass.  db1 = colsum(dh) comes with dW1
    // (dh is that product's A operand), bit for bit aar_colsum_f32's.  (The
    // mask read as the relu's output in the epilogue, aar_gemm_f32_relu_mask,
    // measured slower than the separate pass: 212 against 172 + 62 us at
    // 16384 x 1536 x 384.)
    Tensor dh = Tensor::empty({rows, H}, DType::Fp32, Device::CUDA);
    bool masked = false;
    if (saved_bits) {
      const int rc = aar_gemm_f32_mask_bits_colsum(AAR_GEMM_NN, rows, H, N2, fp(gc), fp(saved_w2),
                                                   static_cast<const uint32_t*>(saved_bits->data()), fp(dh),
                                                   nullptr, nullptr, 0, current_stream());
      if (rc != AAR_EUNSUPPORTED) {
        check_status(rc, "mlp backward");
        masked = true;
      }
    }
    if (!masked) {
      Tensor dpost = matmul_no_grad(gc, saved_w2);
      check_status(aar_relu_bwd_f32(fp(dpost), fp(saved_h), fp(dh), rows * H, current_stream()), "mlp backward");
    }
    Tensor dx = as_view(matmul_no_grad(dh, saved_w1), x_shape);
    auto [dw1, db1] = weight_bias_grads(dh, saved_x, "mlp backward");
    return {dx, dw1, db1, dw2, db2};
  }
  const char* name() const override { return "MlpReluFunction"; }
};

// h = max(0, x W1^T + b1) (x2 [rows, d], h [rows, H]).  For a backward
// (want_bits) also h > 0 as bits, returned for MlpReluFunction::saved_bits,
// or null where aar_gemm_f32_bias_relu_bits does not take the product's plan
// (h is then aar_gemm_f32_bias_relu's, the same values).
std::shared_ptr<Workspace> mlp_hidden(const Tensor& x2, const Tensor& w1c, const Tensor& b1c, Tensor& h,
                                      bool want_bits) {
  const int64_t rows = h.shape[0], H = h.shape[1], d = x2.shape[1];
  Workspace ws(aar_gemm_f32_workspace_bytes(AAR_GEMM_NT, rows, H, d));
  if (want_bits) {
    auto bits = std::make_shared<Workspace>(static_cast<size_t>((rows + 31) / 32) * static_cast<size_t>(H) *
                                            sizeof(uint32_t));
    const int rc = aar_gemm_f32_bias_relu_bits(AAR_GEMM_NT, rows, H, d, fp(x2), fp(w1c), fp(b1c), fp(h),
                                               static_cast<uint32_t*>(bits->data()), ws.data(), ws.bytes(),
                                               current_stream());
    if (rc != AAR_EUNSUPPORTED) {
      check_status(rc, "linear");
      return bits;
    }
  }
  check_status(aar_gemm_f32_bias_relu(AAR_GEMM_NT, rows, H, d, fp(x2), fp(w1c), fp(b1c), fp(h), ws.data(),
                                      ws.bytes(), current_stream()),
               "linear");
  return nullptr;
}

Tensor mlp_relu(const Tensor& x, const Tensor& w1, const Tensor& b1, const Tensor& w2, const Tensor& b2) {
  if (w1.shape.size() != 2 || w2.shape.size() != 2 || x.shape.empty() || w1.shape[0] == 0 ||
      w2.shape[0] == 0 || x.shape.back() == 0) {
    return linear(relu(linear(x, w1, b1)), w2, b2);  // the composition's checks and edge cases
  }
  // The checks (and messages) of both layers' matmul_a_bt and add_bias.
  if (x.shape.size() < 2 || x.dtype != DType::Fp32 || w1.dtype != DType::Fp32 || w2.dtype != DType::Fp32 ||
      b1.dtype != DType::Fp32 || b2.dtype != DType::Fp32 || x.device != w1.device || x.device != w2.device ||
      x.device != b1.device || x.device != b2.device || x.shape.back() != w1.shape[1] ||
      w2.shape[1] != w1.shape[0] || b1.shape.size() != 1 || b2.shape.size() != 1 || b1.shape[0] != w1.shape[0] ||
      b2.shape[0] != w2.shape[0]) {
    return linear(relu(linear(x, w1, b1)), w2, b2);  // raises as the composition does
  }
  if (x.device == Device::CPU) throw_cpu_compute("linear");
  Tensor xc = as_contig(x), w1c = as_contig(w1), b1c = as_contig(b1), w2c = as_contig(w2), b2c = as_contig(b2);
  const int64_t d = x.shape.back(), H = w1.shape[0], N2 = w2.shape[0];
  const int64_t rows = static_cast<int64_t>(x.numel()) / d;
  Tensor x2 = as_view(xc, {rows, d});
  Tensor h = Tensor::empty({rows, H}, DType::Fp32, Device::CUDA);
  const bool grad =
      xc.requires_grad || w1c.requires_grad || b1c.requires_grad || w2c.requires_grad || b2c.requires_grad;
  std::shared_ptr<Workspace> bits;
  if (h.numel() != 0) bits = mlp_hidden(x2, w1c, b1c, h, grad);
  std::vector<int64_t> out_shape(x.shape.begin(), x.shape.end() - 1);
  out_shape.push_back(N2);
  Tensor out = as_view(linear_no_grad(h, w2c, b2c), out_shape);
  if (!grad) return out;
  auto fn = std::make_shared<MlpReluFunction>();
  for (const Tensor* t : {&xc, &w1c, &b1c, &w2c, &b2c}) fn->record_input(*t);
  fn->saved_x = x2;
  fn->saved_w1 = w1c;
  fn->saved_w2 = w2c;
  fn->saved_h = h;
  fn->saved_bits = bits;
  fn->x_shape = x.shape;
  out.requires_grad = true;
  out.grad_fn = fn;
  return out;
}

// r + a W^T: the attention output projection of a pre-norm block (bias-free,
// python/shakespeare/scripts/model.py:12) with its residual add, as one GEMM
// whose epilogue adds r (aar_gemm_f32_add; bit for bit matmul_a_bt followed
// by add).  The node stands for the pair add(r, matmul_a_bt(a, W)): its
// inputs are (r, a, W) in that order, so the autograd walk visits them as it
// visits the pair's, and its backward returns the pair's gradients: g for r,
// g W for a and g^T a for W, from the same kernels.
class LinearResidualFunction : public Function {
 public:
  Tensor saved_a, saved_w;  // a as [rows, K]
  std::vector<int64_t> a_shape;
  std::vector<Tensor> backward(const Tensor& g) override {
    const int64_t rows = saved_a.shape[0], N = saved_w.shape[0];
    Tensor gc = as_view(as_contig(g), {rows, N});
    return {g, as_view(matmul_no_grad(gc, saved_w), a_shape), matmul_at_b_no_grad(gc, saved_a)};
  }
  const char* name() const override { return "LinearResidualFunction"; }
};

Tensor linear_residual(const Tensor& r, const Tensor& a, const Tensor& w) {
  if (w.shape.size() != 2 || a.shape.size() < 2 || a.shape.back() != w.shape[1] || a.shape.back() == 0 ||
      w.shape[0] == 0 || a.dtype != DType::Fp32 || w.dtype != DType::Fp32 || r.dtype != DType::Fp32 ||
      a.device != w.device || r.device != a.device) {
    return add(r, matmul_a_bt(a, w));  // the composition's checks, messages and edge cases
  }
  std::vector<int64_t> out_shape(a.shape.begin(), a.shape.end() - 1);
  out_shape.push_back(w.shape[0]);
  if (r.shape != out_shape) return add(r, matmul_a_bt(a, w));  // raises as add does
  if (a.device == Device::CPU) throw_cpu_compute("matmul_a_bt");
  Tensor rc = as_contig(r), ac = as_contig(a), wc = as_contig(w);
  const int64_t K = a.shape.back(), N = w.shape[0];
  const int64_t rows = static_cast<int64_t>(a.numel()) / K;
  Tensor out = Tensor::empty(out_shape, DType::Fp32, Device::CUDA);
  if (out.numel() != 0) {
    Workspace ws(aar_gemm_f32_workspace_bytes(AAR_GEMM_NT, rows, N, K));
    check_status(aar_gemm_f32_add(AAR_GEMM_NT, rows, N, K, fp(ac), fp(wc), fp(rc), fp(out), ws.data(), ws.bytes(),
                                  current_stream()),
                 "matmul_a_bt");
  }
  if (!rc.requires_grad && !ac.requires_grad && !wc.requires_grad) return out;
  auto fn = std::make_shared<LinearResidualFunction>();
  fn->record_input(rc);
  fn->record_input(ac);
  fn->record_input(wc);
  fn->saved_a = as_view(ac, {rows, K});
  fn->saved_w = wc;
  fn->a_shape = a.shape;
  out.requires_grad = true;
  out.grad_fn = fn;
  return out;
}

// r + mlp_relu(x, W1, b1, W2, b2): the MLP branch of a pre-norm block with its
// residual add in the second GEMM's epilogue (aar_gemm_f32_bias_add; bit for
// bit the mlp_relu + add composition).  Inputs (r, x, W1, b1, W2, b2), in the
// order the pair add(r, mlp_relu(.)) presents them to the autograd walk; the
// backward is MlpReluFunction's plus g for r.
class MlpReluResidualFunction : public MlpReluFunction {
 public:
  std::vector<Tensor> backward(const Tensor& g) override {
    std::vector<Tensor> grads = MlpReluFunction::backward(g);
    grads.insert(grads.begin(), g);
    return grads;
  }
  const char* name() const override { return "MlpReluResidualFunction"; }
};

Tensor mlp_relu_residual(const Tensor& r, const Tensor& x, const Tensor& w1, const Tensor& b1, const Tensor& w2,
                         const Tensor& b2) {
  const bool shapes_ok = w1.shape.size() == 2 && w2.shape.size() == 2 && x.shape.size() >= 2 && w1.shape[0] != 0 &&
                         w2.shape[0] != 0 && x.shape.back() != 0 && x.shape.back() == w1.shape[1] &&
                         w2.shape[1] == w1.shape[0] && b1.shape.size() == 1 && b2.shape.size() == 1 &&
                         b1.shape[0] == w1.shape[0] && b2.shape[0] == w2.shape[0];
  const bool types_ok = x.dtype == DType::Fp32 && w1.dtype == DType::Fp32 && w2.dtype == DType::Fp32 &&
                        b1.dtype == DType::Fp32 && b2.dtype == DType::Fp32 && r.dtype == DType::Fp32 &&
                        x.device == w1.device && x.device == w2.device && x.device == b1.device &&
                        x.device == b2.device && x.device == r.device;
  std::vector<int64_t> out_shape(x.shape.begin(), x.shape.end() - 1);
  if (shapes_ok) out_shape.push_back(w2.shape[0]);
  if (!shapes_ok || !types_ok || r.shape != out_shape) {
    return add(r, mlp_relu(x, w1, b1, w2, b2));  // the composition's checks, messages and edge cases
  }
  if (x.device == Device::CPU) throw_cpu_compute("linear");
  Tensor rc = as_contig(r), xc = as_contig(x), w1c = as_contig(w1), b1c = as_contig(b1), w2c = as_contig(w2),
         b2c = as_contig(b2);
  const int64_t d = x.shape.back(), H = w1.shape[0], N2 = w2.shape[0];
  const int64_t rows = static_cast<int64_t>(x.numel()) / d;
  Tensor x2 = as_view(xc, {rows, d});
  Tensor h = Tensor::empty({rows, H}, DType::Fp32, Device::CUDA);
  Tensor out = Tensor::empty(out_shape, DType::Fp32, Device::CUDA);
  const bool grad = rc.requires_grad || xc.requires_grad || w1c.requires_grad || b1c.requires_grad ||
                    w2c.requires_grad || b2c.requires_grad;
  std::shared_ptr<Workspace> bits;
  if (h.numel() != 0) {
    bits = mlp_hidden(x2, w1c, b1c, h, grad);
    Workspace ws2(aar_gemm_f32_workspace_bytes(AAR_GEMM_NT, rows, N2, H));
    check_status(aar_gemm_f32_bias_add(AAR_GEMM_NT, rows, N2, H, fp(h), fp(w2c), fp(b2c), fp(rc), fp(out),
                                       ws2.data(), ws2.bytes(), current_stream()),
                 "linear");
  }
  if (!grad) return out;
  auto fn = std::make_shared<MlpReluResidualFunction>();
  for (const Tensor* t : {&rc, &xc, &w1c, &b1c, &w2c, &b2c}) fn->record_input(*t);
  fn->saved_x = x2;
  fn->saved_w1 = w1c;
  fn->saved_w2 = w2c;
  fn->saved_h = h;
  fn->saved_bits = bits;
  fn->x_shape = x.shape;
  out.requires_grad = true;
  out.grad_fn = fn;
  return out;
}

Tensor matmul_at_b(const Tensor& a, const Tensor& b) {
  if (a.shape.size() != 2 || b.shape.size() != 2) {
    throw std::invalid_argument("matmul_at_b: inputs must be 2D");
  }
  if (a.dtype != b.dtype || a.device != b.device) {
    throw std::invalid_argument("matmul_at_b: dtype/device mismatch");
  }
  if (a.dtype != DType::Fp32) throw std::invalid_argument("matmul_at_b: only Fp32 supported");
  if (a.shape[0] != b.shape[0]) throw std::invalid_argument("matmul_at_b: contraction dim mismatch");
  return with_matmul_grad<MatmulATBFunction>(as_contig(a), as_contig(b), matmul_at_b_no_grad);
}

Tensor softmax(const Tensor& x) {
  if (x.shape.empty()) throw std::invalid_argument("softmax: input must have at least 1 dim");
  if (x.dtype != DType::Fp32) throw std::invalid_argument("softmax: only Fp32 supported");
  if (x.shape.back() == 0) throw std::invalid_argument("softmax: last dim must be > 0");
  Tensor xc = as_contig(x);
  if (!xc.requires_grad) return softmax_no_grad(xc);
  auto fn = std::make_shared<SoftmaxFunction>();
  fn->record_input(xc);
  Tensor out = softmax_no_grad(xc);
  fn->saved_y = out;
  out.requires_grad = true;
  out.grad_fn = fn;
  return out;
}

Tensor layernorm(const Tensor& x, const Tensor& weight, const Tensor& bias, float eps) {
  if (x.shape.empty()) throw std::invalid_argument("layernorm: input must have at least 1 dim");
  if (x.dtype != DType::Fp32) throw std::invalid_argument("layernorm: only Fp32 supported");
  const int64_t last = x.shape.back();
  if (last == 0) throw std::invalid_argument("layernorm: last dim must be > 0");
  if (weight.shape.size() != 1 || weight.shape[0] != last) {
    throw std::invalid_argument("layernorm: weight must be 1D matching last dim");
  }
  if (bias.shape.size() != 1 || bias.shape[0] != last) {
    throw std::invalid_argument("layernorm: bias must be 1D matching last dim");
  }
  if (weight.dtype != DType::Fp32 || bias.dtype != DType::Fp32) {
    throw std::invalid_argument("layernorm: weight/bias must be Fp32");
  }
  if (x.device != weight.device || x.device != bias.device) {
    throw std::invalid_argument("layernorm: device mismatch");
  }
  if (eps <= 0.0f) throw std::invalid_argument("layernorm: eps must be > 0");

  Tensor xc = as_contig(x), wc = as_contig(weight), bc = as_contig(bias);
  if (xc.device == Device::CPU) throw_cpu_compute("layernorm");
  const int64_t outer = static_cast<int64_t>(xc.numel()) / last;
  Tensor y = Tensor::empty(xc.shape, xc.dtype, xc.device);
  if (!xc.requires_grad && !wc.requires_grad && !bc.requires_grad) {
    check_status(aar_layernorm_fwd_f32(fp(xc), fp(wc), fp(bc), fp(y), nullptr, nullptr, outer, last, eps,
                                       current_stream()),
                 "layernorm");
    return y;
  }
  Tensor mean = Tensor::empty({outer}, xc.dtype, xc.device);
  Tensor rstd = Tensor::empty({outer}, xc.dtype, xc.device);
  check_status(aar_layernorm_fwd_f32(fp(xc), fp(wc), fp(bc), fp(y), fp(mean), fp(rstd), outer, last, eps,
                                     current_stream()),
               "layernorm");
  auto fn = std::make_shared<LayerNormFunction>();
  fn->record_input(xc);
  fn->record_input(wc);
  fn->record_input(bc);
  fn->saved_x = xc;
  fn->saved_w = wc;
  fn->saved_mean = mean;
  fn->saved_rstd = rstd;
  y.requires_grad = true;
  y.grad_fn = fn;
  return y;
}

Tensor flash_attention(const Tensor& q, const Tensor& k, const Tensor& v, bool causal) {
  flash_check(q, k, v);
  if (q.device == Device::CPU) throw_cpu_compute("flash_attention");
  FlashView qv = flash_view(q), kv = flash_view(k), vv = flash_view(v);
  const float s = 1.0f / std::sqrt(static_cast<float>(q.shape.back()));
  auto [out, lse] = flash_forward_device(qv, kv, vv, causal, s);
  if (!q.requires_grad && !k.requires_grad && !v.requires_grad) return out;
  auto fn = std::make_shared<FlashAttentionFunction>();
  fn->record_input(q);
  fn->record_input(k);
  fn->record_input(v);
  fn->q = qv;
  fn->k = kv;
  fn->v = vv;
  fn->saved_o = out;
  fn->saved_lse = lse;
  fn->causal = causal;
  fn->scale_factor = s;
  out.requires_grad = true;
  out.grad_fn = fn;
  return out;
}

std::tuple<Tensor, Tensor> flash_attention_fwd_lse(const Tensor& q, const Tensor& k, const Tensor& v,
                                                   bool causal) {
  flash_check(q, k, v);
  if (q.device == Device::CPU) throw_cpu_compute("flash_attention");
  const float s = 1.0f / std::sqrt(static_cast<float>(q.shape.back()));
  return flash_forward_device(flash_view(q), flash_view(k), flash_view(v), causal, s);
}

Tensor flash_attention_qkv(const Tensor& qkv, int64_t n_heads, bool causal) {
  if (qkv.dtype != DType::Fp32) throw std::invalid_argument("flash_attention_qkv: only Fp32 supported");
  if (qkv.shape.size() < 2) throw std::invalid_argument("flash_attention_qkv: need [..., T, 3*D]");
  const int64_t D3 = qkv.shape.back();
  if (n_heads <= 0 || D3 % (3 * n_heads) != 0) {
    throw std::invalid_argument("flash_attention_qkv: last dim must be 3 * n_heads * d_head");
  }
  if (qkv.device == Device::CPU) throw_cpu_compute("flash_attention_qkv");
  Tensor x = as_contig(qkv);
  const int64_t D = D3 / 3, d = D / n_heads, T = x.shape[x.shape.size() - 2];
  if (d > 128) throw std::invalid_argument("flash_attention: d_head exceeds D_MAX (128)");
  int64_t B = 1;
  for (size_t i = 0; i + 2 < x.shape.size(); ++i) B *= x.shape[i];
  std::vector<int64_t> oshape(x.shape);
  oshape.back() = D;
  Tensor out = Tensor::empty(oshape, x.dtype, x.device);
  Tensor lse = Tensor::empty({B * n_heads, T}, x.dtype, x.device);
  const int64_t pk[3] = {T * 3 * D, d, 3 * D};
  const int64_t po[3] = {T * D, d, D};
  int64_t st[12];
  put3(st, pk);
  put3(st + 3, pk);
  put3(st + 6, pk);
  put3(st + 9, po);
  const float s = 1.0f / std::sqrt(static_cast<float>(d));
  const float* p = fp(x);
  Workspace ws = flash_fwd_workspace(B * n_heads, T, d, causal);
  check_status(aar_flash_fwd_strided_f32(p, p + D, p + 2 * D, fp(out), fp(lse), B, n_heads, T, d, st,
                                         causal ? 1 : 0, s, ws.data(), ws.bytes(), current_stream()),
               "flash_attention_qkv");
  if (!qkv.requires_grad) return out;
  auto fn = std::make_shared<FlashQKVFunction>();
  fn->record_input(qkv);
  fn->saved_qkv = x;
  fn->saved_o = out;
  fn->saved_lse = lse;
  fn->B = B;
  fn->H = n_heads;
  fn->T = T;
  fn->d = d;
  fn->causal = causal;
  fn->scale_factor = s;
  out.requires_grad = true;
  out.grad_fn = fn;
  return out;
}

Tensor add(const Tensor& a, const Tensor& b) {
  check_binary(a, b, "add");
  Tensor ac = as_contig(a), bc = as_contig(b);
  if (!ac.requires_grad && !bc.requires_grad) return add_no_grad(ac, bc);
  auto fn = std::make_shared<AddFunction>();
  fn->record_input(ac);
  fn->record_input(bc);
  Tensor out = add_no_grad(ac, bc);
  out.requires_grad = true;
  out.grad_fn = fn;
  return out;
}

}  // namespace aar
