// bmm family, apply_causal_mask and dropout on the device (the reference's
// non-flash attention path and regulariser).  Validation messages, exception
// types and autograd Functions follow:
//   cppsrc/ops/bmm.cpp:15-43 (checks), :177-209 (Functions), :212-268 (public ops)
//   cppsrc/ops/attention.cpp:14-21 (check), :65-90 (Function, public op)
//   cppsrc/ops/dropout.cpp:16-28 (seed counter), :45-92 (Function, public op)
#include <atomic>
#include <cmath>
#include <limits>
#include <random>

#include "aar_hip.h"
#include "ops.hpp"

namespace aar {

namespace {

const float* fp(const Tensor& t) { return static_cast<const float*>(t.data()); }
float* fp(Tensor& t) { return static_cast<float*>(t.data()); }

template <class Fn>
Tensor attach(std::shared_ptr<Fn> fn, Tensor out) {
  out.requires_grad = true;
  out.grad_fn = std::move(fn);
  return out;
}

// ---------------------------------------------------------------- bmm

void check_bmm_common(const Tensor& a, const Tensor& b, const char* op) {
  if (a.shape.size() < 2 || b.shape.size() < 2) throw std::invalid_argument(std::string(op) + ": rank must be >= 2");
  if (a.shape.size() != b.shape.size()) throw std::invalid_argument(std::string(op) + ": rank mismatch");
  if (a.dtype != b.dtype || a.dtype != DType::Fp32) {
    throw std::invalid_argument(std::string(op) + ": only Fp32 supported");
  }
  if (a.device != b.device) throw std::invalid_argument(std::string(op) + ": device mismatch");
  for (size_t i = 0; i + 2 < a.shape.size(); ++i) {
    if (a.shape[i] != b.shape[i]) throw std::invalid_argument(std::string(op) + ": leading dims must match");
  }
}

// A [.., R, C] operand as the batched GEMM sees it: element (b, r, c) at
// data[b*sb + r*rs + c*cs].  Leading dims fold into one batch stride when
// they nest; otherwise the operand is made contiguous.
struct MatView {
  Tensor t;
  int64_t sb, rs, cs;
};

bool fold_batch(const Tensor& t, int64_t& sb) {
  const size_t nd = t.shape.size();
  int64_t span = 0;
  bool have = false;
  sb = 0;
  for (size_t i = nd - 2; i-- > 0;) {
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
  return true;
}

MatView mat_view(const Tensor& t, bool force_contig = false) {
  MatView v{t, 0, 0, 0};
  const size_t nd = t.shape.size();
  const bool unit = t.strides[nd - 1] == 1 || t.strides[nd - 2] == 1;
  if (force_contig || !unit || !fold_batch(t, v.sb)) {
    v.t = contiguous(t);
    fold_batch(v.t, v.sb);
  }
  v.rs = v.t.strides[nd - 2];
  v.cs = v.t.strides[nd - 1];
  return v;
}

// C_b[M,N] = sum_k X_b(m,k) Y_b(k,n).  x_m_rows: X's m index runs along x's
// dim -2 (else along dim -1); y_k_rows: Y's k index runs along y's dim -2.
// The unit-stride side of each operand picks the kernel layout (NN: X k-,
// Y n-contiguous; NT: both k-contiguous; TN: X m-, Y n-contiguous).  The one
// combination the kernels lack, and strides the kernels cannot take, are
// resolved by copying both operands to row-major first.
Tensor batched_product(const char* name, const MatView& x, bool x_m_rows, const MatView& y, bool y_k_rows,
                       const std::vector<int64_t>& out_shape, int64_t B, int64_t M, int64_t N, int64_t K,
                       bool copied = false) {
  if (x.t.device == Device::CPU) throw_cpu_compute(name);
  Tensor out = Tensor::empty(out_shape, DType::Fp32, Device::CUDA);
  if (out.numel() == 0) return out;
  const int64_t xm = x_m_rows ? x.rs : x.cs, xk = x_m_rows ? x.cs : x.rs;
  const int64_t yk = y_k_rows ? y.rs : y.cs, yn = y_k_rows ? y.cs : y.rs;
  const bool x_kc = xk == 1 || K == 1, x_mc = xm == 1 || M == 1;
  const bool y_nc = yn == 1 || N == 1, y_kc = yk == 1 || K == 1;
  int op = -1;
  int64_t lda = 0, ldb = 0;
  if (x_kc && y_nc) {
    op = AAR_GEMM_NN;
    lda = M == 1 ? K : xm;
    ldb = K == 1 ? N : yk;
  } else if (x_kc && y_kc) {
    op = AAR_GEMM_NT;
    lda = M == 1 ? K : xm;
    ldb = N == 1 ? K : yn;
  } else if (x_mc && y_nc) {
    op = AAR_GEMM_TN;
    lda = K == 1 ? M : xk;
    ldb = K == 1 ? N : yk;
  }
  const int64_t need_a = op == AAR_GEMM_TN ? M : K, need_b = op == AAR_GEMM_NT ? K : N;
  if (op < 0 || lda < need_a || ldb < need_b) {
    if (copied) throw std::runtime_error(std::string(name) + ": unsupported operand layout");
    return batched_product(name, mat_view(x.t, true), x_m_rows, mat_view(y.t, true), y_k_rows, out_shape, B, M, N,
                           K, true);
  }
  check_status(aar_gemm_f32_batched(op, B, M, N, K, fp(x.t), lda, x.sb, fp(y.t), ldb, y.sb, fp(out), N, M * N,
                                    current_stream()),
               name);
  return out;
}

int64_t leading_product(const Tensor& a) {
  int64_t p = 1;
  for (size_t i = 0; i + 2 < a.shape.size(); ++i) p *= a.shape[i];
  return p;
}

std::vector<int64_t> with_last_two(const Tensor& a, int64_t r, int64_t c) {
  std::vector<int64_t> out(a.shape.begin(), a.shape.end() - 2);
  out.push_back(r);
  out.push_back(c);
  return out;
}

// a [.., M, K] . b [.., K, N]
Tensor bmm_no_grad(const Tensor& a, const Tensor& b) {
  const size_t nd = a.shape.size();
  const int64_t M = a.shape[nd - 2], K = a.shape[nd - 1], N = b.shape[nd - 1];
  return batched_product("bmm", mat_view(a), true, mat_view(b), true, with_last_two(a, M, N), leading_product(a), M,
                         N, K);
}
// a [.., M, K] . b [.., N, K]^T
Tensor bmm_a_bt_no_grad(const Tensor& a, const Tensor& b) {
  const size_t nd = a.shape.size();
  const int64_t M = a.shape[nd - 2], K = a.shape[nd - 1], N = b.shape[nd - 2];
  return batched_product("bmm_a_bt", mat_view(a), true, mat_view(b), false, with_last_two(a, M, N),
                         leading_product(a), M, N, K);
}
// a [.., K, M]^T . b [.., K, N]
Tensor bmm_at_b_no_grad(const Tensor& a, const Tensor& b) {
  const size_t nd = a.shape.size();
  const int64_t K = a.shape[nd - 2], M = a.shape[nd - 1], N = b.shape[nd - 1];
  return batched_product("bmm_at_b", mat_view(a), false, mat_view(b), true, with_last_two(a, M, N),
                         leading_product(a), M, N, K);
}

class BmmFunction : public Function {
 public:
  Tensor saved_a, saved_b;
  std::vector<Tensor> backward(const Tensor& g) override {
    return {bmm_a_bt_no_grad(g, saved_b), bmm_at_b_no_grad(saved_a, g)};
  }
  const char* name() const override { return "BmmFunction"; }
};
class BmmABTFunction : public Function {
 public:
  Tensor saved_a, saved_b;
  std::vector<Tensor> backward(const Tensor& g) override {
    return {bmm_no_grad(g, saved_b), bmm_at_b_no_grad(g, saved_a)};
  }
  const char* name() const override { return "BmmABTFunction"; }
};
class BmmATBFunction : public Function {
 public:
  Tensor saved_a, saved_b;
  std::vector<Tensor> backward(const Tensor& g) override {
    return {bmm_a_bt_no_grad(saved_b, g), bmm_no_grad(saved_a, g)};
  }
  const char* name() const override { return "BmmATBFunction"; }
};

template <class Fn>
Tensor bmm_with_grad(const Tensor& a, const Tensor& b, Tensor out) {
  if (!a.requires_grad && !b.requires_grad) return out;
  auto fn = std::make_shared<Fn>();
  fn->record_input(a);
  fn->record_input(b);
  fn->saved_a = a;
  fn->saved_b = b;
  return attach(fn, out);
}

// ---------------------------------------------------------------- causal mask

void check_causal(const Tensor& x) {
  if (x.dtype != DType::Fp32) throw std::invalid_argument("apply_causal_mask: only Fp32 supported");
  if (x.shape.size() < 2 || x.shape[x.shape.size() - 1] != x.shape[x.shape.size() - 2]) {
    throw std::invalid_argument("apply_causal_mask: input must be a square matrix");
  }
}

Tensor causal_fill(const Tensor& xc, float fill, const char* name) {
  if (xc.device == Device::CPU) throw_cpu_compute(name);
  Tensor out = Tensor::empty(xc.shape, xc.dtype, xc.device);
  const int64_t T = xc.shape.back();
  const int64_t mats = T ? static_cast<int64_t>(xc.numel()) / (T * T) : 0;
  check_status(aar_causal_mask_f32(fp(xc), fp(out), mats, T, fill, current_stream()), name);
  return out;
}

class CausalMaskFunction : public Function {
 public:
  std::vector<Tensor> backward(const Tensor& g) override {
    Tensor gc = g.is_contiguous() ? g : contiguous(g);
    return {causal_fill(gc, 0.0f, "apply_causal_mask backward")};
  }
  const char* name() const override { return "CausalMaskFunction"; }
};

// ---------------------------------------------------------------- dropout

std::atomic<uint64_t>& seed_counter() {
  static std::atomic<uint64_t> counter{static_cast<uint64_t>(std::random_device{}())};
  return counter;
}

class DropoutFunction : public Function {
 public:
  Tensor saved_mask;
  std::vector<Tensor> backward(const Tensor& g) override { return {mul(g, saved_mask)}; }
  const char* name() const override { return "DropoutFunction"; }
};

}  // namespace

Tensor bmm(const Tensor& a, const Tensor& b) {
  check_bmm_common(a, b, "bmm");
  const size_t nd = a.shape.size();
  if (a.shape[nd - 1] != b.shape[nd - 2]) throw std::invalid_argument("bmm: contraction dim mismatch");
  return bmm_with_grad<BmmFunction>(a, b, bmm_no_grad(a, b));
}

Tensor bmm_a_bt(const Tensor& a, const Tensor& b) {
  check_bmm_common(a, b, "bmm_a_bt");
  const size_t nd = a.shape.size();
  if (a.shape[nd - 1] != b.shape[nd - 1]) throw std::invalid_argument("bmm_a_bt: contraction dim mismatch");
  return bmm_with_grad<BmmABTFunction>(a, b, bmm_a_bt_no_grad(a, b));
}

Tensor bmm_at_b(const Tensor& a, const Tensor& b) {
  check_bmm_common(a, b, "bmm_at_b");
  const size_t nd = a.shape.size();
  if (a.shape[nd - 2] != b.shape[nd - 2]) throw std::invalid_argument("bmm_at_b: contraction dim mismatch");
  return bmm_with_grad<BmmATBFunction>(a, b, bmm_at_b_no_grad(a, b));
}

Tensor apply_causal_mask(const Tensor& x) {
  check_causal(x);
  Tensor xc = x.is_contiguous() ? x : contiguous(x);
  Tensor out = causal_fill(xc, -std::numeric_limits<float>::infinity(), "apply_causal_mask");
  if (!xc.requires_grad) return out;
  auto fn = std::make_shared<CausalMaskFunction>();
  fn->record_input(xc);
  return attach(fn, out);
}

void manual_seed(uint64_t seed) { seed_counter().store(seed, std::memory_order_relaxed); }

Tensor dropout(const Tensor& x, float p) {
  if (x.dtype != DType::Fp32) throw std::invalid_argument("dropout: only Fp32 supported");
  if (!(p >= 0.0f && p < 1.0f)) throw std::invalid_argument("dropout: p must be in [0, 1)");
  Tensor xc = x.is_contiguous() ? x : contiguous(x);
  if (p == 0.0f) return xc;
  const uint64_t seed = seed_counter().fetch_add(1, std::memory_order_relaxed);
  if (xc.device == Device::CPU) throw_cpu_compute("dropout");
  Tensor out = Tensor::empty(xc.shape, xc.dtype, xc.device);
  Tensor mask = Tensor::empty(xc.shape, xc.dtype, xc.device);
  check_status(aar_dropout_f32(fp(xc), fp(out), fp(mask), static_cast<int64_t>(xc.numel()), p, seed,
                               current_stream()),
               "dropout");
  if (!xc.requires_grad) return out;
  auto fn = std::make_shared<DropoutFunction>();
  fn->record_input(xc);
  fn->saved_mask = mask;
  return attach(fn, out);
}

}  // namespace aar
