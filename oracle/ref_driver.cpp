// ref_driver.cpp -- TEST INFRASTRUCTURE ONLY.
//
// A C entry layer over the reference's own CPU implementation
// (AARONKANG04/aar-vlm, cppsrc/**), compiled from the reference sources where
// they lie (see oracle/Makefile) into oracle/_ref/libaar_ref.so.  Used by the
// tests to pin the C restatement (oracle/aar_oracle.c) bit for bit, and by
// bench.py as the "reference" CPU baseline.  Every function goes through the
// reference's public ops (vlm::matmul, vlm::softmax, ...) on Device::CPU, with
// autograd where the reference computes gradients that way.
#include <cstdint>
#include <cstring>
#include <exception>
#include <vector>

#include "core/tensor.hpp"
#include "ops/adamw.hpp"
#include "ops/cross_entropy.hpp"
#include "ops/elementwise.hpp"
#include "ops/embedding.hpp"
#include "ops/flash_attention.hpp"
#include "ops/layernorm.hpp"
#include "ops/matmul.hpp"
#include "ops/softmax.hpp"

using vlm::DType;
using vlm::Tensor;

namespace {

Tensor make(const float* src, std::vector<int64_t> shape, bool requires_grad = false) {
  Tensor t = Tensor::empty(std::move(shape), DType::Fp32);
  if (t.nbytes()) std::memcpy(t.data(), src, t.nbytes());
  if (requires_grad) t.set_requires_grad(true);
  return t;
}

void out(const Tensor& t, float* dst) {
  Tensor c = t.is_contiguous() ? t : t;  // every op here returns contiguous storage
  if (c.nbytes()) std::memcpy(dst, c.data(), c.nbytes());
}

}  // namespace

extern "C" {

// op: 0 = matmul (A[M,K] B[K,N]), 1 = matmul_a_bt (B[N,K]), 2 = matmul_at_b (A[K,M]).
int ref_matmul(int op, const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K) {
  try {
    Tensor c;
    if (op == 0) c = vlm::matmul(make(A, {M, K}), make(B, {K, N}));
    else if (op == 1) c = vlm::matmul_a_bt(make(A, {M, K}), make(B, {N, K}));
    else c = vlm::matmul_at_b(make(A, {K, M}), make(B, {K, N}));
    out(c, C);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// Forward y = softmax(x); when g != NULL also dx = d(sum(y*g))/dx via autograd.
int ref_softmax(const float* x, const float* g, float* y, float* dx, int64_t rows, int64_t cols) {
  try {
    Tensor xt = make(x, {rows, cols}, g != nullptr);
    Tensor yt = vlm::softmax(xt);
    out(yt, y);
    if (g) {
      yt.backward(make(g, {rows, cols}));
      out(*xt.grad(), dx);
    }
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// Forward y = layernorm(x, w, b, eps); when gy != NULL also dx, dw, db via autograd.
int ref_layernorm(const float* x, const float* w, const float* b, const float* gy, float* y, float* dx,
                  float* dw, float* db, int64_t rows, int64_t cols, float eps) {
  try {
    const bool grad = gy != nullptr;
    Tensor xt = make(x, {rows, cols}, grad);
    Tensor wt = make(w, {cols}, grad);
    Tensor bt = make(b, {cols}, grad);
    Tensor yt = vlm::layernorm(xt, wt, bt, eps);
    out(yt, y);
    if (grad) {
      yt.backward(make(gy, {rows, cols}));
      out(*xt.grad(), dx);
      out(*wt.grad(), dw);
      out(*bt.grad(), db);
    }
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// q,k,v,o [bh,T,d]; when dout != NULL also dq, dk, dv via autograd.
int ref_attention(const float* q, const float* k, const float* v, const float* dout, float* o, float* dq,
                  float* dk, float* dv, int64_t bh, int64_t T, int64_t d, int causal) {
  try {
    const bool grad = dout != nullptr;
    Tensor qt = make(q, {bh, T, d}, grad);
    Tensor kt = make(k, {bh, T, d}, grad);
    Tensor vt = make(v, {bh, T, d}, grad);
    Tensor ot = vlm::flash_attention(qt, kt, vt, causal != 0);
    out(ot, o);
    if (grad) {
      ot.backward(make(dout, {bh, T, d}));
      out(*qt.grad(), dq);
      out(*kt.grad(), dk);
      out(*vt.grad(), dv);
    }
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// Unary/binary elementwise ops, forward and (when g != NULL) the gradient of
// sum(y * g) with respect to a, via autograd.
// op: 0 sub(a,b), 1 mul(a,b), 2 scale(a,alpha), 3 relu(a), 4 gelu(a)
int ref_elementwise(int op, const float* a, const float* b, float alpha, const float* g, float* y,
                    float* da, int64_t n) {
  try {
    const bool grad = g != nullptr;
    Tensor ta = make(a, {n}, grad);
    Tensor tb = b ? make(b, {n}) : Tensor();
    Tensor ty;
    switch (op) {
      case 0: ty = vlm::sub(ta, tb); break;
      case 1: ty = vlm::mul(ta, tb); break;
      case 2: ty = vlm::scale(ta, alpha); break;
      case 3: ty = vlm::relu(ta); break;
      default: ty = vlm::gelu(ta); break;
    }
    out(ty, y);
    if (grad) {
      ty.backward(make(g, {n}));
      out(*ta.grad(), da);
    }
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

int ref_add_bias(const float* x, const float* bias, const float* g, float* y, float* dbias, int64_t rows,
                 int64_t cols) {
  try {
    Tensor tx = make(x, {rows, cols});
    Tensor tb = make(bias, {cols}, g != nullptr);
    Tensor ty = vlm::add_bias(tx, tb);
    out(ty, y);
    if (g) {
      ty.backward(make(g, {rows, cols}));
      out(*tb.grad(), dbias);
    }
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

int ref_sum_all(const float* x, int64_t n, float* result) {
  try {
    Tensor s = vlm::sum_all(make(x, {n}));
    *result = *static_cast<const float*>(s.data());
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

int ref_embedding(const float* w, const int64_t* ids, const float* g, float* y, float* dw, int64_t n,
                  int64_t vocab, int64_t dim) {
  try {
    Tensor tw = make(w, {vocab, dim}, g != nullptr);
    Tensor ti = Tensor::empty({n}, DType::Int64);
    std::memcpy(ti.data(), ids, n * sizeof(int64_t));
    Tensor ty = vlm::embedding(tw, ti);
    out(ty, y);
    if (g) {
      ty.backward(make(g, {n, dim}));
      out(*tw.grad(), dw);
    }
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// loss = cross_entropy(logits, targets); when dlogits != NULL also the
// gradient for an upstream scalar grad `go`.
int ref_cross_entropy(const float* logits, const int64_t* targets, int64_t n, int64_t vocab,
                      int64_t ignore_index, float go, float* loss, float* dlogits) {
  try {
    Tensor tl = make(logits, {n, vocab}, dlogits != nullptr);
    Tensor tt = Tensor::empty({n}, DType::Int64);
    std::memcpy(tt.data(), targets, n * sizeof(int64_t));
    Tensor l = vlm::cross_entropy(tl, tt, ignore_index);
    *loss = *static_cast<const float*>(l.data());
    if (dlogits) {
      Tensor seed = Tensor::empty({}, DType::Fp32);
      *static_cast<float*>(seed.data()) = go;
      l.backward(seed);
      out(*tl.grad(), dlogits);
    }
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

int ref_adamw(float* p, const float* g, float* m, float* v, int64_t n, float lr, float b1, float b2, float eps,
              float wd, float bc1, float bc2) {
  try {
    Tensor tp = make(p, {n}), tg = make(g, {n}), tm = make(m, {n}), tv = make(v, {n});
    vlm::adamw_step(tp, tg, tm, tv, lr, b1, b2, eps, wd, bc1, bc2);
    out(tp, p);
    out(tm, m);
    out(tv, v);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

}  // extern "C"
