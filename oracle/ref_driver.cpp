// ref_driver.cpp -- TEST INFRASTRUCTURE ONLY.
//
// A C entry layer over the reference's own CPU implementation
// (AARONKANG04/aar-vlm, cppsrc/**), compiled from the reference sources where
// they lie (see oracle/Makefile) into oracle/_ref/libaar_ref.so.  Used by the
// tests to pin the C restatement (oracle/aar_oracle.c) bit for bit, and by
// bench.py as the "reference" CPU baseline.  Every function goes through the
// reference's public ops (vlm::matmul, vlm::softmax, ...) on Device::CPU, with
// autograd where the reference computes gradients that way.
//
// Compiled a second time with -DREF_DRIVER_ON_DEVICE into
// oracle/_ref/libaar_glue.so: the same entry points then put every operand on
// Device::CUDA, so the reference's own ops, autograd and optimizer steps run
// on the MI355X kernels through hip_backend.cpp and libaar_hip.so.  Host data
// only enters and leaves through make / make_ids / out / scalar.
#include <cstdint>
#include <cstring>
#include <exception>
#include <vector>

#include "core/tensor.hpp"
#include "ops/adamw.hpp"
#include "ops/attention.hpp"
#include "ops/bmm.hpp"
#include "ops/dropout.hpp"
#include "core/rng.hpp"
#include "ops/cross_entropy.hpp"
#include "ops/elementwise.hpp"
#include "ops/embedding.hpp"
#include "ops/flash_attention.hpp"
#include "ops/layernorm.hpp"
#include "ops/matmul.hpp"
#include "ops/shape.hpp"
#include "ops/softmax.hpp"

using vlm::Device;
using vlm::DType;
using vlm::Tensor;

namespace {

#ifdef REF_DRIVER_ON_DEVICE
constexpr Device kDevice = Device::CUDA;
#else
constexpr Device kDevice = Device::CPU;
#endif

// A tensor on kDevice holding a copy of `src` (host memory).
Tensor upload(const void* src, std::vector<int64_t> shape, DType dtype) {
  Tensor t = Tensor::empty(std::move(shape), dtype);
  if (t.nbytes()) std::memcpy(t.data(), src, t.nbytes());
  return kDevice == Device::CPU ? t : t.to(kDevice);
}

Tensor make(const float* src, std::vector<int64_t> shape, bool requires_grad = false) {
  Tensor t = upload(src, std::move(shape), DType::Fp32);
  if (requires_grad) t.set_requires_grad(true);
  return t;
}

Tensor make_ids(const int64_t* src, std::vector<int64_t> shape) {
  return upload(src, std::move(shape), DType::Int64);
}

// Copies a contiguous result (every op here returns one) to host memory.
void out(const Tensor& t, float* dst) {
  const Tensor h = t.device == Device::CPU ? t : t.to(Device::CPU);
  if (h.nbytes()) std::memcpy(dst, h.data(), h.nbytes());
}

float scalar(const Tensor& t) {
  float v = 0.0f;
  out(t, &v);
  return v;
}

// Position ids 0..T-1 for each of B rows.
Tensor positions(int64_t B, int64_t T) {
  std::vector<int64_t> pos(static_cast<size_t>(B * T));
  for (int64_t b = 0; b < B; ++b)
    for (int64_t t = 0; t < T; ++t) pos[b * T + t] = t;
  return make_ids(pos.data(), {B, T});
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
    *result = scalar(vlm::sum_all(make(x, {n})));
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

int ref_embedding(const float* w, const int64_t* ids, const float* g, float* y, float* dw, int64_t n,
                  int64_t vocab, int64_t dim) {
  try {
    Tensor tw = make(w, {vocab, dim}, g != nullptr);
    Tensor ty = vlm::embedding(tw, make_ids(ids, {n}));
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
    Tensor l = vlm::cross_entropy(tl, make_ids(targets, {n}), ignore_index);
    *loss = scalar(l);
    if (dlogits) {
      l.backward(make(&go, {}));
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

// philox_uniform of the reference (cppsrc/core/rng.hpp:14-46).
float ref_philox_uniform(uint64_t seed, uint64_t idx) { return vlm::philox_uniform(seed, idx); }

// dropout(x, p) after manual_seed(seed): the call draws exactly `seed`.
int ref_dropout(const float* x, float* y, float* dx, int64_t n, float p, uint64_t seed) {
  try {
    Tensor tx = make(x, {n}, dx != nullptr);
    vlm::manual_seed(seed);
    Tensor ty = vlm::dropout(tx, p);
    out(ty, y);
    if (dx) {
      vlm::sum_all(ty).backward();
      out(*tx.grad(), dx);
    }
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// apply_causal_mask on [mats, T, T]; with g also its backward.
int ref_causal_mask(const float* x, const float* g, float* y, float* dx, int64_t mats, int64_t T) {
  try {
    Tensor tx = make(x, {mats, T, T}, g != nullptr);
    Tensor ty = vlm::apply_causal_mask(tx);
    out(ty, y);
    if (g) {
      ty.backward(make(g, {mats, T, T}));
      out(*tx.grad(), dx);
    }
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// op: 0 = bmm (A[b,M,K] B[b,K,N]), 1 = bmm_a_bt (B[b,N,K]), 2 = bmm_at_b (A[b,K,M]).
int ref_bmm(int op, const float* A, const float* B, float* C, int64_t batch, int64_t M, int64_t N, int64_t K) {
  try {
    Tensor c;
    if (op == 0) c = vlm::bmm(make(A, {batch, M, K}), make(B, {batch, K, N}));
    else if (op == 1) c = vlm::bmm_a_bt(make(A, {batch, M, K}), make(B, {batch, N, K}));
    else c = vlm::bmm_at_b(make(A, {batch, K, M}), make(B, {batch, K, N}));
    out(c, C);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// One SGD training step of the decoder-only GPT of BASELINE config 5 on the
// reference CPU path, composed from the reference's public ops exactly as
// python/shakespeare/scripts/model.py composes them (with ReLU and no
// dropout).  params: pointers in Module.parameters() order (tok_emb, pos_emb,
// per block ln1 w/b, qkv, out, ln2 w/b, fc1 w/b, fc2 w/b, then ln_f w/b,
// head), updated in place; *loss_out receives the loss before the update.
int ref_gpt_step(int64_t vocab, int64_t ctx, int64_t layers, int64_t d, int64_t heads, int64_t batch,
                 float* const* params, const int64_t* ids, const int64_t* targets, float lr, float* loss_out) {
  try {
    const int64_t B = batch, T = ctx, f = 4 * d;
    std::vector<std::vector<int64_t>> shapes = {{vocab, d}, {ctx, d}};
    for (int64_t i = 0; i < layers; ++i) {
      for (auto s : std::vector<std::vector<int64_t>>{{d}, {d}, {3 * d, d}, {d, d}, {d}, {d}, {f, d}, {f}, {d, f}, {d}})
        shapes.push_back(s);
    }
    shapes.push_back({d});
    shapes.push_back({d});
    shapes.push_back({vocab, d});
    std::vector<Tensor> P;
    for (size_t i = 0; i < shapes.size(); ++i) P.push_back(make(params[i], shapes[i], true));

    const Tensor tids = make_ids(ids, {B, T});
    const Tensor pos = positions(B, T);
    const Tensor tgt = make_ids(targets, {B * T});

    Tensor x = vlm::add(vlm::embedding(P[0], tids), vlm::embedding(P[1], pos));
    for (int64_t i = 0; i < layers; ++i) {
      const Tensor* w = &P[2 + 10 * i];
      Tensor h = vlm::layernorm(x, w[0], w[1], 1e-5f);
      Tensor qkv = vlm::reshape(vlm::matmul_a_bt(h, w[2]), {B, T, 3, heads, d / heads});
      Tensor q = vlm::transpose(vlm::squeeze(vlm::slice(qkv, 2, 0, 1), 2), 1, 2);
      Tensor k = vlm::transpose(vlm::squeeze(vlm::slice(qkv, 2, 1, 2), 2), 1, 2);
      Tensor v = vlm::transpose(vlm::squeeze(vlm::slice(qkv, 2, 2, 3), 2), 1, 2);
      Tensor a = vlm::reshape(vlm::transpose(vlm::flash_attention(q, k, v, true), 1, 2), {B, T, d});
      x = vlm::add(x, vlm::matmul_a_bt(a, w[3]));
      h = vlm::layernorm(x, w[4], w[5], 1e-5f);
      h = vlm::relu(vlm::add_bias(vlm::matmul_a_bt(h, w[6]), w[7]));
      x = vlm::add(x, vlm::add_bias(vlm::matmul_a_bt(h, w[8]), w[9]));
    }
    const size_t n = P.size();
    x = vlm::layernorm(x, P[n - 3], P[n - 2], 1e-5f);
    Tensor logits = vlm::matmul_a_bt(x, P[n - 1]);
    Tensor loss = vlm::cross_entropy(vlm::reshape(logits, {B * T, vocab}), tgt, -100);
    *loss_out = scalar(loss);
    loss.backward();
    for (size_t i = 0; i < n; ++i) {
      vlm::scaled_add_inplace(P[i], *P[i].grad(), -lr);
      out(P[i], params[i]);
    }
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// One training step of the reference Shakespeare GPT
// (python/shakespeare/scripts/model.py:8-57: pre-LN, GELU MLP with biases,
// bias-free attention, dropout after the embeddings and on both residual
// branches) with AdamW (aargrad/optim.py AdamW.step): forward, backward,
// update.  seed >= 0 calls manual_seed(seed) first; otherwise the dropout
// seed counter carries on from the previous call.  grads_out (may be null)
// receives the gradients before the update; params, m and v are updated in
// place.  bc1/bc2 are AdamW's bias corrections for this step, computed by
// the caller as the Python optimizer does.
int ref_lm_step(int64_t vocab, int64_t ctx, int64_t layers, int64_t d, int64_t heads, int64_t batch,
                float dropout, int64_t seed, float* const* params, float* const* m_state, float* const* v_state,
                const int64_t* ids, const int64_t* targets, float lr, float b1, float b2, float eps, float wd,
                float bc1, float bc2, float* loss_out, float* const* grads_out) {
  try {
    const int64_t B = batch, T = ctx, f = 4 * d;
    std::vector<std::vector<int64_t>> shapes = {{vocab, d}, {ctx, d}};
    for (int64_t i = 0; i < layers; ++i) {
      for (auto s : std::vector<std::vector<int64_t>>{{d}, {d}, {3 * d, d}, {d, d}, {d}, {d}, {f, d}, {f}, {d, f}, {d}})
        shapes.push_back(s);
    }
    shapes.push_back({d});
    shapes.push_back({d});
    shapes.push_back({vocab, d});
    std::vector<Tensor> P, M, V;
    for (size_t i = 0; i < shapes.size(); ++i) {
      P.push_back(make(params[i], shapes[i], true));
      M.push_back(make(m_state[i], shapes[i]));
      V.push_back(make(v_state[i], shapes[i]));
    }
    const Tensor tids = make_ids(ids, {B, T});
    const Tensor pos = positions(B, T);
    const Tensor tgt = make_ids(targets, {B * T});
    if (seed >= 0) vlm::manual_seed((uint64_t)seed);
    auto drop = [&](const Tensor& x) { return dropout > 0.0f ? vlm::dropout(x, dropout) : x; };

    Tensor x = drop(vlm::add(vlm::embedding(P[0], tids), vlm::embedding(P[1], pos)));
    for (int64_t i = 0; i < layers; ++i) {
      const Tensor* w = &P[2 + 10 * i];
      Tensor h = vlm::layernorm(x, w[0], w[1], 1e-5f);
      Tensor qkv = vlm::reshape(vlm::matmul_a_bt(h, w[2]), {B, T, 3, heads, d / heads});
      Tensor q = vlm::transpose(vlm::squeeze(vlm::slice(qkv, 2, 0, 1), 2), 1, 2);
      Tensor k = vlm::transpose(vlm::squeeze(vlm::slice(qkv, 2, 1, 2), 2), 1, 2);
      Tensor v = vlm::transpose(vlm::squeeze(vlm::slice(qkv, 2, 2, 3), 2), 1, 2);
      Tensor a = vlm::reshape(vlm::transpose(vlm::flash_attention(q, k, v, true), 1, 2), {B, T, d});
      x = vlm::add(x, drop(vlm::matmul_a_bt(a, w[3])));
      h = vlm::layernorm(x, w[4], w[5], 1e-5f);
      h = vlm::gelu(vlm::add_bias(vlm::matmul_a_bt(h, w[6]), w[7]));
      x = vlm::add(x, drop(vlm::add_bias(vlm::matmul_a_bt(h, w[8]), w[9])));
    }
    const size_t n = P.size();
    x = vlm::layernorm(x, P[n - 3], P[n - 2], 1e-5f);
    Tensor logits = vlm::matmul_a_bt(x, P[n - 1]);
    Tensor loss = vlm::cross_entropy(vlm::reshape(logits, {B * T, vocab}), tgt, -100);
    *loss_out = scalar(loss);
    loss.backward();
    for (size_t i = 0; i < n; ++i) {
      if (grads_out) out(*P[i].grad(), grads_out[i]);
      vlm::adamw_step(P[i], *P[i].grad(), M[i], V[i], lr, b1, b2, eps, wd, bc1, bc2);
      out(P[i], params[i]);
      out(M[i], m_state[i]);
      out(V[i], v_state[i]);
    }
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// A fixed graph with gradient fan-in, run through the reference's ops and
// autograd (cppsrc/autograd/backward.cpp:50-113), for pinning the order in
// which fan-in gradients are summed:
//   h = x * w0;  u = h * w1;  v = scale(h, 0.75);  z = h * w2;
//   t = x * w3;  root = ((u + v) + z) + t;  root.backward(g)
// h receives three gradients (an interior fan-in), x two (a leaf fan-in).
// w is [4][n]; writes x.grad [n].
int ref_fanin_graph(const float* x, const float* w, const float* g, float* dx, int64_t n) {
  try {
    Tensor tx = make(x, {n}, true);
    Tensor w0 = make(w, {n}), w1 = make(w + n, {n}), w2 = make(w + 2 * n, {n}), w3 = make(w + 3 * n, {n});
    Tensor h = vlm::mul(tx, w0);
    Tensor u = vlm::mul(h, w1);
    Tensor v = vlm::scale(h, 0.75f);
    Tensor z = vlm::mul(h, w2);
    Tensor t = vlm::mul(tx, w3);
    Tensor root = vlm::add(vlm::add(vlm::add(u, v), z), t);
    root.backward(make(g, {n}));
    out(*tx.grad(), dx);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

}  // extern "C"
