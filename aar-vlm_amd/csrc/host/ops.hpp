// Public ops of aargrad._core (same names, argument meaning and exceptions as
// the reference's namespace-vlm functions bound in cppsrc/python/binding.cpp).
#pragma once

#include <tuple>

#include "tensor.hpp"

namespace aar {

// Views and layout (cppsrc/ops/shape.cpp:99-374).
Tensor contiguous(const Tensor& x);
Tensor reshape(const Tensor& x, std::vector<int64_t> new_shape);
Tensor transpose(const Tensor& x, int64_t dim_a, int64_t dim_b);
Tensor slice(const Tensor& x, int64_t dim, int64_t start, int64_t end);
Tensor squeeze(const Tensor& x, int64_t dim);
Tensor unsqueeze(const Tensor& x, int64_t dim);

// GEMM (cppsrc/ops/matmul.cpp:169-257).
Tensor matmul(const Tensor& a, const Tensor& b);
Tensor matmul_a_bt(const Tensor& a, const Tensor& b);
Tensor matmul_at_b(const Tensor& a, const Tensor& b);
// nn.Linear with a bias (aargrad/nn.py:101-105: matmul_a_bt then add_bias)
// as one GEMM with the bias added in its epilogue; same values and gradients.
Tensor linear(const Tensor& x, const Tensor& w, const Tensor& b);
// linear(relu(linear(x, w1, b1)), w2, b2) with bias + relu in the first
// GEMM's epilogue; same values and gradients as the composition.
Tensor mlp_relu(const Tensor& x, const Tensor& w1, const Tensor& b1, const Tensor& w2, const Tensor& b2);
// The pre-norm block's residual adds folded into the last GEMM's epilogue:
// r + matmul_a_bt(a, w) and r + mlp_relu(x, w1, b1, w2, b2), with the values
// and gradients (and fan-in order) of the add + op compositions.
Tensor linear_residual(const Tensor& r, const Tensor& a, const Tensor& w);
Tensor mlp_relu_residual(const Tensor& r, const Tensor& x, const Tensor& w1, const Tensor& b1, const Tensor& w2,
                         const Tensor& b2);

// Row-wise (cppsrc/ops/softmax.cpp:75-96, cppsrc/ops/layernorm.cpp:174-227).
Tensor softmax(const Tensor& x);
Tensor layernorm(const Tensor& x, const Tensor& weight, const Tensor& bias, float eps);

// Attention (cppsrc/ops/flash_attention.cpp:65-98).
Tensor flash_attention(const Tensor& q, const Tensor& k, const Tensor& v, bool causal);
// Attention over a packed projection [..., T, 3*D] -> [..., T, D] (the
// MultiHeadAttention composition without materialised head views).
Tensor flash_attention_qkv(const Tensor& qkv, int64_t n_heads, bool causal);
// Forward returning (O, lse) for benchmarks and parity checks; no autograd node.
std::tuple<Tensor, Tensor> flash_attention_fwd_lse(const Tensor& q, const Tensor& k, const Tensor& v,
                                                   bool causal);

// Elementwise (cppsrc/ops/elementwise.cpp:315-330) and gradient fan-in
// (cppsrc/autograd/backward.cpp:17-36).
Tensor add(const Tensor& a, const Tensor& b);
Tensor add_grads(const Tensor& a, const Tensor& b);

// Ops of the GPT training step around the path (cppsrc/ops/elementwise.cpp:315-474,
// embedding.cpp:78-104, cross_entropy.cpp:121-152, adamw.cpp:47-75).
Tensor sub(const Tensor& a, const Tensor& b);
Tensor mul(const Tensor& a, const Tensor& b);
Tensor scale(const Tensor& x, float alpha);
Tensor relu(const Tensor& a);
Tensor gelu(const Tensor& a);
Tensor sum_all(const Tensor& a);
Tensor add_bias(const Tensor& x, const Tensor& bias);
void scaled_add_inplace(Tensor& dst, const Tensor& src, float alpha);
Tensor embedding(const Tensor& weight, const Tensor& ids);
// add(embedding(w1, ids1), embedding(w2, ids2)) in one pass, same values and gradients.
Tensor embedding_add(const Tensor& w1, const Tensor& ids1, const Tensor& w2, const Tensor& ids2);
Tensor cross_entropy(const Tensor& logits, const Tensor& targets, int64_t ignore_index);
void adamw_step(Tensor& param, const Tensor& grad, Tensor& m, Tensor& v, float lr, float beta1, float beta2,
                float eps, float weight_decay, float bias_correction1, float bias_correction2);
// One launch per up to 48 parameters instead of one per parameter (the
// reference optimizers' loops, aargrad/optim.py:13-18, :36-54); same
// validation and messages, bit-identical results.
void scaled_add_inplace_multi(std::vector<Tensor>& dsts, const std::vector<Tensor>& srcs, float alpha);
void adamw_step_multi(std::vector<Tensor>& params, const std::vector<Tensor>& grads, std::vector<Tensor>& ms,
                      std::vector<Tensor>& vs, float lr, float beta1, float beta2, float eps, float weight_decay,
                      float bias_correction1, float bias_correction2);

// Batched products, causal mask, dropout (cppsrc/ops/bmm.cpp:212-268,
// attention.cpp:77-90, dropout.cpp:66-92).
Tensor bmm(const Tensor& a, const Tensor& b);
Tensor bmm_a_bt(const Tensor& a, const Tensor& b);
Tensor bmm_at_b(const Tensor& a, const Tensor& b);
Tensor apply_causal_mask(const Tensor& x);
Tensor dropout(const Tensor& x, float p);
void manual_seed(uint64_t seed);

// Token-window batch (x, y) of shape [starts, seq_len] gathered on the device
// from an int64 token stream (python/shakespeare/scripts/data.py:38-53).
std::tuple<Tensor, Tensor> token_windows(const Tensor& tokens, const Tensor& starts, int64_t seq_len);

}  // namespace aar
