/*
 * aar_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatement of the reference CPU path (AARONKANG04/aar-vlm,
 * cppsrc/ops/*.cpp) for the ops the MI355X backend accelerates.  It is the
 * parity checker for tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg, and nothing else: the product (aar-vlm_amd/) never links,
 * loads or calls it.
 *
 * Arithmetic order follows the reference loop by loop (fp32 accumulators,
 * sequential sums, the same evaluation order), and the file is compiled with
 * -O3 -ffp-contract=off and no fast-math, matching the reference's Release
 * build on x86-64, so results agree bit for bit with the reference compiled
 * from its own sources (checked against oracle/_ref where that is built).
 *
 * Pinning of each function (see tests/test_oracle.py):
 *   orc_matmul_*        reference KATs (tests/cpp/test_matmul.cpp:21-88,
 *                       test_autograd_ops.cpp:277-306), float64 brute force,
 *                       bit-exact vs oracle/_ref.
 *   orc_softmax_*       invariants of tests/cpp/test_softmax.cpp:20-65 and
 *                       test_autograd_ops.cpp:364-378, float64 closed form,
 *                       finite differences, bit-exact vs oracle/_ref.
 *   orc_layernorm_*     tests/cpp/test_layernorm.cpp:27-98, dbeta row-sum KAT
 *                       (test_autograd_ops.cpp:443-460), float64 closed form,
 *                       finite differences, bit-exact vs oracle/_ref.
 *   orc_attention_*     numpy attention_ref closed form
 *                       (tests/python/test_flash_attention.py:16-26), float64
 *                       closed-form gradients, finite differences on dQ,
 *                       bit-exact vs oracle/_ref.
 *   orc_attention_lse   the reference CPU path has no lse; float64 closed form
 *                       L_i = m_i + ln sum_{j} exp(s_ij - m_i) (the
 *                       definition), checked against a log-sum-exp computed
 *                       independently in numpy.
 *   orc_add             exact (c = a + b in fp32), fan-in KATs of
 *                       tests/cpp/test_autograd.cpp:169-186.
 *   GPT-step ops        (sub, mul, scale, relu, gelu, add_bias, bias_grad,
 *                       sum_all, scaled_add, embedding, cross_entropy, adamw):
 *                       KATs of tests/cpp/test_elementwise.cpp and
 *                       tests/python/test_{embedding,cross_entropy,adamw}.py,
 *                       float64 closed forms, bit-exact vs oracle/_ref.
 *   orc_philox4x32_10   the published Philox-4x32-10 known-answer vectors
 *                       (Random123 kat_vectors), bit-exact vs the reference's
 *                       philox_uniform through oracle/_ref.
 *   orc_dropout         the properties of tests/python/test_dropout.py
 *                       (drop rate, rescaled survivors, reproducibility),
 *                       bit-exact vs oracle/_ref.
 *   orc_causal_mask     numpy triangle closed form, bit-exact vs oracle/_ref.
 *   bmm                 per-batch orc_matmul_* (the reference's bmm_cpu loops
 *                       accumulate exactly as matmul_cpu does), bit-exact vs
 *                       oracle/_ref.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ GEMM */

/* Rows [r0, r1) of C = A[M,K] . B[K,N]  (cppsrc/ops/matmul.cpp:24-45). */
void orc_matmul_nn(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
                   int64_t r0, int64_t r1) {
  (void)M;
  for (int64_t i = r0; i < r1; ++i) {
    for (int64_t j = 0; j < N; ++j) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) acc += A[i * K + k] * B[k * N + j];
      C[i * N + j] = acc;
    }
  }
}

/* Rows [r0, r1) of C = A[M,K] . B[N,K]^T  (cppsrc/ops/matmul.cpp:47-68). */
void orc_matmul_nt(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
                   int64_t r0, int64_t r1) {
  (void)M;
  for (int64_t i = r0; i < r1; ++i) {
    for (int64_t j = 0; j < N; ++j) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) acc += A[i * K + k] * B[j * K + k];
      C[i * N + j] = acc;
    }
  }
}

/* Rows [r0, r1) of C = A[K,M]^T . B[K,N]  (cppsrc/ops/matmul.cpp:70-91). */
void orc_matmul_tn(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
                   int64_t r0, int64_t r1) {
  for (int64_t i = r0; i < r1; ++i) {
    for (int64_t j = 0; j < N; ++j) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) acc += A[k * M + i] * B[k * N + j];
      C[i * N + j] = acc;
    }
  }
}

/* --------------------------------------------------------------- softmax */

/* cppsrc/ops/softmax.cpp:15-37: max, exp(x - max) stored, sequential sum,
 * multiply by 1/sum. */
void orc_softmax_fwd(const float* X, float* Y, int64_t rows, int64_t cols) {
  for (int64_t i = 0; i < rows; ++i) {
    const float* row = X + i * cols;
    float* out = Y + i * cols;
    float max_val = row[0];
    for (int64_t j = 1; j < cols; ++j)
      if (row[j] > max_val) max_val = row[j];
    float sum = 0.0f;
    for (int64_t j = 0; j < cols; ++j) {
      out[j] = expf(row[j] - max_val);
      sum += out[j];
    }
    const float inv_sum = 1.0f / sum;
    for (int64_t j = 0; j < cols; ++j) out[j] *= inv_sum;
  }
}

/* cppsrc/ops/softmax.cpp:39-55: dx = y * (g - sum(g*y)). */
void orc_softmax_bwd(const float* G, const float* Y, float* DX, int64_t rows, int64_t cols) {
  for (int64_t i = 0; i < rows; ++i) {
    const float* g = G + i * cols;
    const float* y = Y + i * cols;
    float* dx = DX + i * cols;
    float dot = 0.0f;
    for (int64_t j = 0; j < cols; ++j) dot += g[j] * y[j];
    for (int64_t j = 0; j < cols; ++j) dx[j] = y[j] * (g[j] - dot);
  }
}

/* ------------------------------------------------------------- layernorm */

/* cppsrc/ops/layernorm.cpp:20-51 (no stats) and :53-89 (with stats): two-pass
 * mean / biased variance, rstd = 1/sqrt(var+eps), y = (x-mean)*rstd*w + b.
 * mean/rstd may be NULL. */
void orc_layernorm_fwd(const float* X, const float* W, const float* B, float* Y, float* mean,
                       float* rstd, int64_t rows, int64_t cols, float eps) {
  const float D = (float)cols;
  for (int64_t i = 0; i < rows; ++i) {
    const float* x = X + i * cols;
    float* y = Y + i * cols;
    float sum = 0.0f;
    for (int64_t j = 0; j < cols; ++j) sum += x[j];
    const float mu = sum / D;
    float sq = 0.0f;
    for (int64_t j = 0; j < cols; ++j) {
      const float d = x[j] - mu;
      sq += d * d;
    }
    const float var = sq / D;
    const float r = 1.0f / sqrtf(var + eps);
    if (mean) mean[i] = mu;
    if (rstd) rstd[i] = r;
    for (int64_t j = 0; j < cols; ++j) y[j] = (x[j] - mu) * r * W[j] + B[j];
  }
}

/* cppsrc/ops/layernorm.cpp:91-134: dx per row; dw, db accumulated over rows
 * in row order. */
void orc_layernorm_bwd(const float* GY, const float* X, const float* W, const float* M,
                       const float* R, float* DX, float* DW, float* DB, int64_t rows, int64_t cols) {
  const float D = (float)cols;
  const float inv_D = 1.0f / D;
  memset(DW, 0, (size_t)cols * sizeof(float));
  memset(DB, 0, (size_t)cols * sizeof(float));
  for (int64_t i = 0; i < rows; ++i) {
    const float* gy = GY + i * cols;
    const float* x = X + i * cols;
    float* dx = DX + i * cols;
    const float mu = M[i], r = R[i];
    float sum_g = 0.0f, sum_gn = 0.0f;
    for (int64_t j = 0; j < cols; ++j) {
      const float n = (x[j] - mu) * r;
      const float g = gy[j] * W[j];
      sum_g += g;
      sum_gn += g * n;
      DW[j] += gy[j] * n;
      DB[j] += gy[j];
    }
    for (int64_t j = 0; j < cols; ++j) {
      const float n = (x[j] - mu) * r;
      const float g = gy[j] * W[j];
      dx[j] = r * (g - sum_g * inv_D - n * sum_gn * inv_D);
    }
  }
}

/* ------------------------------------------------------------- attention */

/* The reference CPU flash attention is the composite
 *   bmm(softmax(mask(scale(bmm_a_bt(q, k), s))), v)
 * (cppsrc/ops/flash_attention.cpp:40-45) with s = 1/sqrt(float(d)), and its
 * gradient is what autograd derives from that graph.  Per (b,h) slice:
 *   raw = q k^T            bmm_a_bt_cpu        cppsrc/ops/bmm.cpp:101-132
 *   sc  = s * raw          scale_cpu           cppsrc/ops/elementwise.cpp:64-71
 *   msk = j<=i ? sc : -inf apply_causal_mask   cppsrc/ops/attention.cpp:24-40
 *   P   = softmax(msk)     softmax_cpu
 *   out = P v              bmm_cpu             cppsrc/ops/bmm.cpp:68-99
 * Scratch: one [T,T] float buffer per call (P), plus a second in backward. */

static float orc_scale_of(int64_t d) { return 1.0f / sqrtf((float)d); }

static void orc_scores(const float* q, const float* k, float* S, int64_t T, int64_t d, int causal) {
  const float s = orc_scale_of(d);
  for (int64_t i = 0; i < T; ++i)
    for (int64_t j = 0; j < T; ++j) {
      float acc = 0.0f;
      for (int64_t e = 0; e < d; ++e) acc += q[i * d + e] * k[j * d + e];
      S[i * T + j] = s * acc;
    }
  if (causal) {
    const float neg_inf = -INFINITY;
    for (int64_t i = 0; i < T; ++i)
      for (int64_t j = 0; j < T; ++j)
        if (j > i) S[i * T + j] = neg_inf;
  }
}

/* out[bh][T][d]; returns 0, or -1 when scratch cannot be allocated. */
int orc_attention_fwd(const float* Q, const float* K, const float* V, float* O, int64_t bh, int64_t T,
                      int64_t d, int causal) {
  float* S = (float*)malloc((size_t)T * (size_t)T * sizeof(float));
  float* P = (float*)malloc((size_t)T * (size_t)T * sizeof(float));
  if (!S || !P) {
    free(S);
    free(P);
    return -1;
  }
  for (int64_t b = 0; b < bh; ++b) {
    const float* q = Q + b * T * d;
    const float* k = K + b * T * d;
    const float* v = V + b * T * d;
    float* o = O + b * T * d;
    orc_scores(q, k, S, T, d, causal);
    orc_softmax_fwd(S, P, T, T);
    for (int64_t i = 0; i < T; ++i)
      for (int64_t e = 0; e < d; ++e) {
        float acc = 0.0f;
        for (int64_t j = 0; j < T; ++j) acc += P[i * T + j] * v[j * d + e];
        o[i * d + e] = acc;
      }
  }
  free(S);
  free(P);
  return 0;
}

/* Gradients of the composite graph for upstream dO, in the order autograd
 * applies the Functions (cppsrc/ops/bmm.cpp:177-197, softmax.cpp:65-72,
 * attention.cpp:42-73, elementwise.cpp:242-249):
 *   dP  = dO v^T                  BmmFunction dA = bmm_a_bt(grad, v)
 *   dV  = P^T dO                  BmmFunction dB = bmm_at_b(P, grad)
 *   dS  = P * (dP - sum(dP*P))    softmax_backward_cpu
 *   dS  = j<=i ? dS : 0           causal_mask_backward_cpu
 *   dR  = s * dS                  ScaleFunction
 *   dQ  = dR k                    BmmABTFunction dA = bmm(grad, k)
 *   dK  = dR^T q                  BmmABTFunction dB = bmm_at_b(grad, q) */
int orc_attention_bwd(const float* Q, const float* K, const float* V, const float* dO, float* dQ,
                      float* dK, float* dV, int64_t bh, int64_t T, int64_t d, int causal) {
  float* S = (float*)malloc((size_t)T * (size_t)T * sizeof(float));
  float* P = (float*)malloc((size_t)T * (size_t)T * sizeof(float));
  if (!S || !P) {
    free(S);
    free(P);
    return -1;
  }
  const float s = orc_scale_of(d);
  for (int64_t b = 0; b < bh; ++b) {
    const float* q = Q + b * T * d;
    const float* k = K + b * T * d;
    const float* v = V + b * T * d;
    const float* go = dO + b * T * d;
    float* gq = dQ + b * T * d;
    float* gk = dK + b * T * d;
    float* gv = dV + b * T * d;
    orc_scores(q, k, S, T, d, causal);
    orc_softmax_fwd(S, P, T, T);
    /* dP into S */
    for (int64_t i = 0; i < T; ++i)
      for (int64_t j = 0; j < T; ++j) {
        float acc = 0.0f;
        for (int64_t e = 0; e < d; ++e) acc += go[i * d + e] * v[j * d + e];
        S[i * T + j] = acc;
      }
    /* dV = P^T dO */
    for (int64_t j = 0; j < T; ++j)
      for (int64_t e = 0; e < d; ++e) {
        float acc = 0.0f;
        for (int64_t i = 0; i < T; ++i) acc += P[i * T + j] * go[i * d + e];
        gv[j * d + e] = acc;
      }
    /* softmax backward, mask backward, scale backward, in place in S */
    for (int64_t i = 0; i < T; ++i) {
      float dot = 0.0f;
      for (int64_t j = 0; j < T; ++j) dot += S[i * T + j] * P[i * T + j];
      for (int64_t j = 0; j < T; ++j) S[i * T + j] = P[i * T + j] * (S[i * T + j] - dot);
    }
    if (causal)
      for (int64_t i = 0; i < T; ++i)
        for (int64_t j = 0; j < T; ++j)
          if (j > i) S[i * T + j] = 0.0f;
    for (int64_t n = 0; n < T * T; ++n) S[n] = s * S[n];
    /* dQ = dR k */
    for (int64_t i = 0; i < T; ++i)
      for (int64_t e = 0; e < d; ++e) {
        float acc = 0.0f;
        for (int64_t j = 0; j < T; ++j) acc += S[i * T + j] * k[j * d + e];
        gq[i * d + e] = acc;
      }
    /* dK = dR^T q */
    for (int64_t j = 0; j < T; ++j)
      for (int64_t e = 0; e < d; ++e) {
        float acc = 0.0f;
        for (int64_t i = 0; i < T; ++i) acc += S[i * T + j] * q[i * d + e];
        gk[j * d + e] = acc;
      }
  }
  free(S);
  free(P);
  return 0;
}

/* lse[bh][T] in float64 from the definition: L_i = m_i + ln sum_j exp(z_ij - m_i)
 * over z_ij = s * q_i . k_j (j <= i when causal), s = 1/sqrt(float(d)). */
void orc_attention_lse(const float* Q, const float* K, double* L, int64_t bh, int64_t T, int64_t d,
                       int causal) {
  const double s = (double)orc_scale_of(d);
  double* z = (double*)malloc((size_t)T * sizeof(double));
  if (!z) return;
  for (int64_t b = 0; b < bh; ++b) {
    const float* q = Q + b * T * d;
    const float* k = K + b * T * d;
    for (int64_t i = 0; i < T; ++i) {
      const int64_t jn = causal ? i + 1 : T;
      double m = -INFINITY;
      for (int64_t j = 0; j < jn; ++j) {
        double acc = 0.0;
        for (int64_t e = 0; e < d; ++e) acc += (double)q[i * d + e] * (double)k[j * d + e];
        z[j] = s * acc;
        if (z[j] > m) m = z[j];
      }
      double sum = 0.0;
      for (int64_t j = 0; j < jn; ++j) sum += exp(z[j] - m);
      L[b * T + i] = m + log(sum);
    }
  }
  free(z);
}

/* ------------------------------------------------------------ add_grads */

/* cppsrc/autograd/backward.cpp:28-35: c = a + b. */
void orc_add(const float* a, const float* b, float* c, int64_t n) {
  for (int64_t i = 0; i < n; ++i) c[i] = a[i] + b[i];
}

/* ------------------------------------------------- GPT-step ops (next row) */

/* cppsrc/ops/elementwise.cpp:104-112 */
void orc_sub(const float* a, const float* b, float* c, int64_t n) {
  for (int64_t i = 0; i < n; ++i) c[i] = a[i] - b[i];
}
/* cppsrc/ops/elementwise.cpp:54-62 */
void orc_mul(const float* a, const float* b, float* c, int64_t n) {
  for (int64_t i = 0; i < n; ++i) c[i] = a[i] * b[i];
}
/* cppsrc/ops/elementwise.cpp:64-71 */
void orc_scale(const float* x, float* y, float alpha, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = alpha * x[i];
}
/* cppsrc/ops/elementwise.cpp:73-80 (std::max(0.0f, x)) */
void orc_relu(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = x[i] > 0.0f ? x[i] : 0.0f;
}
/* cppsrc/ops/elementwise.cpp:210-218 */
void orc_relu_bwd(const float* g, const float* x, float* dx, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dx[i] = x[i] > 0.0f ? g[i] : 0.0f;
}
/* cppsrc/ops/elementwise.cpp:131-141 (exact erf GELU) */
void orc_gelu(const float* x, float* y, int64_t n) {
  const float inv_sqrt2 = 0.70710678118654752440f;
  for (int64_t i = 0; i < n; ++i) y[i] = 0.5f * x[i] * (1.0f + erff(x[i] * inv_sqrt2));
}
/* cppsrc/ops/elementwise.cpp:143-159 */
void orc_gelu_bwd(const float* g, const float* x, float* dx, int64_t n) {
  const float inv_sqrt2 = 0.70710678118654752440f;
  const float inv_sqrt_2pi = 0.39894228040143267794f;
  for (int64_t i = 0; i < n; ++i) {
    const float xi = x[i];
    const float cdf = 0.5f * (1.0f + erff(xi * inv_sqrt2));
    const float pdf = inv_sqrt_2pi * expf(-0.5f * xi * xi);
    dx[i] = g[i] * (cdf + xi * pdf);
  }
}
/* cppsrc/ops/elementwise.cpp:180-189: y[i] = x[i] + bias[i % D] */
void orc_add_bias(const float* x, const float* bias, float* y, int64_t n, int64_t D) {
  for (int64_t i = 0; i < n; ++i) y[i] = x[i] + bias[i % D];
}
/* cppsrc/ops/elementwise.cpp:191-199: db[i % D] += g[i] in element order */
void orc_bias_grad(const float* g, float* db, int64_t n, int64_t D) {
  memset(db, 0, (size_t)D * sizeof(float));
  for (int64_t i = 0; i < n; ++i) db[i % D] += g[i];
}
/* cppsrc/ops/elementwise.cpp:82-90: sequential fp32 sum */
float orc_sum_all(const float* x, int64_t n) {
  float acc = 0.0f;
  for (int64_t i = 0; i < n; ++i) acc += x[i];
  return acc;
}
/* cppsrc/ops/elementwise.cpp:473: d[i] += alpha * s[i] */
void orc_scaled_add(float* dst, const float* src, float alpha, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] += alpha * src[i];
}
/* cppsrc/ops/embedding.cpp:16-34; returns -1 on an id outside [0, V) */
int orc_embedding_fwd(const float* w, const int64_t* ids, float* out, int64_t n, int64_t V, int64_t D) {
  for (int64_t i = 0; i < n; ++i) {
    const int64_t idx = ids[i];
    if (idx < 0 || idx >= V) return -1;
    memcpy(out + i * D, w + idx * D, (size_t)D * sizeof(float));
  }
  return 0;
}
/* cppsrc/ops/embedding.cpp:36-50: rows accumulated in token order */
void orc_embedding_bwd(const float* g, const int64_t* ids, float* dw, int64_t n, int64_t V, int64_t D) {
  memset(dw, 0, (size_t)V * (size_t)D * sizeof(float));
  for (int64_t i = 0; i < n; ++i) {
    const float* grow = g + i * D;
    float* drow = dw + ids[i] * D;
    for (int64_t k = 0; k < D; ++k) drow[k] += grow[k];
  }
}
/* cppsrc/ops/cross_entropy.cpp:20-49: per-row float lse, double total over
 * active rows, float mean; returns -1 on a target outside [0, V). */
int orc_cross_entropy_fwd(const float* L, const int64_t* T, float* loss, int64_t N, int64_t V,
                          int64_t ignore_index) {
  double total = 0.0;
  int64_t active = 0;
  for (int64_t i = 0; i < N; ++i) {
    const int64_t t = T[i];
    if (t == ignore_index) continue;
    if (t < 0 || t >= V) return -1;
    const float* row = L + i * V;
    float m = row[0];
    for (int64_t v = 1; v < V; ++v)
      if (row[v] > m) m = row[v];
    float s = 0.0f;
    for (int64_t v = 0; v < V; ++v) s += expf(row[v] - m);
    const float lse = m + logf(s);
    total += (double)(lse - row[t]);
    ++active;
  }
  *loss = active > 0 ? (float)(total / (double)active) : 0.0f;
  return 0;
}
/* cppsrc/ops/cross_entropy.cpp:51-85 */
void orc_cross_entropy_bwd(float go, const float* L, const int64_t* T, float* DL, int64_t N, int64_t V,
                           int64_t ignore_index) {
  memset(DL, 0, (size_t)N * (size_t)V * sizeof(float));
  int64_t active = 0;
  for (int64_t i = 0; i < N; ++i)
    if (T[i] != ignore_index) ++active;
  if (active == 0) return;
  const float scale = go / (float)active;
  for (int64_t i = 0; i < N; ++i) {
    const int64_t t = T[i];
    if (t == ignore_index) continue;
    const float* row = L + i * V;
    float* drow = DL + i * V;
    float m = row[0];
    for (int64_t v = 1; v < V; ++v)
      if (row[v] > m) m = row[v];
    float s = 0.0f;
    for (int64_t v = 0; v < V; ++v) {
      drow[v] = expf(row[v] - m);
      s += drow[v];
    }
    const float inv_s = 1.0f / s;
    for (int64_t v = 0; v < V; ++v) drow[v] = (drow[v] * inv_s) * scale;
    drow[t] -= scale;
  }
}
/* cppsrc/ops/adamw.cpp:27-45 */
void orc_adamw(float* p, const float* g, float* mp, float* vp, int64_t n, float lr, float beta1, float beta2,
               float eps, float weight_decay, float bc1, float bc2) {
  const float one_minus_b1 = 1.0f - beta1;
  const float one_minus_b2 = 1.0f - beta2;
  const float wd_factor = 1.0f - lr * weight_decay;
  for (int64_t i = 0; i < n; ++i) {
    const float gi = g[i];
    const float mi = beta1 * mp[i] + one_minus_b1 * gi;
    const float vi = beta2 * vp[i] + one_minus_b2 * gi * gi;
    mp[i] = mi;
    vp[i] = vi;
    const float m_hat = mi / bc1;
    const float v_hat = vi / bc2;
    p[i] = p[i] * wd_factor - lr * m_hat / (sqrtf(v_hat) + eps);
  }
}

/* ------------------------------------------------------------- dropout */

/* Philox-4x32-10 block function (Salmon et al., SC'11): counter ctr[4], key
 * key[2] -> out[4].  Round: (c0,c1,c2,c3) <- (hi(c2*M1)^c1^k0, lo(c2*M1),
 * hi(c0*M0)^c3^k1, lo(c0*M0)); key += (W0, W1) between rounds
 * (cppsrc/core/rng.hpp:14-43). */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  uint32_t c[4] = {ctr[0], ctr[1], ctr[2], ctr[3]};
  uint32_t k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)c[0] * 0xD2511F53u;
    const uint64_t p1 = (uint64_t)c[2] * 0xCD9E8D57u;
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
    const uint32_t n1 = (uint32_t)p1;
    const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
    const uint32_t n3 = (uint32_t)p0;
    c[0] = n0;
    c[1] = n1;
    c[2] = n2;
    c[3] = n3;
    if (r < 9) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
  }
  memcpy(out, c, sizeof(c));
}

/* Uniform in [0, 1) of element idx under seed: word 0 of the block for
 * counter (idx lo, idx hi, 0, 0) and key (seed lo, seed hi), times 2^-32 in
 * float (cppsrc/core/rng.hpp:14-46). */
float orc_philox_uniform(uint64_t seed, uint64_t idx) {
  const uint32_t ctr[4] = {(uint32_t)idx, (uint32_t)(idx >> 32), 0u, 0u};
  const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  uint32_t out[4];
  orc_philox4x32_10(ctr, key, out);
  return (float)out[0] * (1.0f / 4294967296.0f);
}

/* dropout_cpu (cppsrc/ops/dropout.cpp:30-42). */
void orc_dropout(const float* X, float* O, float* M, int64_t n, float p, uint64_t seed) {
  const float scale = 1.0f / (1.0f - p);
  for (int64_t i = 0; i < n; ++i) {
    const float r = orc_philox_uniform(seed, (uint64_t)i);
    const float keep = (r >= p) ? scale : 0.0f;
    M[i] = keep;
    O[i] = X[i] * keep;
  }
}

/* --------------------------------------------------------- causal mask */

/* apply_causal_mask_cpu / causal_mask_backward_cpu
 * (cppsrc/ops/attention.cpp:24-56): fill = -inf forward, 0 backward. */
void orc_causal_mask(const float* X, float* Y, int64_t mats, int64_t T, float fill) {
  for (int64_t m = 0; m < mats; ++m)
    for (int64_t i = 0; i < T; ++i)
      for (int64_t j = 0; j < T; ++j) {
        const int64_t idx = m * T * T + i * T + j;
        Y[idx] = (j <= i) ? X[idx] : fill;
      }
}
