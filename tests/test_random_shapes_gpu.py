"""Seeded random-shape sweep over the hot path and its neighbours against the
oracle: GEMM in all three layouts (forward and both gradients through
autograd), softmax and layernorm (forward and backward), causal and
non-causal flash attention at random head dims (forward, lse, backward),
batched products and dropout.  Shapes are drawn from fixed seeds so every run
checks the same cases; tolerances as in the per-op tests (1e-4*sqrt(K) for
GEMM contractions, 1e-4 otherwise, both metrics; dropout bit-exact)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from conftest import TOL, assert_close, gemm_tol
from devutil import dev, host

pytestmark = pytest.mark.gpu
f32 = np.float32
SEEDS = list(range(12))


@pytest.mark.parametrize("seed", SEEDS)
def test_random_gemm(gpu, seed):
    rng = np.random.default_rng(10_000 + seed)
    M, N, K = (int(x) for x in rng.integers(1, 700, 3))
    a = rng.standard_normal((M, K)).astype(f32)
    g = rng.standard_normal((M, N)).astype(f32)
    for op, fn in (("nn", gpu.matmul), ("nt", gpu.matmul_a_bt)):
        b = rng.standard_normal((K, N) if op == "nn" else (N, K)).astype(f32)
        ta, tb = dev(gpu, a, True), dev(gpu, b, True)
        c = fn(ta, tb)
        c.backward(dev(gpu, g))
        assert_close(host(gpu, c), O.matmul(op, a, b), gemm_tol(K), f"{op} {M}x{N}x{K}")
        da = O.matmul("nt", g, b) if op == "nn" else O.matmul("nn", g, b)
        db = O.matmul("tn", a, g) if op == "nn" else O.matmul("tn", g, a)
        assert_close(host(gpu, ta.grad), da, gemm_tol(N), f"{op} dA")
        assert_close(host(gpu, tb.grad), db, gemm_tol(M), f"{op} dB")
    at = rng.standard_normal((K, M)).astype(f32)
    bt = rng.standard_normal((K, N)).astype(f32)
    c = gpu.matmul_at_b(dev(gpu, at), dev(gpu, bt))
    assert_close(host(gpu, c), O.matmul("tn", at, bt), gemm_tol(K), f"tn {M}x{N}x{K}")


@pytest.mark.parametrize("seed", SEEDS)
def test_random_rowwise(gpu, seed):
    rng = np.random.default_rng(20_000 + seed)
    rows, cols = int(rng.integers(1, 3000)), int(rng.integers(1, 5000))
    x = (2 * rng.standard_normal((rows, cols))).astype(f32)
    g = rng.standard_normal((rows, cols)).astype(f32)
    w = (1 + 0.1 * rng.standard_normal(cols)).astype(f32)
    b = (0.1 * rng.standard_normal(cols)).astype(f32)
    tx = dev(gpu, x, True)
    y = gpu.softmax(tx)
    y.backward(dev(gpu, g))
    ys = O.softmax(x)
    assert_close(host(gpu, y), ys, TOL, f"softmax {rows}x{cols}")
    assert_close(host(gpu, tx.grad), O.softmax_backward(g, ys), TOL, "softmax dx")
    tx, tw, tb = dev(gpu, x, True), dev(gpu, w, True), dev(gpu, b, True)
    yl = gpu.layernorm(tx, tw, tb, 1e-5)
    yl.backward(dev(gpu, g))
    yr, mu, rs = O.layernorm(x, w, b, 1e-5, stats=True)
    dx, dw, db = O.layernorm_backward(g, x, w, mu, rs)
    assert_close(host(gpu, yl), yr, TOL, f"layernorm {rows}x{cols}")
    assert_close(host(gpu, tx.grad), dx, TOL, "layernorm dx")
    assert_close(host(gpu, tw.grad), dw, TOL, "layernorm dw")
    assert_close(host(gpu, tb.grad), db, TOL, "layernorm db")


@pytest.mark.parametrize("seed", SEEDS)
def test_random_flash(gpu, seed):
    rng = np.random.default_rng(30_000 + seed)
    B, H = int(rng.integers(1, 4)), int(rng.integers(1, 4))
    T, d = int(rng.integers(1, 300)), int(rng.integers(1, 129))
    causal = bool(seed % 2)
    q, k, v, do = (rng.standard_normal((B, H, T, d)).astype(f32) for _ in range(4))
    tq, tk, tv = dev(gpu, q, True), dev(gpu, k, True), dev(gpu, v, True)
    o = gpu.flash_attention(tq, tk, tv, causal)
    o.backward(dev(gpu, do))
    what = f"B{B} H{H} T{T} d{d} causal={causal}"
    assert_close(host(gpu, o), O.attention(q, k, v, causal), TOL, "O " + what)
    rq, rk, rv = O.attention_backward(q, k, v, do, causal)
    for t, r, n in ((tq, rq, "dq"), (tk, rk, "dk"), (tv, rv, "dv")):
        assert_close(host(gpu, t.grad), r, TOL, f"{n} {what}")
    _, lse = gpu._core._flash_attention_fwd(dev(gpu, q), dev(gpu, k), dev(gpu, v), causal)
    assert_close(host(gpu, lse), O.attention_lse(q, k, causal), TOL, "lse " + what)


@pytest.mark.parametrize("seed", SEEDS)
def test_random_bmm_and_dropout(gpu, seed):
    rng = np.random.default_rng(40_000 + seed)
    Bn, M, N, K = (int(x) for x in rng.integers(1, 200, 4))
    for op in O.BMM_OPS:
        a = rng.standard_normal((Bn, K, M) if op == "bmm_at_b" else (Bn, M, K)).astype(f32)
        b = rng.standard_normal((Bn, N, K) if op == "bmm_a_bt" else (Bn, K, N)).astype(f32)
        c = getattr(gpu, op)(dev(gpu, a), dev(gpu, b))
        assert_close(host(gpu, c), O.bmm(op, a, b), gemm_tol(K), f"{op} {Bn}x{M}x{N}x{K}")
    n = int(rng.integers(1, 200_000))
    p = float(rng.uniform(0.05, 0.95))
    s = int(rng.integers(0, 2**63 - 1))
    x = rng.standard_normal(n).astype(f32)
    gpu.manual_seed(s)
    np.testing.assert_array_equal(host(gpu, gpu.dropout(dev(gpu, x), p)), O.dropout(x, p, s)[0])
