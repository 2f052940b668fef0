"""Pins the oracle (oracle/aar_oracle.c) before it is trusted as the checker.

Each oracle function is checked against (a) the reference's own known-answer
tests restated here, (b) float64 closed forms and invariants, (c) finite
differences for gradients, (d) the golden vectors in tests/golden (written by
the reference's own CPU build) and (e) bit-exact agreement with oracle/_ref
(the reference CPU build) where that library exists.  The planted-mistake
tests at the end show that the checks catch a transposed operand, a dropped
term and a wrong sign.
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest

import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"
f32 = np.float32


def rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------- GEMM

def test_matmul_kat_nn():
    # tests/cpp/test_matmul.cpp:21-36
    a = np.array([[1, 2, 3], [4, 5, 6]], f32)
    b = np.array([[7, 8], [9, 10], [11, 12]], f32)
    np.testing.assert_array_equal(O.matmul("nn", a, b), [[58, 64], [139, 154]])


def test_matmul_kat_nt():
    # tests/cpp/test_matmul.cpp:58-72
    a = np.array([[1, 2, 3], [4, 5, 6]], f32)
    b = np.array([[7, 9, 11], [8, 10, 12]], f32)
    np.testing.assert_array_equal(O.matmul("nt", a, b), [[58, 64], [139, 154]])


def test_matmul_kat_tn():
    # tests/cpp/test_matmul.cpp:74-88
    a = np.array([[1, 4], [2, 5], [3, 6]], f32)
    b = np.array([[7, 8], [9, 10], [11, 12]], f32)
    np.testing.assert_array_equal(O.matmul("tn", a, b), [[58, 64], [139, 154]])


def test_matmul_identity():
    # tests/cpp/test_matmul.cpp:38-50
    a = np.arange(1, 10, dtype=f32).reshape(3, 3)
    np.testing.assert_array_equal(O.matmul("nn", a, np.eye(3, dtype=f32)), a)


def test_matmul_backward_kat():
    # tests/cpp/test_autograd_ops.cpp:277-306: d(sum(A B))/dA = 1 B^T, /dB = A^T 1
    a = np.array([[1, 2, 3], [4, 5, 6]], f32)
    b = np.array([[7, 8], [9, 10], [11, 12]], f32)
    g = np.ones((2, 2), f32)
    np.testing.assert_array_equal(O.matmul("nt", g, b), [[15, 19, 23], [15, 19, 23]])
    np.testing.assert_array_equal(O.matmul("tn", a, g), [[5, 5], [7, 7], [9, 9]])


@pytest.mark.parametrize("op", O.OPS)
@pytest.mark.parametrize("shape", [(1, 1, 1), (5, 7, 3), (37, 29, 53), (64, 48, 96)])
def test_matmul_closed_form(op, shape):
    M, N, K = shape
    r = rng(M * 1000 + N * 10 + K)
    a = r.standard_normal((M, K) if op != "tn" else (K, M)).astype(f32)
    b = r.standard_normal((K, N) if op != "nt" else (N, K)).astype(f32)
    A = a.astype(np.float64) if op != "tn" else a.T.astype(np.float64)
    B = b.astype(np.float64) if op != "nt" else b.T.astype(np.float64)
    ref = A @ B
    got = O.matmul(op, a, b)
    # sequential fp32 accumulation: |err| <= K * eps * sum|a||b|
    bound = K * np.finfo(f32).eps * (np.abs(A) @ np.abs(B)) + 1e-30
    assert np.all(np.abs(got - ref) <= bound)


def test_matmul_row_band():
    r = rng(3)
    a = r.standard_normal((40, 24)).astype(f32)
    b = r.standard_normal((24, 16)).astype(f32)
    full = O.matmul("nn", a, b)
    band = O.matmul("nn", a, b, rows=(10, 20))
    np.testing.assert_array_equal(band[10:20], full[10:20])
    assert not band[:10].any() and not band[20:].any()


# --------------------------------------------------------------- softmax

def test_softmax_sums_to_one():
    # tests/cpp/test_softmax.cpp:20-28
    y = O.softmax(np.array([[1, 2, 3, 4]], f32))
    assert abs(y.sum() - 1) < 1e-6 and (y > 0).all()


def test_softmax_uniform():
    # tests/cpp/test_softmax.cpp:30-35
    np.testing.assert_array_equal(O.softmax(np.zeros((1, 5), f32)), np.full((1, 5), 0.2, f32))


def test_softmax_stable_large():
    # tests/cpp/test_softmax.cpp:37-48
    y = O.softmax(np.array([[1000, 1001, 1002]], f32))[0]
    assert np.isfinite(y).all() and abs(y.sum() - 1) < 1e-6 and y[0] < y[1] < y[2]


def test_softmax_multirow():
    # tests/cpp/test_softmax.cpp:50-65
    x = np.array([[1, 2, 3, 4], [-1, -2, -3, -4], [100, 100, 100, 100]], f32)
    y = O.softmax(x)
    np.testing.assert_allclose(y.sum(1), 1, atol=1e-5)
    np.testing.assert_array_equal(y[2], np.full(4, 0.25, f32))


def test_softmax_closed_form():
    x = (3 * rng(5).standard_normal((64, 384))).astype(f32)
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(1, keepdims=True))
    np.testing.assert_allclose(O.softmax(x), e / e.sum(1, keepdims=True), rtol=2e-6, atol=1e-9)


def test_softmax_backward_of_sum_is_zero():
    # tests/cpp/test_autograd_ops.cpp:364-378
    x = np.array([[0.1, -0.5, 1.2, -0.3, 0.4]], f32)
    y = O.softmax(x)
    np.testing.assert_allclose(O.softmax_backward(np.ones_like(y), y), 0, atol=1e-5)


def test_softmax_backward_finite_diff():
    # tests/cpp/test_autograd_ops.cpp:380-403 (loss = sum(softmax(x) * w))
    x = (np.sin(np.arange(12) * 0.31) * 0.7).astype(f32).reshape(3, 4)
    w = (np.arange(12) * 0.13 - 0.5).astype(f32).reshape(3, 4)
    dx = O.softmax_backward(w, O.softmax(x))
    x64, w64 = x.astype(np.float64), w.astype(np.float64)

    def loss(xx):
        e = np.exp(xx - xx.max(1, keepdims=True))
        return float(((e / e.sum(1, keepdims=True)) * w64).sum())

    num = np.zeros_like(x64)
    for idx in np.ndindex(*x.shape):
        p, m = x64.copy(), x64.copy()
        p[idx] += 1e-6
        m[idx] -= 1e-6
        num[idx] = (loss(p) - loss(m)) / 2e-6
    np.testing.assert_allclose(dx, num, atol=1e-5)


# ------------------------------------------------------------- layernorm

def _ln64(x, w, b, eps=1e-5):
    x = x.astype(np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    n = (x - mu) / np.sqrt(var + eps)
    return n * w + b, mu[..., 0], 1 / np.sqrt(var[..., 0] + eps)


def test_layernorm_unit_stats():
    # tests/cpp/test_layernorm.cpp:27-44
    y = O.layernorm(np.arange(1, 9, dtype=f32)[None], np.ones(8, f32), np.zeros(8, f32))[0]
    assert abs(y.mean()) < 1e-5 and abs(((y - y.mean()) ** 2).mean() - 1) < 1e-3


def test_layernorm_affine():
    # tests/cpp/test_layernorm.cpp:46-63
    y = O.layernorm(np.arange(1, 9, dtype=f32)[None], np.full(8, 2, f32), np.full(8, 3, f32))[0]
    assert abs(y.mean() - 3) < 1e-5 and abs(((y - y.mean()) ** 2).mean() - 4) < 1e-2


def test_layernorm_constant_gives_bias():
    # tests/cpp/test_layernorm.cpp:65-72
    y = O.layernorm(np.full((1, 6), 7, f32), np.full(6, 5, f32), np.full(6, -1, f32))
    np.testing.assert_allclose(y, -1, atol=1e-3)


def test_layernorm_closed_form_and_stats():
    r = rng(9)
    x = (3 * r.standard_normal((48, 257))).astype(f32)
    w = (1 + 0.02 * r.standard_normal(257)).astype(f32)
    b = (0.02 * r.standard_normal(257)).astype(f32)
    y, mu, rs = O.layernorm(x, w, b, 1e-5, stats=True)
    y64, mu64, rs64 = _ln64(x, w, b)
    np.testing.assert_allclose(y, y64, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(mu, mu64, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(rs, rs64, rtol=1e-5)


def test_layernorm_backward_closed_form():
    r = rng(10)
    x = (3 * r.standard_normal((40, 96))).astype(f32)
    w = (1 + 0.02 * r.standard_normal(96)).astype(f32)
    b = (0.02 * r.standard_normal(96)).astype(f32)
    gy = r.standard_normal((40, 96)).astype(f32)
    _, mu, rs = O.layernorm(x, w, b, 1e-5, stats=True)
    dx, dw, db = O.layernorm_backward(gy, x, w, mu, rs)
    x64, g64 = x.astype(np.float64), gy.astype(np.float64)
    mu64 = x64.mean(1, keepdims=True)
    rs64 = 1 / np.sqrt(((x64 - mu64) ** 2).mean(1, keepdims=True) + 1e-5)
    n = (x64 - mu64) * rs64
    gg = g64 * w
    dx64 = rs64 * (gg - gg.mean(1, keepdims=True) - n * (gg * n).mean(1, keepdims=True))
    np.testing.assert_allclose(dx, dx64, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dw, (g64 * n).sum(0), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(db, g64.sum(0), rtol=1e-5, atol=1e-5)


def test_layernorm_dbias_row_sum_kat():
    # tests/cpp/test_autograd_ops.cpp:443-460: d(sum(y))/d(beta) = number of rows
    x = np.array([[1, 2, 3, 4], [-1, -2, -3, -4], [0.5, 1.5, 2.5, 3.5]], f32)
    _, mu, rs = O.layernorm(x, np.ones(4, f32), np.zeros(4, f32), 1e-5, stats=True)
    _, _, db = O.layernorm_backward(np.ones_like(x), x, np.ones(4, f32), mu, rs)
    np.testing.assert_array_equal(db, np.full(4, 3.0, f32))


def test_layernorm_backward_finite_diff():
    # tests/cpp/test_autograd_ops.cpp:405-441 (loss = sum(layernorm(x, w, b)))
    x = (np.sin(np.arange(24) * 0.21) * 1.5 + 0.1).astype(f32).reshape(4, 6)
    w = (1 + 0.2 * np.cos(np.arange(6) * 0.4)).astype(f32)
    b = (0.05 * np.arange(6)).astype(f32)
    r = rng(4)
    gy = r.standard_normal((4, 6)).astype(f32)
    _, mu, rs = O.layernorm(x, w, b, 1e-5, stats=True)
    dx, dw, db = O.layernorm_backward(gy, x, w, mu, rs)
    g64 = gy.astype(np.float64)

    def loss(xx, ww, bb):
        return float((_ln64(xx, ww, bb)[0] * g64).sum())

    for arr, got in ((x, dx), (w, dw), (b, db)):
        base = [x.astype(np.float64), w.astype(np.float64), b.astype(np.float64)]
        k = [id(x), id(w), id(b)].index(id(arr))
        num = np.zeros(arr.shape)
        for idx in np.ndindex(*arr.shape):
            p = [t.copy() for t in base]
            m = [t.copy() for t in base]
            p[k][idx] += 1e-6
            m[k][idx] -= 1e-6
            num[idx] = (loss(*p) - loss(*m)) / 2e-6
        np.testing.assert_allclose(got, num, atol=2e-4)


# ------------------------------------------------------------- attention

def attention_ref64(q, k, v, do, causal):
    """float64 closed forms of O, lse and the three gradients."""
    q, k, v, do = (t.astype(np.float64) for t in (q, k, v, do))
    d = q.shape[-1]
    s = q @ np.swapaxes(k, -1, -2) / math.sqrt(d)
    T = s.shape[-1]
    if causal:
        s = np.where(np.triu(np.ones((T, T), bool), 1), -np.inf, s)
    m = s.max(-1, keepdims=True)
    e = np.exp(s - m)
    p = e / e.sum(-1, keepdims=True)
    o = p @ v
    dv = np.swapaxes(p, -1, -2) @ do
    dp = do @ np.swapaxes(v, -1, -2)
    ds = p * (dp - (dp * p).sum(-1, keepdims=True))
    dq = ds @ k / math.sqrt(d)
    dk = np.swapaxes(ds, -1, -2) @ q / math.sqrt(d)
    return o, dq, dk, dv


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("T", [8, 32, 33, 64])
def test_attention_forward_closed_form(causal, T):
    # tests/python/test_flash_attention.py:29-44 (B2 H4 d16, atol 1e-4), fixed seed
    r = rng(100 + T + 1000 * causal)
    q, k, v = (r.standard_normal((2, 4, T, 16)).astype(f32) for _ in range(3))
    o_ref = attention_ref64(q, k, v, np.zeros_like(q), causal)[0]
    np.testing.assert_allclose(O.attention(q, k, v, causal), o_ref, atol=1e-5)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_backward_closed_form(causal):
    r = rng(21 + causal)
    q, k, v, do = (r.standard_normal((2, 3, 40, 16)).astype(f32) for _ in range(4))
    _, dq64, dk64, dv64 = attention_ref64(q, k, v, do, causal)
    dq, dk, dv = O.attention_backward(q, k, v, do, causal)
    for got, ref in ((dq, dq64), (dk, dk64), (dv, dv64)):
        np.testing.assert_allclose(got, ref, atol=2e-5)


def test_attention_dq_finite_diff():
    # tests/python/test_flash_attention.py:47-77 (B1 H2 T4 d8, causal, loss = sum(out))
    r = rng(7)
    q, k, v = (r.standard_normal((1, 2, 4, 8)).astype(f32) for _ in range(3))
    dq = O.attention_backward(q, k, v, np.ones_like(q), True)[0]
    k64, v64 = k.astype(np.float64), v.astype(np.float64)

    def loss(qq):
        return float(attention_ref64(qq, k64, v64, np.zeros_like(qq), True)[0].sum())

    q64 = q.astype(np.float64)
    num = np.zeros_like(q64)
    for idx in np.ndindex(*q.shape):
        p, m = q64.copy(), q64.copy()
        p[idx] += 1e-6
        m[idx] -= 1e-6
        num[idx] = (loss(p) - loss(m)) / 2e-6
    np.testing.assert_allclose(dq, num, atol=1e-5)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_lse_independent(causal):
    from scipy.special import logsumexp

    r = rng(31)
    q, k = (r.standard_normal((2, 2, 37, 24)).astype(f32) for _ in range(2))
    s = q.astype(np.float64) @ np.swapaxes(k.astype(np.float64), -1, -2) * float(f32(1) / np.sqrt(f32(24)))
    if causal:
        s = np.where(np.triu(np.ones((37, 37), bool), 1), -np.inf, s)
    np.testing.assert_allclose(O.attention_lse(q, k, causal), logsumexp(s, axis=-1), rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------- add

def test_add_exact_and_fanin_kat():
    r = rng(2)
    a, b = r.standard_normal(1000).astype(f32), r.standard_normal(1000).astype(f32)
    np.testing.assert_array_equal(O.add(a, b), a + b)
    # tests/cpp/test_autograd.cpp:169-186: 10000 fan-in additions of 1.0 give 10001
    acc = np.ones(1, f32)
    for _ in range(10000):
        acc = O.add(acc, np.ones(1, f32))
    assert acc[0] == 10001.0


# --------------------------------------------------------- golden vectors

def test_golden_gemm():
    z = np.load(GOLDEN / "gemm_64x96x48.npz")
    for op in O.OPS:
        np.testing.assert_array_equal(O.matmul(op, z[f"{op}_a"], z[f"{op}_b"]), z[f"{op}_c"])


def test_golden_softmax():
    z = np.load(GOLDEN / "softmax_32x257.npz")
    np.testing.assert_array_equal(O.softmax(z["x"]), z["y"])
    np.testing.assert_array_equal(O.softmax_backward(z["g"], z["y"]), z["dx"])


def test_golden_layernorm():
    z = np.load(GOLDEN / "layernorm_32x257.npz")
    y, mu, rs = O.layernorm(z["x"], z["w"], z["b"], float(z["eps"]), stats=True)
    np.testing.assert_array_equal(y, z["y"])
    dx, dw, db = O.layernorm_backward(z["gy"], z["x"], z["w"], mu, rs)
    np.testing.assert_array_equal(dx, z["dx"])
    np.testing.assert_array_equal(dw, z["dw"])
    np.testing.assert_array_equal(db, z["db"])


@pytest.mark.parametrize("causal", [0, 1])
def test_golden_attention(causal):
    z = np.load(GOLDEN / "attention_b2h4t64d16.npz")
    np.testing.assert_array_equal(O.attention(z["q"], z["k"], z["v"], causal), z[f"o_{causal}"])
    dq, dk, dv = O.attention_backward(z["q"], z["k"], z["v"], z["do"], causal)
    np.testing.assert_array_equal(dq, z[f"dq_{causal}"])
    np.testing.assert_array_equal(dk, z[f"dk_{causal}"])
    np.testing.assert_array_equal(dv, z[f"dv_{causal}"])


# ------------------------------------------- reference CPU build (oracle/_ref)

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference tree)")


@needs_ref
@pytest.mark.parametrize("op", O.OPS)
def test_ref_bitexact_gemm(op):
    r = rng(41)
    M, N, K = 33, 70, 45
    a = r.standard_normal((M, K) if op != "tn" else (K, M)).astype(f32)
    b = r.standard_normal((K, N) if op != "nt" else (N, K)).astype(f32)
    np.testing.assert_array_equal(O.matmul(op, a, b), O.ref_matmul(op, a, b))


@needs_ref
def test_ref_bitexact_rowwise():
    r = rng(42)
    x = (3 * r.standard_normal((20, 300))).astype(f32)
    g = r.standard_normal(x.shape).astype(f32)
    y, dx = O.ref_softmax(x, g)
    np.testing.assert_array_equal(O.softmax(x), y)
    np.testing.assert_array_equal(O.softmax_backward(g, O.softmax(x)), dx)
    w = (1 + 0.02 * r.standard_normal(300)).astype(f32)
    b = (0.02 * r.standard_normal(300)).astype(f32)
    yr, dxr, dwr, dbr = O.ref_layernorm(x, w, b, 1e-5, g)
    yo, mu, rs = O.layernorm(x, w, b, 1e-5, stats=True)
    np.testing.assert_array_equal(yo, yr)
    for got, ref in zip(O.layernorm_backward(g, x, w, mu, rs), (dxr, dwr, dbr)):
        np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(O.layernorm(x, w, b), O.ref_layernorm(x, w, b))


@needs_ref
@pytest.mark.parametrize("causal", [0, 1])
def test_ref_bitexact_attention(causal):
    r = rng(43)
    q, k, v, do = (r.standard_normal((3, 45, 24)).astype(f32) for _ in range(4))
    o, dq, dk, dv = O.ref_attention(q, k, v, causal, do)
    np.testing.assert_array_equal(O.attention(q, k, v, causal), o)
    for got, ref in zip(O.attention_backward(q, k, v, do, causal), (dq, dk, dv)):
        np.testing.assert_array_equal(got, ref)


# --------------------------------------------------------- planted mistakes
# The checks above must fail for plausible mistakes in an oracle.  Each test
# builds a deliberately wrong variant on the CPU and asserts the check rejects it.

def test_planted_transposed_operand_is_caught():
    a = np.array([[1, 2, 3], [4, 5, 6]], f32)
    b = np.array([[7, 8], [9, 10], [11, 12]], f32)
    wrong = O.matmul("nt", a, np.ascontiguousarray(b.reshape(2, 3)))  # B read with the wrong layout
    assert not np.array_equal(wrong, [[58, 64], [139, 154]])


def test_planted_dropped_term_is_caught():
    z = np.load(GOLDEN / "layernorm_32x257.npz")
    _, mu, rs = O.layernorm(z["x"], z["w"], z["b"], 1e-5, stats=True)
    dx = O.layernorm_backward(z["gy"], z["x"], z["w"], mu, rs)[0]
    gg = z["gy"] * z["w"]
    wrong = rs[:, None] * (gg - gg.mean(1, keepdims=True))  # dropped the xhat term
    assert np.abs(wrong - z["dx"]).max() > 1e-2
    assert np.abs(dx - z["dx"]).max() == 0


def test_planted_wrong_sign_is_caught():
    z = np.load(GOLDEN / "softmax_32x257.npz")
    wrong = z["y"] * (z["g"] + (z["g"] * z["y"]).sum(1, keepdims=True))
    assert np.abs(wrong - z["dx"]).max() > 1e-3
