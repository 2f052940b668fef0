"""Pins the oracle's GPT-step ops (sub, mul, scale, relu, gelu, add_bias,
bias_grad, sum_all, scaled_add, embedding, cross_entropy, adamw): reference
known answers restated, float64 closed forms, finite differences, and
bit-exact agreement with oracle/_ref (the reference's own CPU build)."""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle as O

f32 = np.float32
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference tree)")


def test_elementwise_kats():
    # tests/cpp/test_elementwise.cpp:20-56, :127-148
    a = np.array([1, 2, 3, 4], f32)
    b = np.array([5, 6, 7, 8], f32)
    np.testing.assert_array_equal(O.mul(a, b), [5, 12, 21, 32])
    np.testing.assert_array_equal(O.sub(b, a), [4, 4, 4, 4])
    np.testing.assert_array_equal(O.relu(np.array([-1, 0, 2, -3.5], f32)), [0, 0, 2, 0])
    np.testing.assert_array_equal(O.scale(a, 0.5), [0.5, 1, 1.5, 2])
    assert O.sum_all(np.arange(1, 11, dtype=f32)) == 55.0
    assert O.sum_all(np.array([3.5], f32)) == 3.5


def test_gelu_closed_form_and_derivative():
    x = np.linspace(-6, 6, 1001).astype(f32)
    x64 = x.astype(np.float64)
    erf = np.vectorize(math.erf)
    np.testing.assert_allclose(O.gelu(x), 0.5 * x64 * (1 + erf(x64 / math.sqrt(2))), rtol=1e-6, atol=1e-7)
    h = 1e-4
    num = (0.5 * (x64 + h) * (1 + erf((x64 + h) / math.sqrt(2))) -
           0.5 * (x64 - h) * (1 + erf((x64 - h) / math.sqrt(2)))) / (2 * h)
    np.testing.assert_allclose(O.gelu_backward(np.ones_like(x), x), num, atol=1e-5)


def test_bias_add_and_grad_closed_form():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((50, 24)).astype(f32)
    bias = rng.standard_normal(24).astype(f32)
    np.testing.assert_array_equal(O.add_bias(x, bias), x + bias)
    g = rng.standard_normal((50, 24)).astype(f32)
    np.testing.assert_allclose(O.bias_grad(g, 24), g.astype(np.float64).sum(0), rtol=1e-5, atol=1e-5)


def test_scaled_add_is_sgd():
    # aargrad/optim.py:14-18: p += -lr * g
    p = np.array([1, 2, 3], f32)
    g = np.array([10, 20, 30], f32)
    np.testing.assert_array_equal(O.scaled_add(p, g, -0.1), p + f32(-0.1) * g)


def test_embedding_kats():
    # tests/python/test_embedding.py:16-26 and the repeated-id scatter-add
    rng = np.random.default_rng(0)
    w = rng.standard_normal((7, 4)).astype(f32)
    ids = np.array([[0, 1, 5], [3, 0, 6]], np.int64)
    np.testing.assert_array_equal(O.embedding(w, ids), w[ids])
    g = rng.standard_normal((6, 3)).astype(f32)
    ids2 = np.array([0, 2, 0, 1, 2, 0], np.int64)
    ref = np.zeros((5, 3))
    np.add.at(ref, ids2, g.astype(np.float64))
    np.testing.assert_allclose(O.embedding_backward(g, ids2, 5), ref, rtol=1e-6, atol=1e-6)
    with pytest.raises(IndexError):
        O.embedding(w, np.array([7], np.int64))


def _ce64(logits, targets, ignore=-100):
    # tests/python/test_cross_entropy.py:17-25
    mask = targets != ignore
    if not mask.any():
        return 0.0
    l64 = logits.astype(np.float64)
    m = l64.max(-1, keepdims=True)
    lse = (m + np.log(np.exp(l64 - m).sum(-1, keepdims=True)))[:, 0]
    return float((lse - l64[np.arange(len(targets)), targets.clip(min=0)])[mask].mean())


def test_cross_entropy_kats_and_grad():
    rng = np.random.default_rng(0)
    logits = rng.standard_normal((6, 5)).astype(f32)
    t = np.array([0, 4, 2, 1, 3, 0], np.int64)
    assert abs(O.cross_entropy(logits, t) - _ce64(logits, t)) < 1e-6
    t2 = np.array([2, -100, 1, -100, 0, 3], np.int64)
    assert abs(O.cross_entropy(logits, t2) - _ce64(logits, t2)) < 1e-6
    assert O.cross_entropy(logits, np.full(6, -100, np.int64)) == 0.0
    # gradient: (softmax - onehot) * go / active, finite differences
    go = 1.3
    d = O.cross_entropy_backward(go, logits, t2)
    num = np.zeros(logits.shape)
    for idx in np.ndindex(*logits.shape):
        p, m = logits.astype(np.float64).copy(), logits.astype(np.float64).copy()
        p[idx] += 1e-6
        m[idx] -= 1e-6
        num[idx] = go * (_ce64(p, t2) - _ce64(m, t2)) / 2e-6
    np.testing.assert_allclose(d, num, atol=1e-5)
    with pytest.raises(IndexError):
        O.cross_entropy(logits, np.array([0, 5, 0, 0, 0, 0], np.int64))


def test_adamw_closed_form():
    rng = np.random.default_rng(1)
    p, g = rng.standard_normal(100).astype(f32), rng.standard_normal(100).astype(f32)
    m, v = np.zeros(100, f32), np.zeros(100, f32)
    lr, b1, b2, eps, wd = 1e-3, 0.9, 0.999, 1e-8, 0.01
    # the op's constants are fp32: 1 - beta computed in fp32 (cppsrc/ops/adamw.cpp:33-35)
    omb1, omb2 = float(f32(1) - f32(b1)), float(f32(1) - f32(b2))
    pn, mn, vn = O.adamw(p, g, m, v, lr, b1, b2, eps, wd, omb1, omb2)
    m64 = omb1 * g.astype(np.float64)
    v64 = omb2 * g.astype(np.float64) ** 2
    p64 = p * float(f32(1) - f32(lr) * f32(wd)) - lr * (m64 / omb1) / (np.sqrt(v64 / omb2) + eps)
    np.testing.assert_allclose(mn, m64, rtol=1e-6)
    np.testing.assert_allclose(vn, v64, rtol=1e-5)
    np.testing.assert_allclose(pn, p64, rtol=1e-5, atol=1e-7)


@needs_ref
def test_ref_bitexact_nn_ops():
    rng = np.random.default_rng(7)
    a, b, g = (rng.standard_normal(777).astype(f32) for _ in range(3))
    for op, bb in (("sub", b), ("mul", b), ("scale", None), ("relu", None), ("gelu", None)):
        y, da = O.ref_elementwise(op, a, bb, 0.37, g)
        mine = {"sub": O.sub(a, b), "mul": O.mul(a, b), "scale": O.scale(a, 0.37), "relu": O.relu(a),
                "gelu": O.gelu(a)}[op]
        np.testing.assert_array_equal(y, mine)
        if op == "relu":
            np.testing.assert_array_equal(da, O.relu_backward(g, a))
        if op == "gelu":
            np.testing.assert_array_equal(da, O.gelu_backward(g, a))
    x = rng.standard_normal((33, 20)).astype(f32)
    bias = rng.standard_normal(20).astype(f32)
    gg = rng.standard_normal((33, 20)).astype(f32)
    y, db = O.ref_add_bias(x, bias, gg)
    np.testing.assert_array_equal(y, O.add_bias(x, bias))
    np.testing.assert_array_equal(db, O.bias_grad(gg, 20))
    assert O.ref_sum_all(a) == O.sum_all(a)
    w = rng.standard_normal((65, 16)).astype(f32)
    ids = rng.integers(0, 65, 90)
    ge = rng.standard_normal((90, 16)).astype(f32)
    y, dw = O.ref_embedding(w, ids, ge)
    np.testing.assert_array_equal(y, O.embedding(w, ids))
    np.testing.assert_array_equal(dw, O.embedding_backward(ge, ids, 65))
    lg = rng.standard_normal((90, 65)).astype(f32)
    t = rng.integers(0, 65, 90)
    t[5] = -100
    loss, dl = O.ref_cross_entropy(lg, t, -100, 0.8)
    assert loss == O.cross_entropy(lg, t)
    np.testing.assert_array_equal(dl, O.cross_entropy_backward(0.8, lg, t))
    m, v = 0.1 * b, np.abs(g) * 0.1
    for x1, x2 in zip(O.ref_adamw(a, g, m, v, 1e-3, 0.9, 0.999, 1e-8, 0.01, 0.19, 0.002),
                      O.adamw(a, g, m, v, 1e-3, 0.9, 0.999, 1e-8, 0.01, 0.19, 0.002)):
        np.testing.assert_array_equal(x1, x2)


@needs_ref
def test_ref_lm_step_matches_oracle_forward():
    """The reference Shakespeare-model step (oracle/_ref, dropout off) has the
    loss of the oracle's forward of the same model, and AdamW lowers it."""
    import lmutil

    cfg = {"vocab": 65, "ctx": 16, "layers": 2, "d_model": 32, "heads": 4}
    rng = np.random.default_rng(3)
    shapes = [(65, 32), (16, 32)] + [(32,), (32,), (96, 32), (32, 32), (32,), (32,), (128, 32), (128,),
                                     (32, 128), (32,)] * 2 + [(32,), (32,), (65, 32)]
    params = [(1.0 + 0.1 * rng.standard_normal(s)) if len(s) == 1 and i > 1 else 0.2 * rng.standard_normal(s)
              for i, s in enumerate(shapes)]
    params = [np.ascontiguousarray(p, np.float32) for p in params]
    m = [np.zeros_like(p) for p in params]
    v = [np.zeros_like(p) for p in params]
    ids = rng.integers(0, 65, (3, 16))
    tgt = rng.integers(0, 65, (3, 16))
    lcfg = {"vocab_size": 65, "max_seq_len": 16, "n_layer": 2, "n_head": 4, "d_model": 32}
    want = float(O.cross_entropy(lmutil.oracle_forward(params, lcfg, ids).reshape(-1, 65), tgt.reshape(-1)))
    kw = dict(dropout=0.0, seed=0, lr=1e-2, betas=(0.9, 0.95), eps=1e-8, wd=0.01)
    loss0 = O.ref_lm_step(cfg, params, m, v, ids, tgt, t=1, **kw)
    assert abs(loss0 - want) <= 1e-5 * max(abs(want), 1)
    losses = [O.ref_lm_step(cfg, params, m, v, ids, tgt, t=t, **kw) for t in range(2, 6)]
    assert losses[-1] < loss0


def _fanin_inputs(n=4099, seed=31):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n).astype(f32)
    w = rng.standard_normal((4, n)).astype(f32)
    g = rng.standard_normal(n).astype(f32)
    return x, w, g


def _fanin_in_order(x, w, g, order):
    """x.grad of the fan-in graph with h's three incoming gradients summed in
    `order` (indices into (g*w1, g*0.75, g*w2)), in float32."""
    parts = [g * w[1], g * f32(0.75), g * w[2]]
    acc = parts[order[0]]
    for i in order[1:]:
        acc = (acc + parts[i]).astype(f32)
    return (acc * w[0] + g * w[3]).astype(f32)


@needs_ref
def test_reference_fanin_summation_order():
    # The reference's autograd (cppsrc/autograd/backward.cpp:50-113) runs the
    # nodes in reverse DFS post-order, a node's inputs pushed in order and the
    # last popped first.  For root = ((u + v) + z) + t that runs u, v, z (the
    # consumers of h) in that order, so h's gradient is ((g*w1 + 0.75 g) + g*w2),
    # and then x's: (h_grad * w0) + g*w3.  Bit-exact against the reference.
    x, w, g = _fanin_inputs()
    got = O.ref_fanin_graph(x, w, g)
    np.testing.assert_array_equal(got, _fanin_in_order(x, w, g, (0, 1, 2)))
    # the inputs separate the orders: any other summation order differs somewhere
    for other in ((0, 2, 1), (1, 0, 2), (1, 2, 0), (2, 0, 1), (2, 1, 0)):
        alt = _fanin_in_order(x, w, g, other)
        if other != (1, 0, 2):  # (a + b) + c == (b + a) + c bit for bit
            assert not np.array_equal(alt, got), other
