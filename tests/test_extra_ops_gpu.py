"""GPU parity of dropout (the reference's Philox-4x32-10 stream, bit-exact),
apply_causal_mask (bit-exact, forward and backward) and the batched products
bmm / bmm_a_bt / bmm_at_b (GEMM tolerance 1e-4*sqrt(K), both metrics) against
the oracle, plus the behaviour the reference's tests/python/test_dropout.py,
test_bmm.py and test_attention.py assert."""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle as O
from conftest import assert_close, gemm_tol
from devutil import dev, host

pytestmark = pytest.mark.gpu
f32 = np.float32


# ---------------------------------------------------------------- dropout
@pytest.mark.parametrize("n", [1, 3, 128, 4097, 1_000_003])
@pytest.mark.parametrize("p", [0.1, 0.3, 0.9])
def test_dropout_bitexact_vs_oracle(gpu, n, p):
    x = np.random.default_rng(n).standard_normal(n).astype(f32)
    gpu.manual_seed(2026)
    tx = dev(gpu, x, True)
    y = gpu.dropout(tx, p)
    out, mask = O.dropout(x, p, 2026)
    np.testing.assert_array_equal(host(gpu, y), out)
    g = np.random.default_rng(n + 1).standard_normal(n).astype(f32)
    y.backward(dev(gpu, g))
    np.testing.assert_array_equal(host(gpu, tx.grad), O.mul(g, mask))


def test_dropout_seed_stream_advances_per_call(gpu):
    # cppsrc/ops/dropout.cpp:63-75: each call draws the next seed
    x = np.random.default_rng(0).standard_normal(999).astype(f32)
    gpu.manual_seed(2**40 + 5)
    a = host(gpu, gpu.dropout(dev(gpu, x), 0.5))
    b = host(gpu, gpu.dropout(dev(gpu, x), 0.5))
    np.testing.assert_array_equal(a, O.dropout(x, 0.5, 2**40 + 5)[0])
    np.testing.assert_array_equal(b, O.dropout(x, 0.5, 2**40 + 6)[0])


def test_dropout_reference_behaviour(gpu):
    # tests/python/test_dropout.py:16-73 on device tensors
    gpu.manual_seed(0)
    out = host(gpu, gpu.dropout(dev(gpu, np.ones(20000, f32)), 0.3))
    assert abs(float((out == 0).mean()) - 0.3) < 0.02
    gpu.manual_seed(1)
    out = host(gpu, gpu.dropout(dev(gpu, np.full(1000, 2.0, f32)), 0.4))
    np.testing.assert_allclose(out[out != 0], 2.0 / 0.6, atol=1e-5)
    x = dev(gpu, np.random.default_rng(0).standard_normal(50).astype(f32))
    gpu.manual_seed(123)
    a = host(gpu, gpu.dropout(x, 0.5))
    gpu.manual_seed(123)
    np.testing.assert_array_equal(a, host(gpu, gpu.dropout(x, 0.5)))
    gpu.manual_seed(7)
    ones = dev(gpu, np.ones(200, f32))
    assert not np.array_equal(host(gpu, gpu.dropout(ones, 0.5)), host(gpu, gpu.dropout(ones, 0.5)))
    x_np = np.random.default_rng(0).standard_normal((4, 8)).astype(f32)
    x = dev(gpu, x_np, True)
    gpu.manual_seed(42)
    out = gpu.dropout(x, 0.4)
    gpu.sum_all(out).backward()
    expect = np.where(host(gpu, out) != 0, 1.0 / 0.6, 0.0).astype(f32)
    np.testing.assert_allclose(host(gpu, x.grad), expect, atol=1e-5)
    x = dev(gpu, x_np, True)
    out = gpu.dropout(x, 0.0)
    np.testing.assert_array_equal(host(gpu, out), x_np)
    gpu.sum_all(out).backward()
    np.testing.assert_array_equal(host(gpu, x.grad), np.ones_like(x_np))
    for bad in (1.0, -0.1, 1.5):
        with pytest.raises(ValueError):
            gpu.dropout(dev(gpu, x_np), bad)


def test_dropout_module_and_strided_input(gpu):
    from aargrad import nn
    drop = nn.Dropout(0.5)
    x_np = np.random.default_rng(0).standard_normal((64, 48)).astype(f32)
    drop.eval()
    np.testing.assert_array_equal(host(gpu, drop(dev(gpu, x_np))), x_np)
    drop.train()
    gpu.manual_seed(99)
    out = host(gpu, drop(dev(gpu, np.ones(1000, f32))))
    assert 0.4 < float((out == 0).mean()) < 0.6
    # a transposed view is made contiguous first, so the stream follows the
    # logical (row-major) element order of the view
    xt = gpu.transpose(dev(gpu, x_np), 0, 1)
    gpu.manual_seed(5)
    got = host(gpu, gpu.dropout(xt, 0.25))
    want = O.dropout(np.ascontiguousarray(x_np.T), 0.25, 5)[0].reshape(48, 64)
    np.testing.assert_array_equal(got, want)
    # a slice at an odd offset is contiguous but not 16-byte aligned: the
    # element-wise kernel takes it
    flat = np.random.default_rng(1).standard_normal(10001).astype(f32)
    sl = gpu.slice(dev(gpu, flat), 0, 1, 10001)
    gpu.manual_seed(6)
    np.testing.assert_array_equal(host(gpu, gpu.dropout(sl, 0.6)), O.dropout(flat[1:], 0.6, 6)[0])


# ------------------------------------------------------------ causal mask
@pytest.mark.parametrize("shape", [(1, 1), (4, 4), (3, 17, 17), (2, 3, 64, 64), (2, 257, 257), (1, 1024, 1024)])
def test_causal_mask_fwd_bwd(gpu, shape):
    rng = np.random.default_rng(sum(shape))
    x = rng.standard_normal(shape).astype(f32)
    g = rng.standard_normal(shape).astype(f32)
    tx = dev(gpu, x, True)
    y = gpu.apply_causal_mask(tx)
    np.testing.assert_array_equal(host(gpu, y), O.causal_mask(x))
    y.backward(dev(gpu, g))
    np.testing.assert_array_equal(host(gpu, tx.grad), O.causal_mask(g, 0.0))


def test_causal_mask_view_softmax_and_errors(gpu):
    # tests/python/test_attention.py:52-60
    s = np.random.default_rng(2).standard_normal((4, 4)).astype(f32)
    probs = host(gpu, gpu.softmax(gpu.apply_causal_mask(dev(gpu, s))))
    assert np.all(probs[np.triu_indices(4, 1)] == 0.0)
    x = np.random.default_rng(3).standard_normal((2, 33, 33)).astype(f32)
    xt = gpu.transpose(dev(gpu, x), 1, 2)
    np.testing.assert_array_equal(host(gpu, gpu.apply_causal_mask(xt)),
                                  O.causal_mask(np.ascontiguousarray(x.transpose(0, 2, 1))))
    for bad in ((5,), (3, 4)):
        with pytest.raises(ValueError):
            gpu.apply_causal_mask(dev(gpu, np.zeros(bad, f32)))


def _attention_np(q, k, v, causal):
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    s = q @ k.T / math.sqrt(q.shape[-1])
    if causal:
        s = np.where(np.triu(np.ones(s.shape, bool), 1), -np.inf, s)
    e = np.exp(s - s.max(-1, keepdims=True))
    return (e / e.sum(-1, keepdims=True)) @ v


@pytest.mark.parametrize("T,d", [(4, 8), (6, 8), (100, 64), (513, 32)])
def test_scaled_dot_product_attention(gpu, T, d):
    # tests/python/test_attention.py:30-50, :96-110
    from aargrad import nn
    rng = np.random.default_rng(T)
    q, k, v, go = (rng.standard_normal((T, d)).astype(f32) for _ in range(4))
    for causal in (False, True):
        tq = dev(gpu, q, True)
        out = nn.scaled_dot_product_attention(tq, dev(gpu, k), dev(gpu, v), causal=causal)
        assert_close(host(gpu, out), _attention_np(q, k, v, causal), 1e-4, f"sdpa causal={causal}")
        out.backward(dev(gpu, go))
        dq = O.attention_backward(q[None], k[None], v[None], go[None], causal)[0]
        assert_close(host(gpu, tq.grad), dq[0], 1e-4, f"sdpa dq causal={causal}")


# ----------------------------------------------------------- batched GEMM
def _bmm_case(op, lead, M, N, K, rng):
    a_shape = lead + ((K, M) if op == "bmm_at_b" else (M, K))
    b_shape = lead + ((N, K) if op == "bmm_a_bt" else (K, N))
    return rng.standard_normal(a_shape).astype(f32), rng.standard_normal(b_shape).astype(f32)


def _bmm_oracle(op, a, b):
    lead = a.shape[:-2]
    n = int(np.prod(lead))
    a3 = a.reshape((n,) + a.shape[-2:])
    b3 = b.reshape((n,) + b.shape[-2:])
    c = O.bmm(op, a3, b3)
    return c.reshape(lead + c.shape[-2:])


@pytest.mark.parametrize("op", O.BMM_OPS)
def test_bmm_one_tile_per_cu_grid(gpu, op):
    """2 x 8192 x 384 x 384: a batched grid of one 128 x 192 tile per CU (256
    tiles, as the single 16384 x 384 x 384 product), which the planner runs on
    the 8-wave 128 x 192 tile for bmm and bmm_a_bt.  Forward only, against a
    float64 numpy product (the oracle's loops take seconds per product at
    this size)."""
    rng = np.random.default_rng(8192)
    a, b = _bmm_case(op, (2,), 8192, 384, 384, rng)
    c = getattr(gpu, op)(dev(gpu, a), dev(gpu, b))
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    if op == "bmm":
        want = a64 @ b64
    elif op == "bmm_a_bt":
        want = a64 @ b64.transpose(0, 2, 1)
    else:
        want = a64.transpose(0, 2, 1) @ b64
    assert tuple(c.shape) == want.shape
    assert_close(host(gpu, c), want, gemm_tol(384), op)


@pytest.mark.parametrize("op", O.BMM_OPS)
@pytest.mark.parametrize("lead,M,N,K", [((2, 3), 4, 6, 5), ((6,), 1, 1, 1), ((12,), 256, 256, 64),
                                        ((4,), 300, 77, 129), ((2, 2), 64, 520, 33), ((3,), 5, 7, 0),
                                        ((0,), 4, 4, 4)])
def test_bmm_variants_fwd_bwd(gpu, op, lead, M, N, K):
    rng = np.random.default_rng(M * 7 + N + K)
    a, b = _bmm_case(op, lead, M, N, K, rng)
    fn = getattr(gpu, op)
    ta, tb = dev(gpu, a, True), dev(gpu, b, True)
    c = fn(ta, tb)
    want = _bmm_oracle(op, a, b)
    assert tuple(c.shape) == want.shape
    if want.size == 0:
        return
    assert_close(host(gpu, c), want, gemm_tol(max(K, 1)), f"{op} fwd")
    if K == 0:
        return
    g = rng.standard_normal(want.shape).astype(f32)
    c.backward(dev(gpu, g))
    # cppsrc/ops/bmm.cpp backward formulas, evaluated with the oracle
    if op == "bmm":
        da, db = _bmm_oracle("bmm_a_bt", g, b), _bmm_oracle("bmm_at_b", a, g)
    elif op == "bmm_a_bt":
        da, db = _bmm_oracle("bmm", g, b), _bmm_oracle("bmm_at_b", g, a)
    else:
        da, db = _bmm_oracle("bmm_a_bt", b, g), _bmm_oracle("bmm", a, g)
    assert_close(host(gpu, ta.grad), da, gemm_tol(want.shape[-1]), f"{op} dA")
    assert_close(host(gpu, tb.grad), db, gemm_tol(max(M, 1)), f"{op} dB")


def test_bmm_strided_operands(gpu):
    # transposed views take the matching GEMM layout without a copy; sliced
    # (non-unit inner stride) views are copied once
    rng = np.random.default_rng(11)
    a = rng.standard_normal((5, 96, 40)).astype(f32)
    b = rng.standard_normal((5, 72, 40)).astype(f32)
    ta, tb = dev(gpu, a), dev(gpu, b)
    got = host(gpu, gpu.bmm(ta, gpu.transpose(tb, 1, 2)))
    assert_close(got, O.bmm("bmm_a_bt", a, b), gemm_tol(40), "bmm with transposed B")
    got = host(gpu, gpu.bmm_a_bt(gpu.transpose(dev(gpu, a.transpose(0, 2, 1).copy()), 1, 2), tb))
    assert_close(got, O.bmm("bmm_a_bt", a, b), gemm_tol(40), "bmm_a_bt with transposed A")
    big = rng.standard_normal((5, 96, 80)).astype(f32)
    sl = gpu.slice(dev(gpu, big), 2, 10, 50)
    got = host(gpu, gpu.bmm_a_bt(sl, tb))
    assert_close(got, O.bmm("bmm_a_bt", np.ascontiguousarray(big[:, :, 10:50]), b), gemm_tol(40), "sliced A")
    # batch-dimension transpose of a rank-4 tensor (unfoldable leading dims)
    a4 = rng.standard_normal((3, 4, 16, 24)).astype(f32)
    b4 = rng.standard_normal((4, 3, 24, 8)).astype(f32)
    ta4 = gpu.transpose(dev(gpu, a4.transpose(1, 0, 2, 3).copy()), 0, 1)
    got = host(gpu, gpu.bmm(ta4, gpu.transpose(dev(gpu, b4), 0, 1)))
    want = _bmm_oracle("bmm", a4, np.ascontiguousarray(b4.transpose(1, 0, 2, 3)))
    assert_close(got, want, gemm_tol(24), "rank-4 batch views")


@pytest.mark.parametrize("op", O.BMM_OPS)
def test_bmm_more_batches_than_one_launch(gpu, op):
    # 70001 batches: a launch carries at most 65535 on blockIdx.z, so the
    # second launch's operand offsets are exercised (forward and both grads)
    rng = np.random.default_rng(70001)
    a, b = _bmm_case(op, (70001,), 3, 5, 4, rng)
    ta, tb = dev(gpu, a, True), dev(gpu, b, True)
    c = getattr(gpu, op)(ta, tb)
    assert_close(host(gpu, c), _bmm_oracle(op, a, b), gemm_tol(4), f"{op} fwd")
    g = rng.standard_normal((70001, 3, 5)).astype(f32)
    c.backward(dev(gpu, g))
    if op == "bmm":
        da, db = _bmm_oracle("bmm_a_bt", g, b), _bmm_oracle("bmm_at_b", a, g)
    elif op == "bmm_a_bt":
        da, db = _bmm_oracle("bmm", g, b), _bmm_oracle("bmm_at_b", g, a)
    else:
        da, db = _bmm_oracle("bmm_a_bt", b, g), _bmm_oracle("bmm", a, g)
    assert_close(host(gpu, ta.grad), da, gemm_tol(5), f"{op} dA")
    assert_close(host(gpu, tb.grad), db, gemm_tol(3), f"{op} dB")


def test_bmm_errors(gpu):
    z = lambda *s: dev(gpu, np.zeros(s, f32))  # noqa: E731
    with pytest.raises(ValueError):
        gpu.bmm(z(2, 3, 4), z(2, 5, 6))
    with pytest.raises(ValueError):
        gpu.bmm(z(2, 3, 4), z(3, 4, 6))
    with pytest.raises(ValueError):
        gpu.bmm(z(2, 3, 4), z(2, 3, 4, 5))
    with pytest.raises(ValueError):
        gpu.bmm(z(3), z(3))
