"""Softmax and layernorm parity on the GPU against the oracle: the reference
tests' known answers, the golden vectors from the reference CPU build, the
BASELINE config-3 sizes in full, odd widths (scalar and wide-row kernels) and
bit-reproducible dgamma/dbeta.  Tolerance 1e-4 on both error metrics."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from conftest import TOL, assert_close
from devutil import Abi, dev, host

pytestmark = pytest.mark.gpu
f32 = np.float32
GOLDEN = O.HERE.parent / "tests" / "golden"


def test_softmax_kats(gpu):
    # tests/cpp/test_softmax.cpp:20-65
    y = host(gpu, gpu.softmax(dev(gpu, np.array([1, 2, 3, 4], f32))))
    assert abs(y.sum() - 1) < 1e-6 and (y > 0).all()
    np.testing.assert_allclose(host(gpu, gpu.softmax(dev(gpu, np.zeros(5, f32)))), 0.2, rtol=1e-6)
    y = host(gpu, gpu.softmax(dev(gpu, np.array([1000, 1001, 1002], f32))))
    assert np.isfinite(y).all() and abs(y.sum() - 1) < 1e-6 and y[0] < y[1] < y[2]
    x = np.array([[1, 2, 3, 4], [-1, -2, -3, -4], [100, 100, 100, 100]], f32)
    y = host(gpu, gpu.softmax(dev(gpu, x)))
    np.testing.assert_allclose(y.sum(1), 1, atol=1e-5)
    np.testing.assert_array_equal(y[2], np.full(4, 0.25, f32))


def test_layernorm_kats(gpu):
    # tests/cpp/test_layernorm.cpp:27-98
    ones, zeros = np.ones(8, f32), np.zeros(8, f32)
    y = host(gpu, gpu.layernorm(dev(gpu, np.arange(1, 9, dtype=f32)), dev(gpu, ones), dev(gpu, zeros)))
    assert abs(y.mean()) < 1e-5 and abs(((y - y.mean()) ** 2).mean() - 1) < 1e-3
    y = host(gpu, gpu.layernorm(dev(gpu, np.arange(1, 9, dtype=f32)), dev(gpu, 2 * ones), dev(gpu, 3 + zeros)))
    assert abs(y.mean() - 3) < 1e-5 and abs(((y - y.mean()) ** 2).mean() - 4) < 1e-2
    y = host(gpu, gpu.layernorm(dev(gpu, np.full(6, 7, f32)), dev(gpu, np.full(6, 5, f32)),
                                dev(gpu, np.full(6, -1, f32))))
    np.testing.assert_allclose(y, -1, atol=1e-3)
    x = np.array([[1, 2, 3, 4], [10, 20, 30, 40], [-5, -3, -1, 1]], f32)
    y = host(gpu, gpu.layernorm(dev(gpu, x), dev(gpu, np.ones(4, f32)), dev(gpu, np.zeros(4, f32))))
    np.testing.assert_allclose(y.mean(1), 0, atol=1e-5)
    np.testing.assert_allclose(((y - y.mean(1, keepdims=True)) ** 2).mean(1), 1, atol=1e-3)


def test_layernorm_dbias_row_sum_on_device(gpu):
    # tests/cpp/test_autograd_ops.cpp:443-460
    x = np.array([[1, 2, 3, 4], [-1, -2, -3, -4], [0.5, 1.5, 2.5, 3.5]], f32)
    b = dev(gpu, np.zeros(4, f32), True)
    y = gpu.layernorm(dev(gpu, x), dev(gpu, np.ones(4, f32)), b)
    y.backward(dev(gpu, np.ones_like(x)))
    np.testing.assert_array_equal(host(gpu, b.grad), np.full(4, 3.0, f32))


def test_golden_softmax(gpu):
    z = np.load(GOLDEN / "softmax_32x257.npz")
    x = dev(gpu, z["x"], True)
    y = gpu.softmax(x)
    y.backward(dev(gpu, z["g"]))
    yh = host(gpu, y)
    # the reference's own CudaMatchesCpu bound (tests/cpp/test_softmax.cpp:85-91) ...
    assert np.all(np.abs(yh - z["y"]) <= 1e-5 * np.maximum(np.abs(z["y"]), 1) + 1e-6)
    # ... and the parity bar
    assert_close(yh, z["y"], TOL, "y")
    assert_close(host(gpu, x.grad), z["dx"], TOL, "dx")


def test_golden_layernorm(gpu):
    z = np.load(GOLDEN / "layernorm_32x257.npz")
    x, w, b = dev(gpu, z["x"], True), dev(gpu, z["w"], True), dev(gpu, z["b"], True)
    y = gpu.layernorm(x, w, b, float(z["eps"]))
    y.backward(dev(gpu, z["gy"]))
    yh = host(gpu, y)
    assert np.all(np.abs(yh - z["y"]) <= 1e-4 * np.maximum(np.abs(z["y"]), 1) + 1e-5)
    assert_close(yh, z["y"], TOL, "y")
    assert_close(host(gpu, x.grad), z["dx"], TOL, "dx")
    assert_close(host(gpu, w.grad), z["dw"], TOL, "dw")
    assert_close(host(gpu, b.grad), z["db"], TOL, "db")


def config3_inputs(rows, cols, seed=0):
    # draw order x, gamma, beta, g
    rng = np.random.default_rng(seed)
    x = (3 * rng.standard_normal((rows, cols))).astype(f32)
    w = (1 + 0.02 * rng.standard_normal(cols)).astype(f32)
    b = (0.02 * rng.standard_normal(cols)).astype(f32)
    g = rng.standard_normal((rows, cols)).astype(f32)
    return x, w, b, g


@pytest.mark.parametrize("cols", [384, 768, 4096])
def test_config3_softmax_full(gpu, cols):
    x, _, _, g = config3_inputs(65536, cols)
    tx = dev(gpu, x, True)
    y = gpu.softmax(tx)
    y.backward(dev(gpu, g))
    y_ref = O.softmax(x)
    assert_close(host(gpu, y), y_ref, TOL, "softmax y")
    assert_close(host(gpu, tx.grad), O.softmax_backward(g, y_ref), TOL, "softmax dx")


@pytest.mark.parametrize("cols", [384, 768, 4096])
def test_config3_layernorm_full(gpu, cols):
    x, w, b, g = config3_inputs(65536, cols)
    tx, tw, tb = dev(gpu, x, True), dev(gpu, w, True), dev(gpu, b, True)
    y = gpu.layernorm(tx, tw, tb, 1e-5)
    y.backward(dev(gpu, g))
    y_ref, mu, rs = O.layernorm(x, w, b, 1e-5, stats=True)
    dx, dw, db = O.layernorm_backward(g, x, w, mu, rs)
    assert_close(host(gpu, y), y_ref, TOL, "ln y")
    assert_close(host(gpu, tx.grad), dx, TOL, "ln dx")
    assert_close(host(gpu, tw.grad), dw, TOL, "ln dgamma")
    assert_close(host(gpu, tb.grad), db, TOL, "ln dbeta")


@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 3), (5, 64), (33, 257), (9, 1000), (4, 2049), (3, 8192),
                                       (2, 9000), (300, 96), (50, 150), (17, 700), (6, 190), (5000, 768)])
def test_odd_widths_vs_oracle(gpu, rows, cols):
    x, w, b, g = config3_inputs(rows, cols, seed=rows * 31 + cols)
    tx = dev(gpu, x, True)
    y = gpu.softmax(tx)
    y.backward(dev(gpu, g))
    y_ref = O.softmax(x)
    assert_close(host(gpu, y), y_ref, TOL, "softmax")
    assert_close(host(gpu, tx.grad), O.softmax_backward(g, y_ref), TOL, "softmax dx")
    tx, tw, tb = dev(gpu, x, True), dev(gpu, w, True), dev(gpu, b, True)
    yl = gpu.layernorm(tx, tw, tb, 1e-5)
    yl.backward(dev(gpu, g))
    yl_ref, mu, rs = O.layernorm(x, w, b, 1e-5, stats=True)
    dx, dw, db = O.layernorm_backward(g, x, w, mu, rs)
    assert_close(host(gpu, yl), yl_ref, TOL, "ln")
    assert_close(host(gpu, tx.grad), dx, TOL, "ln dx")
    assert_close(host(gpu, tw.grad), dw, TOL, "ln dw")
    assert_close(host(gpu, tb.grad), db, TOL, "ln db")


@pytest.mark.parametrize("rows,cols", [(3, 140000), (2, 140001)])
def test_layernorm_backward_wide_reduce_grid(gpu, rows, cols):
    """Rows so wide that the dgamma/dbeta reduce has more column blocks (70000
    float4 blocks; 280002 single columns) than its 2^16-workgroup grid, which
    then strides over them.  Layernorm only: at 140001 columns the oracle's
    sequential softmax sum carries more rounding than the tolerance."""
    x, w, b, g = config3_inputs(rows, cols, seed=rows * 31 + cols)
    tx, tw, tb = dev(gpu, x, True), dev(gpu, w, True), dev(gpu, b, True)
    yl = gpu.layernorm(tx, tw, tb, 1e-5)
    yl.backward(dev(gpu, g))
    yl_ref, mu, rs = O.layernorm(x, w, b, 1e-5, stats=True)
    dx, dw, db = O.layernorm_backward(g, x, w, mu, rs)
    assert_close(host(gpu, yl), yl_ref, TOL, "ln")
    assert_close(host(gpu, tx.grad), dx, TOL, "ln dx")
    assert_close(host(gpu, tw.grad), dw, TOL, "ln dw")
    assert_close(host(gpu, tb.grad), db, TOL, "ln db")


def test_layernorm_no_grad_matches_with_stats(gpu):
    x, w, b, _ = config3_inputs(1000, 384, seed=4)
    y0 = host(gpu, gpu.layernorm(dev(gpu, x), dev(gpu, w), dev(gpu, b)))
    y1 = host(gpu, gpu.layernorm(dev(gpu, x, True), dev(gpu, w), dev(gpu, b)))
    np.testing.assert_array_equal(y0, y1)
    assert_close(y0, O.layernorm(x, w, b), TOL, "ln no-grad")


@pytest.mark.parametrize("cols", [384, 768, 4096])
def test_layernorm_backward_is_reproducible(gpu, cols):
    """dgamma/dbeta use a fixed-order reduction: bit-identical reruns."""
    x, w, b, g = config3_inputs(8192, cols, seed=6)
    outs = []
    for _ in range(2):
        tx, tw, tb = dev(gpu, x, True), dev(gpu, w, True), dev(gpu, b, True)
        y = gpu.layernorm(tx, tw, tb, 1e-5)
        y.backward(dev(gpu, g))
        outs.append([host(gpu, t.grad) for t in (tx, tw, tb)])
    for a, c in zip(*outs):
        np.testing.assert_array_equal(a, c)


def test_abi_misaligned_rows(gpu):
    rows, cols = 40, 384
    x, w, b, g = config3_inputs(rows, cols, seed=12)
    abi = Abi()
    try:
        px, py = abi.put(x, 1), abi.empty(rows * cols, 1)
        abi.check(abi.L.aar_softmax_fwd_f32(px, py, rows, cols, None))
        assert_close(abi.get(py, (rows, cols)), O.softmax(x), TOL, "misaligned softmax")
        pw, pb = abi.put(w, 1), abi.put(b, 1)
        pm, pr = abi.empty(rows), abi.empty(rows)
        abi.check(abi.L.aar_layernorm_fwd_f32(px, pw, pb, py, pm, pr, rows, cols, 1e-5, None))
        y_ref, mu, rs = O.layernorm(x, w, b, 1e-5, stats=True)
        assert_close(abi.get(py, (rows, cols)), y_ref, TOL, "misaligned layernorm")
        pg, pdx, pdw, pdb = abi.put(g, 1), abi.empty(rows * cols, 1), abi.empty(cols), abi.empty(cols)
        wsb = abi.L.aar_layernorm_bwd_workspace_bytes(rows, cols)
        assert abi.L.aar_layernorm_bwd_f32(pg, px, pw, pm, pr, pdx, pdw, pdb, rows, cols, None, 0, None) == -2
        abi.check(abi.L.aar_layernorm_bwd_f32(pg, px, pw, pm, pr, pdx, pdw, pdb, rows, cols,
                                              abi.alloc(wsb), wsb, None))
        dx, dw, db = O.layernorm_backward(g, x, w, mu, rs)
        assert_close(abi.get(pdx, (rows, cols)), dx, TOL, "misaligned ln dx")
        assert_close(abi.get(pdw, (cols,)), dw, TOL, "misaligned ln dw")
        assert_close(abi.get(pdb, (cols,)), db, TOL, "misaligned ln db")
    finally:
        abi.free()
