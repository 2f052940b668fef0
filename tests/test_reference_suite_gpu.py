"""The reference's Python test files for shape ops, nn modules, the FFN ops,
AdamW and the MLP training loop (tests/python/test_shape.py, test_nn.py,
test_ffn.py, test_adamw.py, test_train_mlp.py), restated on the device.

Each test names the reference test it follows.  The reference runs many of
them on its CPU device too; this backend computes only on the GPU (CPU
tensors are storage and views), so those cases check the device against the
closed forms the reference tests use (numpy expressions, finite differences,
erf-GELU, the numpy AdamW step) with the reference's own tolerances."""
from __future__ import annotations

import math

import numpy as np
import pytest

from devutil import dev, host

pytestmark = pytest.mark.gpu
f32 = np.float32


def _scalar(gpu, t):
    return float(host(gpu, t))


def hv(gpu, t):
    # Tensor.to needs a contiguous source, as in the reference (tensor.cpp:89-94)
    return host(gpu, gpu.contiguous(t))


# ------------------------------------------------------------ test_shape.py

def test_reshape_round_trip_and_inferred_dim(gpu):
    # test_shape.py:15-26
    x_np = np.arange(24, dtype=f32)
    r = gpu.reshape(dev(gpu, x_np), [2, 3, 4])
    assert r.shape == [2, 3, 4]
    np.testing.assert_array_equal(hv(gpu, r), x_np.reshape(2, 3, 4))
    assert gpu.reshape(dev(gpu, np.arange(12, dtype=f32)), [3, -1]).shape == [3, 4]


def test_reshape_backward(gpu):
    # test_shape.py:29-34
    x_np = np.arange(12, dtype=f32).reshape(3, 4)
    x = dev(gpu, x_np, True)
    r = gpu.reshape(x, [4, 3])
    gpu.sum_all(gpu.mul(r, r)).backward()
    np.testing.assert_allclose(host(gpu, x.grad), 2 * x_np)


def test_transpose_matches_numpy_and_is_involutive(gpu):
    # test_shape.py:37-50, :62-72 (device result against the host view)
    rng = np.random.default_rng(0)
    x_np = rng.standard_normal((2, 3, 4, 5)).astype(f32)
    x = dev(gpu, x_np)
    np.testing.assert_array_equal(host(gpu, gpu.contiguous(gpu.transpose(x, 1, 2))), np.swapaxes(x_np, 1, 2))
    np.testing.assert_array_equal(host(gpu, gpu.contiguous(gpu.transpose(x, 1, 3))),
                                  gpu.to_numpy(gpu.transpose(gpu.from_numpy(x_np), 1, 3)))
    y_np = np.random.default_rng(1).standard_normal((2, 3, 4)).astype(f32)
    y = gpu.transpose(gpu.transpose(dev(gpu, y_np), 0, 2), 0, 2)
    np.testing.assert_array_equal(hv(gpu, y), y_np)


def test_transpose_backward(gpu):
    # test_shape.py:53-59
    x_np = np.random.default_rng(2).standard_normal((2, 3, 4)).astype(f32)
    x = dev(gpu, x_np, True)
    y = gpu.transpose(x, 0, 2)
    gpu.sum_all(gpu.mul(y, y)).backward()
    np.testing.assert_allclose(host(gpu, x.grad), 2 * x_np, atol=1e-5)


def test_slice_squeeze_unsqueeze(gpu):
    # test_shape.py:86-127
    rng = np.random.default_rng(11)
    x_np = rng.standard_normal((4, 6, 8)).astype(f32)
    x = dev(gpu, x_np)
    s = gpu.slice(x, 1, 2, 5)
    assert s.shape == [4, 3, 8]
    np.testing.assert_array_equal(hv(gpu, s), x_np[:, 2:5, :])
    np.testing.assert_array_equal(hv(gpu, gpu.slice(x, 2, 1, 7)), x_np[:, :, 1:7])
    z_np = np.random.default_rng(12).standard_normal((2, 3, 4, 5)).astype(f32)
    sq = gpu.squeeze(gpu.slice(dev(gpu, z_np), 1, 1, 2), 1)
    assert sq.shape == [2, 4, 5]
    np.testing.assert_array_equal(hv(gpu, sq), z_np[:, 1, :, :])
    u_np = np.random.default_rng(14).standard_normal((2, 3, 4)).astype(f32)
    u = gpu.unsqueeze(dev(gpu, u_np), 1)
    assert u.shape == [2, 1, 3, 4]
    np.testing.assert_array_equal(hv(gpu, u), u_np[:, None, :, :])
    back = gpu.squeeze(u, 1)
    assert back.shape == [2, 3, 4]
    np.testing.assert_array_equal(hv(gpu, back), u_np)


def test_to_host_of_offset_view(gpu):
    # A view with a storage offset is not contiguous (tensor.cpp:52-53), so to() refuses it as the
    # reference does (tensor.cpp:89-94); contiguous() first moves the view's own elements.
    x_np = np.arange(24, dtype=f32).reshape(4, 6)
    s = gpu.slice(dev(gpu, x_np), 0, 1, 3)
    assert s.storage_offset == 6 and not s.is_contiguous()
    with pytest.raises(RuntimeError, match="contiguous"):
        s.to(gpu.Device.CPU)
    np.testing.assert_array_equal(hv(gpu, s), x_np[1:3])


def test_slice_backward_accumulates(gpu):
    # test_shape.py:107-115: two slice grads fan into one leaf
    x_np = np.random.default_rng(13).standard_normal((3, 4, 5)).astype(f32)
    x = dev(gpu, x_np, True)
    a = gpu.slice(x, 1, 0, 2)
    b = gpu.slice(x, 1, 2, 4)
    gpu.add(gpu.sum_all(gpu.mul(a, a)), gpu.sum_all(gpu.mul(b, b))).backward()
    np.testing.assert_allclose(host(gpu, x.grad), 2 * x_np, atol=1e-5)


def test_contiguous_on_device(gpu):
    # test_shape.py:130-147
    x_np = np.random.default_rng(15).standard_normal((3, 4)).astype(f32)
    c = gpu.contiguous(dev(gpu, x_np))
    assert c.is_contiguous()
    np.testing.assert_array_equal(host(gpu, c), x_np)
    y_np = np.random.default_rng(16).standard_normal((2, 3, 4)).astype(f32)
    t = gpu.transpose(dev(gpu, y_np), 0, 2)
    assert not t.is_contiguous()
    m = gpu.contiguous(t)
    assert m.is_contiguous()
    np.testing.assert_array_equal(host(gpu, m), np.swapaxes(y_np, 0, 2))


def test_bmm_a_bt_with_strided_inputs(gpu):
    # test_shape.py:150-163: q, k as strided views of a packed qkv
    rng = np.random.default_rng(17)
    B, H, T, dh = 2, 3, 5, 4
    qkv_np = rng.standard_normal((B, T, 3, H, dh)).astype(f32)
    qkv = dev(gpu, qkv_np)
    q = gpu.transpose(gpu.squeeze(gpu.slice(qkv, 2, 0, 1), 2), 1, 2)
    k = gpu.transpose(gpu.squeeze(gpu.slice(qkv, 2, 1, 2), 2), 1, 2)
    assert not q.is_contiguous() and not k.is_contiguous()
    q_np = qkv_np[:, :, 0].transpose(0, 2, 1, 3)
    k_np = qkv_np[:, :, 1].transpose(0, 2, 1, 3)
    ref = np.matmul(q_np, np.ascontiguousarray(np.swapaxes(k_np, -1, -2)))
    np.testing.assert_allclose(host(gpu, gpu.bmm_a_bt(q, k)), ref, atol=1e-5)


# --------------------------------------------------------------- test_nn.py

def test_linear_forward_shape_and_finite_diff(gpu, ag):
    # test_nn.py:45-79 (forward shape; dW against central differences, eps 1e-3, atol 1e-2)
    rng = np.random.default_rng(0)
    layer = ag.nn.Linear(8, 4, rng=rng).to(ag.Device.CUDA)
    assert layer(dev(gpu, rng.standard_normal((2, 8)).astype(f32))).shape == [2, 4]

    rng = np.random.default_rng(1)
    layer = ag.nn.Linear(3, 2, rng=rng).to(ag.Device.CUDA)
    x_np = rng.standard_normal((4, 3)).astype(f32)
    y = layer(dev(gpu, x_np, True))
    gpu.sum_all(gpu.mul(y, y)).backward()
    w_grad = host(gpu, layer.weight.tensor.grad)
    w_val = host(gpu, layer.weight.tensor)

    def loss_at(w):
        yp = gpu.matmul_a_bt(dev(gpu, x_np), dev(gpu, w))
        return _scalar(gpu, gpu.sum_all(gpu.mul(yp, yp)))

    eps = 1e-3
    num = np.zeros_like(w_grad)
    for i, j in np.ndindex(*w_val.shape):
        wp, wm = w_val.copy(), w_val.copy()
        wp[i, j] += eps
        wm[i, j] -= eps
        num[i, j] = (loss_at(wp) - loss_at(wm)) / (2 * eps)
    np.testing.assert_allclose(w_grad, num, atol=1e-2)


def test_module_to_cuda_preserves_requires_grad(gpu, ag):
    # test_nn.py:82-90
    rng = np.random.default_rng(0)
    nn = ag.nn
    model = nn.Sequential(nn.Linear(4, 8, rng=rng), nn.ReLU(), nn.Linear(8, 1, rng=rng))
    model.to(ag.Device.CUDA)
    for p in model.parameters():
        assert p.tensor.device == ag.Device.CUDA
        assert p.tensor.requires_grad is True


def test_sgd_step_updates_in_place(gpu, ag):
    # test_nn.py:93-103
    p = ag.nn.Parameter(dev(gpu, np.array([1.0, 2.0, 3.0], f32)))
    gpu.sum_all(p.tensor).backward()
    ag.optim.SGD([p], lr=0.1).step()
    np.testing.assert_allclose(host(gpu, p.tensor), np.array([0.9, 1.9, 2.9], f32))


# -------------------------------------------------------------- test_ffn.py

def _gelu_ref(x):
    erf = np.vectorize(math.erf)
    return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))


def test_sub_forward_and_backward(gpu):
    # test_ffn.py:24-33
    a_np, b_np = np.array([3.0, 5.0, 7.0], f32), np.array([1.0, 2.0, 4.0], f32)
    a, b = dev(gpu, a_np, True), dev(gpu, b_np, True)
    c = gpu.sub(a, b)
    np.testing.assert_array_equal(host(gpu, c), a_np - b_np)
    gpu.sum_all(c).backward()
    np.testing.assert_array_equal(host(gpu, a.grad), np.ones_like(a_np))
    np.testing.assert_array_equal(host(gpu, b.grad), -np.ones_like(b_np))


def test_gelu_forward_erf_and_backward_finite_diff(gpu, ag):
    # test_ffn.py:36-62, :129-131
    x_np = np.random.default_rng(0).standard_normal((4, 5)).astype(f32)
    np.testing.assert_allclose(host(gpu, gpu.gelu(dev(gpu, x_np))), _gelu_ref(x_np), atol=1e-6)
    xm_np = np.array([-1.0, 0.0, 1.0, 2.0], f32)
    np.testing.assert_array_equal(host(gpu, ag.nn.GELU()(dev(gpu, xm_np))), host(gpu, gpu.gelu(dev(gpu, xm_np))))

    x_np = (np.random.default_rng(1).standard_normal((3, 4)) * 1.5).astype(f32)
    x = dev(gpu, x_np, True)
    gpu.sum_all(gpu.gelu(x)).backward()
    g = host(gpu, x.grad)
    eps = 1e-3
    num = np.zeros_like(g)
    for i, j in np.ndindex(*x_np.shape):
        xp, xm = x_np.copy(), x_np.copy()
        xp[i, j] += eps
        xm[i, j] -= eps
        num[i, j] = (_scalar(gpu, gpu.sum_all(gpu.gelu(dev(gpu, xp))))
                     - _scalar(gpu, gpu.sum_all(gpu.gelu(dev(gpu, xm))))) / (2 * eps)
    np.testing.assert_allclose(g, num, atol=1e-3)


def test_add_bias_forward_and_backward_finite_diff(gpu):
    # test_ffn.py:65-101
    x_np = np.arange(12, dtype=f32).reshape(4, 3)
    b_np = np.array([10.0, 20.0, 30.0], f32)
    np.testing.assert_array_equal(host(gpu, gpu.add_bias(dev(gpu, x_np), dev(gpu, b_np))), x_np + b_np)

    rng = np.random.default_rng(2)
    x_np = rng.standard_normal((5, 3)).astype(f32)
    b_np = rng.standard_normal(3).astype(f32)
    x, b = dev(gpu, x_np, True), dev(gpu, b_np, True)
    gpu.sum_all(gpu.mul(gpu.add_bias(x, b), gpu.add_bias(x, b))).backward()

    def fwd(xa, ba):
        y = xa.astype(np.float64) + ba
        return float(np.sum(y * y))

    eps = 1e-3
    dx_num = np.zeros_like(x_np)
    for i, j in np.ndindex(*x_np.shape):
        xp, xm = x_np.copy(), x_np.copy()
        xp[i, j] += eps
        xm[i, j] -= eps
        dx_num[i, j] = (fwd(xp, b_np) - fwd(xm, b_np)) / (2 * eps)
    db_num = np.zeros_like(b_np)
    for j in range(3):
        bp, bm = b_np.copy(), b_np.copy()
        bp[j] += eps
        bm[j] -= eps
        db_num[j] = (fwd(x_np, bp) - fwd(x_np, bm)) / (2 * eps)
    np.testing.assert_allclose(host(gpu, x.grad), dx_num, atol=1e-2)
    np.testing.assert_allclose(host(gpu, b.grad), db_num, atol=1e-2)


def test_linear_with_bias_and_layernorm_module(gpu, ag):
    # test_ffn.py:104-126
    layer = ag.nn.Linear(4, 6, bias=True, rng=np.random.default_rng(0)).to(ag.Device.CUDA)
    assert layer(dev(gpu, np.zeros((2, 4), f32))).shape == [2, 6]
    assert len(list(layer.parameters())) == 2
    x_np = np.random.default_rng(3).standard_normal((4, 8)).astype(f32)
    ln = ag.nn.LayerNorm(8).to(ag.Device.CUDA)
    mu = x_np.mean(axis=-1, keepdims=True)
    var = x_np.var(axis=-1, keepdims=True)
    np.testing.assert_allclose(host(gpu, ln(dev(gpu, x_np))), (x_np - mu) / np.sqrt(var + 1e-5), atol=1e-5)


# ------------------------------------------------------------ test_adamw.py

def _adamw_numpy_step(param, grad, m, v, lr, b1, b2, eps, wd, t):
    # test_adamw.py:17-25
    bc1, bc2 = 1.0 - b1 ** t, 1.0 - b2 ** t
    m = b1 * m + (1 - b1) * grad
    v = b2 * v + (1 - b2) * grad * grad
    param = param * (1 - lr * wd) - lr * (m / bc1) / (np.sqrt(v / bc2) + eps)
    return param, m, v


@pytest.mark.parametrize("seed,shape,steps,lr,wd,atol", [(0, (4, 5), 5, 1e-2, 0.01, 1e-6),
                                                         (1, (6, 7), 10, 1e-3, 0.05, 1e-5)])
def test_adamw_matches_numpy(gpu, ag, seed, shape, steps, lr, wd, atol):
    # test_adamw.py:29-55 (5 steps, atol 1e-6) and :58-78 (10 steps; the reference compares its
    # CPU path, here the same numpy step)
    rng = np.random.default_rng(seed)
    p_np = rng.standard_normal(shape).astype(f32)
    g_np = rng.standard_normal(shape).astype(f32)
    m_np, v_np = np.zeros_like(p_np), np.zeros_like(p_np)
    b1, b2, eps = 0.9, 0.999, 1e-8
    p, g = dev(gpu, p_np), dev(gpu, g_np)
    m = ag.Tensor.zeros(list(shape), ag.DType.Fp32, ag.Device.CUDA)
    v = ag.Tensor.zeros(list(shape), ag.DType.Fp32, ag.Device.CUDA)
    for t in range(1, steps + 1):
        gpu.adamw_step(p, g, m, v, lr, b1, b2, eps, wd, 1.0 - b1 ** t, 1.0 - b2 ** t)
        p_np, m_np, v_np = _adamw_numpy_step(p_np, g_np, m_np, v_np, lr, b1, b2, eps, wd, t)
    np.testing.assert_allclose(host(gpu, p), p_np, atol=atol)
    np.testing.assert_allclose(host(gpu, m), m_np, atol=atol)
    np.testing.assert_allclose(host(gpu, v), v_np, atol=atol)


# ---------------------------------------- test_train_mlp.py, test_adamw.py

@pytest.mark.parametrize("opt", ["sgd", "adamw"])
def test_mlp_loss_decreases(gpu, ag, opt):
    # test_train_mlp.py:17-49 (SGD lr 0.01) and test_adamw.py:80-112 (AdamW lr 1e-2, wd 0.01):
    # 200 steps of a Linear-GELU-Linear regression, loss must halve
    rng = np.random.default_rng(0)
    A_true = rng.standard_normal((4, 8)).astype(f32)
    B_true = rng.standard_normal((8, 1)).astype(f32)
    X = rng.standard_normal((32, 4)).astype(f32)
    Y = np.maximum(X @ A_true, 0) @ B_true
    nn = ag.nn
    model = nn.Sequential(nn.Linear(4, 8, bias=True, rng=np.random.default_rng(1)), nn.GELU(),
                          nn.Linear(8, 1, bias=True, rng=np.random.default_rng(2)))
    model.to(ag.Device.CUDA)
    params = list(model.parameters())
    optim = ag.optim.SGD(params, lr=0.01) if opt == "sgd" else ag.optim.AdamW(params, lr=1e-2, weight_decay=0.01)
    losses = []
    for _ in range(200):
        diff = gpu.sub(model(dev(gpu, X)), dev(gpu, Y))
        loss = gpu.sum_all(gpu.mul(diff, diff))
        optim.zero_grad()
        loss.backward()
        optim.step()
        losses.append(_scalar(gpu, loss))
    assert np.all(np.isfinite(losses))
    assert losses[-1] < losses[0] * 0.5, f"{losses[0]:.4f} -> {losses[-1]:.4f}"


# ---------------------------------------------------------- test_tensor.cpp

def test_device_zeros_match_host(gpu, ag):
    # tests/cpp/test_tensor.cpp:38-46
    t = ag.Tensor.zeros([8], ag.DType.Fp32, ag.Device.CUDA)
    np.testing.assert_array_equal(host(gpu, t), np.zeros(8, f32))
