"""Autograd engine on the GPU: gradient fan-in through add_grads (device add),
leaf accumulation across backward calls, a 10 000-deep chain, device
round trips and the strided copy kernel.  Reference behaviour:
cppsrc/autograd/backward.cpp:17-113, tests/cpp/test_autograd.cpp:78-186,
tests/cpp/test_autograd_ops.cpp:64-85, :462-477."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from conftest import assert_close, gemm_tol
from devutil import Abi, dev, host

pytestmark = pytest.mark.gpu
f32 = np.float32


def test_device_round_trip_and_zeros(gpu):
    a = np.arange(12, dtype=f32).reshape(3, 4)
    np.testing.assert_array_equal(host(gpu, dev(gpu, a)), a)
    z = gpu.Tensor.zeros([3, 5], gpu.DType.Fp32, gpu.Device.CUDA)
    np.testing.assert_array_equal(host(gpu, z), np.zeros((3, 5), f32))
    o = gpu.Tensor.ones([7], gpu.DType.Fp32, gpu.Device.CUDA)
    np.testing.assert_array_equal(host(gpu, o), np.ones(7, f32))
    # fp32 ones on the device are a fill kernel (several workgroups here, none
    # for an empty shape); other dtypes are uploaded
    o = gpu.Tensor.ones([3, 1000, 7], gpu.DType.Fp32, gpu.Device.CUDA)
    np.testing.assert_array_equal(host(gpu, o), np.ones((3, 1000, 7), f32))
    o = gpu.Tensor.ones([0, 4], gpu.DType.Fp32, gpu.Device.CUDA)
    assert host(gpu, o).shape == (0, 4)
    o = gpu.Tensor.ones([5], gpu.DType.Int64, gpu.Device.CUDA)
    np.testing.assert_array_equal(gpu.to_numpy(o.to(gpu.Device.CPU)), np.ones(5, np.int64))
    gpu.cuda_synchronize()


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference tree)")
def test_fanin_order_bit_identical_to_reference_autograd(gpu):
    """h = x*w0 feeds three consumers (u = h*w1, v = 0.75*h, z = h*w2) and x
    also feeds t = x*w3; root = ((u + v) + z) + t.  Every product and sum is a
    single fp32 operation on both sides, so x.grad agrees bit for bit with the
    reference's own autograd (oracle/_ref) only if both sum the three
    gradients of h, and then the two of x, in the same order."""
    rng = np.random.default_rng(31)
    n = 4099
    x = rng.standard_normal(n).astype(f32)
    w = rng.standard_normal((4, n)).astype(f32)
    g = rng.standard_normal(n).astype(f32)
    tx = dev(gpu, x, True)
    w0, w1, w2, w3 = (dev(gpu, w[i]) for i in range(4))
    h = gpu.mul(tx, w0)
    u, v, z = gpu.mul(h, w1), gpu.scale(h, 0.75), gpu.mul(h, w2)
    t = gpu.mul(tx, w3)
    root = gpu.add(gpu.add(gpu.add(u, v), z), t)
    root.backward(dev(gpu, g))
    np.testing.assert_array_equal(host(gpu, tx.grad), O.ref_fanin_graph(x, w, g))


def test_add_and_fan_in(gpu):
    rng = np.random.default_rng(0)
    a, b = rng.standard_normal((64, 33)).astype(f32), rng.standard_normal((64, 33)).astype(f32)
    ta, tb = dev(gpu, a, True), dev(gpu, b, True)
    c = gpu.add(ta, tb)
    np.testing.assert_array_equal(host(gpu, c), O.add(a, b))
    # a used twice: add(add(a, b), a) -> da = 2g, db = g, via device add_grads
    d = gpu.add(c, ta)
    g = rng.standard_normal((64, 33)).astype(f32)
    d.backward(dev(gpu, g))
    np.testing.assert_array_equal(host(gpu, ta.grad), O.add(g, g))
    np.testing.assert_array_equal(host(gpu, tb.grad), g)


def test_deep_chain(gpu):
    # tests/cpp/test_autograd.cpp:169-186: y = x + x + ... (10000 adds) -> dy/dx = 10001
    x = dev(gpu, np.ones(1, f32), True)
    y = x
    for _ in range(10000):
        y = gpu.add(y, x)
    y.backward()
    assert host(gpu, x.grad)[0] == 10001.0


def test_accumulates_across_backward_calls(gpu):
    # tests/cpp/test_autograd_ops.cpp:462-477
    a = dev(gpu, np.array([1, 2, 3], f32), True)
    b = dev(gpu, np.array([0.1, 0.2, 0.3], f32))
    seed = dev(gpu, np.ones(3, f32))
    gpu.add(a, b).backward(seed)
    gpu.add(a, b).backward(seed)
    np.testing.assert_array_equal(host(gpu, a.grad), np.full(3, 2.0, f32))
    a.zero_grad()
    assert a.grad is None


def test_matmul_fan_in_gradient(gpu):
    """x feeds two GEMMs; dx = G W1 + G W2 is summed by add_grads on the device."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((128, 64)).astype(f32)
    w1 = rng.standard_normal((48, 64)).astype(f32)
    w2 = rng.standard_normal((48, 64)).astype(f32)
    tx = dev(gpu, x, True)
    j = gpu.add(gpu.matmul_a_bt(tx, dev(gpu, w1)), gpu.matmul_a_bt(tx, dev(gpu, w2)))
    g = rng.standard_normal((128, 48)).astype(f32)
    j.backward(dev(gpu, g))
    ref = O.add(O.matmul("nn", g, w1), O.matmul("nn", g, w2))
    assert_close(host(gpu, tx.grad), ref, gemm_tol(48), "fan-in dx")


def test_slice_backward_and_contiguous(gpu):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 6, 5)).astype(f32)
    tx = dev(gpu, x, True)
    s = gpu.slice(tx, 1, 2, 5)
    t = gpu.transpose(s, 0, 2)
    c = gpu.contiguous(t)
    assert c.is_contiguous()
    np.testing.assert_array_equal(host(gpu, c), np.ascontiguousarray(x[:, 2:5].transpose(2, 1, 0)))
    g = rng.standard_normal(c.shape).astype(f32)
    c.backward(dev(gpu, g))
    ref = np.zeros_like(x)
    ref[:, 2:5] = g.transpose(2, 1, 0)
    np.testing.assert_array_equal(host(gpu, tx.grad), ref)


def test_abi_strided_copy_and_memset(gpu):
    import ctypes

    abi = Abi()
    try:
        a = np.arange(2 * 3 * 4, dtype=f32).reshape(2, 3, 4)
        pa = abi.put(a)
        pd = abi.empty(24)
        shape = (ctypes.c_int64 * 3)(4, 3, 2)
        src = (ctypes.c_int64 * 3)(1, 4, 12)
        dst = (ctypes.c_int64 * 3)(6, 2, 1)
        abi.check(abi.L.aar_strided_copy_f32(pa, pd, 3, shape, src, dst, None))
        np.testing.assert_array_equal(abi.get(pd, (4, 3, 2)), np.ascontiguousarray(a.transpose(2, 1, 0)))
        abi.check(abi.L.aar_memset_zero(pd + 4, 13, None))  # unaligned start, odd byte count
        got = abi.get(pd, (24,)).view(np.uint32)
        ref = np.ascontiguousarray(a.transpose(2, 1, 0)).reshape(-1).view(np.uint32).copy()
        raw = ref.view(np.uint8)
        raw[4:17] = 0
        np.testing.assert_array_equal(got, ref)
    finally:
        abi.free()


def test_large_add(gpu):
    rng = np.random.default_rng(6)
    n = (1 << 22) + 3
    a, b = rng.standard_normal(n).astype(f32), rng.standard_normal(n).astype(f32)
    np.testing.assert_array_equal(host(gpu, gpu.add(dev(gpu, a), dev(gpu, b))), a + b)
