"""The fused linear layer (x W^T + b, bias added in the GEMM epilogue or after
the split-K reduction) against the reference's two-op composition
add_bias(matmul_a_bt(x, W), b) (aargrad/nn.py:101-105): values and all three
gradients must be bit-identical, since the epilogue performs the same single
fp32 addition per element.  Cases cover the unsplit DMA path, the
register (unaligned) path, split-K with the vector and the scalar reduce, and
the C ABI directly, including a misaligned bias.  The composition itself is
pinned to the oracle by the GEMM and bias tests; one case rechecks the fused
result against the oracle at the GEMM tolerance 1e-4*sqrt(K)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle as O
from conftest import assert_close, gemm_tol
from devutil import Abi, dev, host

pytestmark = pytest.mark.gpu
f32 = np.float32

# (leading dims of x, K, N); the comment says which GEMM path the forward takes
CASES = [
    ((5, 7), 16, 3),           # tiny, N % 4 != 0
    ((64, 256), 384, 1536),    # GPT MLP up-projection, unsplit DMA path
    ((64, 256), 1536, 384),    # GPT MLP down-projection
    ((64,), 8192, 96),         # split-K (32 splits), vector reduce adds the bias
    ((64,), 8192, 100),        # split-K, N % 4 == 0 with 100 columns
    ((33,), 4999, 30),         # split-K, register path, scalar reduce
    ((3, 50), 17, 65),         # unaligned K and N, register path
    ((372,), 384, 16384),      # configuration 15 (64 x 128, deep ring), ragged last row tile
    ((480,), 384, 20000),      # configuration 15, ragged last column tile
]


def _split_count(op, M, N, K):
    L = ctypes.CDLL(str(__import__("devutil").LIB))
    i64, sz = ctypes.c_int64, ctypes.c_size_t
    L.aar_gemm_f32_workspace_bytes.restype = sz
    L.aar_gemm_f32_workspace_bytes.argtypes = [ctypes.c_int, i64, i64, i64]
    ip = ctypes.POINTER(ctypes.c_int)
    L.aar_gemm_f32_plan.argtypes = [ctypes.c_int, i64, i64, i64, sz, ip, ip]
    cfg, splits = ctypes.c_int(), ctypes.c_int()
    L.aar_gemm_f32_plan(op, M, N, K, L.aar_gemm_f32_workspace_bytes(op, M, N, K), ctypes.byref(cfg),
                        ctypes.byref(splits))
    return splits.value


def test_split_cases_really_split():
    assert _split_count(1, 64, 96, 8192) > 1
    assert _split_count(1, 64, 100, 8192) > 1
    assert _split_count(1, 33, 30, 4999) > 1
    assert _split_count(1, 64 * 256, 1536, 384) == 1


@pytest.mark.parametrize("lead,K,N", CASES)
def test_linear_bit_identical_to_composition(gpu, lead, K, N):
    rng = np.random.default_rng(K * 131 + N)
    x = rng.standard_normal(lead + (K,)).astype(f32)
    w = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(f32)
    b = rng.standard_normal(N).astype(f32)
    g = rng.standard_normal(lead + (N,)).astype(f32)

    tx, tw, tb = dev(gpu, x, True), dev(gpu, w, True), dev(gpu, b, True)
    y = gpu._core._linear(tx, tw, tb)
    assert list(y.shape) == list(lead) + [N]
    y.backward(dev(gpu, g))

    rx, rw, rb = dev(gpu, x, True), dev(gpu, w, True), dev(gpu, b, True)
    ry = gpu.add_bias(gpu.matmul_a_bt(rx, rw), rb)
    ry.backward(dev(gpu, g))

    np.testing.assert_array_equal(host(gpu, y), host(gpu, ry))
    np.testing.assert_array_equal(host(gpu, tx.grad), host(gpu, rx.grad))
    np.testing.assert_array_equal(host(gpu, tw.grad), host(gpu, rw.grad))
    np.testing.assert_array_equal(host(gpu, tb.grad), host(gpu, rb.grad))
    if N == 96:
        x2 = x.reshape(-1, K)
        assert_close(host(gpu, y).reshape(-1, N), O.add_bias(O.matmul("nt", x2, w), b), gemm_tol(K), "linear")


def test_linear_without_grad_and_through_nn(gpu, ag):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((4, 9, 40)).astype(f32)
    lin = ag.nn.Linear(40, 24, bias=True, rng=rng).to(ag.Device.CUDA)
    lin.bias.tensor = dev(gpu, rng.standard_normal(24).astype(f32), True)
    y = lin(dev(gpu, x))
    ref = gpu.add_bias(gpu.matmul_a_bt(dev(gpu, x), lin.weight.tensor), lin.bias.tensor)
    np.testing.assert_array_equal(host(gpu, y), host(gpu, ref))
    # no input needs a gradient: no graph node
    y0 = gpu._core._linear(dev(gpu, x), dev(gpu, host(gpu, lin.weight.tensor)), dev(gpu, host(gpu, lin.bias.tensor)))
    assert not y0.requires_grad
    np.testing.assert_array_equal(host(gpu, y0), host(gpu, ref))


def test_linear_empty_contraction_is_bias_broadcast(gpu):
    b = np.arange(5, dtype=f32)
    tx, tw, tb = dev(gpu, np.zeros((3, 0), f32), True), dev(gpu, np.zeros((5, 0), f32), True), dev(gpu, b, True)
    y = gpu._core._linear(tx, tw, tb)
    np.testing.assert_array_equal(host(gpu, y), np.broadcast_to(b, (3, 5)))
    y.backward(dev(gpu, np.ones((3, 5), f32)))
    np.testing.assert_array_equal(host(gpu, tb.grad), np.full(5, 3, f32))


def test_linear_zero_width_layer(gpu):
    # A layer with no outputs (W [0, K], bias [0]): empty output, and the
    # backward returns an empty dW/db and a zero dX (no division by zero, no
    # zero-column reduction).
    rng = np.random.default_rng(8)
    x = rng.standard_normal((2, 3, 7)).astype(f32)
    tx, tw, tb = dev(gpu, x, True), dev(gpu, np.zeros((0, 7), f32), True), dev(gpu, np.zeros(0, f32), True)
    y = gpu._core._linear(tx, tw, tb)
    assert y.shape == [2, 3, 0]
    gpu.sum_all(y).backward()
    np.testing.assert_array_equal(host(gpu, tx.grad), np.zeros_like(x))
    assert tw.grad.shape == [0, 7] and tb.grad.shape == [0]
    # the MLP op with a zero-width second layer, and with a zero-width hidden layer
    w1, b1 = rng.standard_normal((5, 7)).astype(f32), np.zeros(5, f32)
    for w2, b2 in ((np.zeros((0, 5), f32), np.zeros(0, f32)),):
        ts = [dev(gpu, a, True) for a in (x, w1, b1, w2, b2)]
        out = gpu._core._mlp_relu(*ts)
        assert out.shape == [2, 3, 0]
        gpu.sum_all(out).backward()
        np.testing.assert_array_equal(host(gpu, ts[0].grad), np.zeros_like(x))
    ts = [dev(gpu, a, True) for a in (x, np.zeros((0, 7), f32), np.zeros(0, f32), np.zeros((4, 0), f32),
                                      np.arange(4, dtype=f32))]
    out = gpu._core._mlp_relu(*ts)
    np.testing.assert_array_equal(host(gpu, out), np.broadcast_to(np.arange(4, dtype=f32), (2, 3, 4)))
    gpu.sum_all(out).backward()
    np.testing.assert_array_equal(host(gpu, ts[4].grad), np.full(4, 6, f32))


@pytest.mark.parametrize("M,N,K", [(64, 96, 8192), (33, 30, 4999), (150, 65, 17), (512, 256, 256)])
@pytest.mark.parametrize("use_ws,bias_off", [(True, 0), (True, 1), (False, 0)])
def test_abi_gemm_bias_matches_gemm_then_add_bias(M, N, K, use_ws, bias_off):
    abi = Abi()
    L = abi.L
    vp, i64, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t
    L.aar_gemm_f32_bias.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, vp, sz, vp]
    L.aar_add_bias_f32.argtypes = [vp, vp, vp, i64, i64, vp]
    try:
        rng = np.random.default_rng(M + N + K)
        a = rng.standard_normal((M, K)).astype(f32)
        bm = rng.standard_normal((N, K)).astype(f32)
        b = rng.standard_normal(N).astype(f32)
        pa, pb, pbias = abi.put(a), abi.put(bm), abi.put(b, bias_off)
        wsb = L.aar_gemm_f32_workspace_bytes(1, M, N, K) if use_ws else 0
        ws = abi.alloc(wsb) if wsb else None
        c_fused, c_prod, c_ref = abi.empty(M * N), abi.empty(M * N), abi.empty(M * N)
        abi.check(L.aar_gemm_f32_bias(1, M, N, K, pa, pb, pbias, c_fused, ws, wsb, None))
        abi.check(L.aar_gemm_f32(1, M, N, K, pa, pb, c_prod, ws, wsb, None))
        abi.check(L.aar_add_bias_f32(c_prod, pbias, c_ref, M, N, None))
        np.testing.assert_array_equal(abi.get(c_fused, (M, N)), abi.get(c_ref, (M, N)))
    finally:
        abi.free()
