"""The fused feed-forward block _mlp_relu(x, W1, b1, W2, b2): bias + relu in
the first GEMM's epilogue; the backward takes the relu mask from the saved
output h, or, where the GEMM plans allow (the 16384-row GPT case), from bits
the first GEMM's epilogue wrote, applying it and db1's column-sum partials in
the dh GEMM's epilogue.  Against the composition
linear(relu(linear(x, W1, b1)), W2, b2) of the same backend (aargrad/nn.py:101-122,
the GPT block's MLP) the values and all five gradients must be bit-identical:
each epilogue performs the same fp32 operation as the separate op.  Cases
cover the unsplit DMA path, the register (unaligned) path and split-K with the
vector and the scalar reduce; one case rechecks the result against the oracle
at the GEMM tolerance.  The C-ABI relu-mask GEMM (aar_gemm_f32_relu_mask, which
the op does not use) is checked against the GEMM followed by relu backward,
including a shape the plain GEMM plans on the thin-output kernel."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from conftest import assert_close, gemm_tol
import ctypes

from devutil import Abi, dev, host
from test_linear_gpu import _split_count

pytestmark = pytest.mark.gpu
f32 = np.float32

# (leading dims of x, d, hidden, out)
CASES = [
    ((4, 64), 384, 1536, 384),   # GPT block shape (256 rows), unsplit
    ((64, 256), 384, 1536, 384),  # GPT block at config 5 (16384 rows): the mask-bits epilogues
    ((3, 50), 17, 33, 65),       # unaligned everywhere: register path, scalar epilogue
    ((64,), 4096, 96, 64),       # forward bias+relu under split-K, vector reduce
    ((33,), 4999, 30, 7),        # forward split-K, scalar reduce
    ((64,), 64, 96, 8192),       # backward dh GEMM under split-K (K = 8192 outputs), vector reduce
    ((33,), 16, 30, 4999),       # backward dh GEMM under split-K, scalar reduce
]


def test_split_cases_really_split():
    assert _split_count(1, 64, 96, 4096) > 1     # NT forward, first layer
    assert _split_count(1, 33, 30, 4999) > 1
    assert _split_count(0, 64, 96, 8192) > 1     # NN dh = g W2
    assert _split_count(0, 33, 30, 4999) > 1


def _run(gpu, fused, x, w1, b1, w2, b2, g):
    ts = [dev(gpu, a, True) for a in (x, w1, b1, w2, b2)]
    if fused:
        out = gpu._core._mlp_relu(*ts)
    else:
        out = gpu._core._linear(gpu.relu(gpu._core._linear(ts[0], ts[1], ts[2])), ts[3], ts[4])
    out.backward(dev(gpu, g))
    return [host(gpu, out)] + [host(gpu, t.grad) for t in ts]


@pytest.mark.parametrize("lead,d,H,N2", CASES)
def test_mlp_bit_identical_to_composition(gpu, lead, d, H, N2):
    rng = np.random.default_rng(d * 7 + H * 131 + N2)
    x = rng.standard_normal(lead + (d,)).astype(f32)
    w1 = (rng.standard_normal((H, d)) / np.sqrt(d)).astype(f32)
    b1 = (0.1 * rng.standard_normal(H)).astype(f32)
    w2 = (rng.standard_normal((N2, H)) / np.sqrt(H)).astype(f32)
    b2 = (0.1 * rng.standard_normal(N2)).astype(f32)
    g = rng.standard_normal(lead + (N2,)).astype(f32)
    got = _run(gpu, True, x, w1, b1, w2, b2, g)
    ref = _run(gpu, False, x, w1, b1, w2, b2, g)
    for a, b, n in zip(got, ref, ("out", "dx", "dW1", "db1", "dW2", "db2")):
        assert a.shape == b.shape, n
        np.testing.assert_array_equal(a, b, err_msg=n)
    h_pre = x.reshape(-1, d) @ w1.T + b1
    assert 0.2 < np.mean(h_pre > 0) < 0.8  # the mask has both signs


def test_mlp_against_oracle(gpu):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((96, 64)).astype(f32)
    w1 = (rng.standard_normal((256, 64)) / 8).astype(f32)
    b1 = (0.1 * rng.standard_normal(256)).astype(f32)
    w2 = (rng.standard_normal((48, 256)) / 16).astype(f32)
    b2 = (0.1 * rng.standard_normal(48)).astype(f32)
    out = host(gpu, gpu._core._mlp_relu(*(dev(gpu, a) for a in (x, w1, b1, w2, b2))))
    h = O.relu(O.matmul("nt", x, w1) + b1)
    assert_close(out, O.matmul("nt", h, w2) + b2, gemm_tol(256), "out")


def test_mlp_no_grad_and_errors(gpu):
    rng = np.random.default_rng(6)
    x, w1, b1 = rng.standard_normal((8, 16)).astype(f32), rng.standard_normal((32, 16)).astype(f32), np.zeros(32, f32)
    w2, b2 = rng.standard_normal((4, 32)).astype(f32), np.zeros(4, f32)
    out = gpu._core._mlp_relu(*(dev(gpu, a) for a in (x, w1, b1, w2, b2)))
    assert not out.requires_grad and out.shape == [8, 4]
    with pytest.raises(ValueError):  # W2's in-features must match W1's out-features
        gpu._core._mlp_relu(*(dev(gpu, a) for a in (x, w1, b1, w2[:, :31], b2)))


@pytest.mark.parametrize("M,N,K", [(64, 96, 8192), (33, 30, 4999), (150, 65, 17), (512, 256, 256),
                                   (16384, 96, 384)])
def test_abi_relu_mask_gemm_matches_gemm_then_relu_backward(gpu, M, N, K):
    rng = np.random.default_rng(M + N + K)
    a = rng.standard_normal((M, K)).astype(f32)
    b = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(f32)
    h = np.maximum(0, rng.standard_normal((M, N))).astype(f32)
    abi = Abi()
    L = abi.L
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    L.aar_gemm_f32_relu_mask.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, vp, ctypes.c_size_t, vp]
    L.aar_gemm_f32.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, ctypes.c_size_t, vp]
    L.aar_gemm_f32_workspace_bytes.restype = ctypes.c_size_t
    L.aar_gemm_f32_workspace_bytes.argtypes = [ctypes.c_int, i64, i64, i64]
    L.aar_relu_bwd_f32.argtypes = [vp, vp, vp, i64, vp]
    try:
        pa, pb, ph = abi.put(a), abi.put(b), abi.put(h)
        wsb = L.aar_gemm_f32_workspace_bytes(0, M, N, K)
        ws = abi.alloc(wsb) if wsb else None
        pc, pp, pr = abi.empty(M * N), abi.empty(M * N), abi.empty(M * N)
        abi.check(L.aar_gemm_f32_relu_mask(0, M, N, K, pa, pb, ph, pc, ws, wsb, None))
        abi.check(L.aar_gemm_f32(0, M, N, K, pa, pb, pp, ws, wsb, None))
        abi.check(L.aar_relu_bwd_f32(pp, ph, pr, M * N, None))
        np.testing.assert_array_equal(abi.get(pc, (M, N)), abi.get(pr, (M, N)))
    finally:
        abi.free()
