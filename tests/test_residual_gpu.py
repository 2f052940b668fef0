"""The pre-norm block's residual adds, fused on the device.

  * _linear_residual(r, a, W) = r + a W^T, the add in the GEMM epilogue
    (aar_gemm_f32_add), against add(r, matmul_a_bt(a, W));
  * _mlp_relu_residual(r, x, W1, b1, W2, b2) = r + mlp, the add in the second
    GEMM's epilogue (aar_gemm_f32_bias_add), against add(r, _mlp_relu(...));
  * the gradient fan-in of a layernorm input that also feeds the residual
    (x + f(LN(x))): the autograd engine hands the held gradient to the
    layernorm backward, which writes held + its own gradient
    (aar_layernorm_bwd_acc_f32), against the two gradients summed apart.

Each is the same fp32 operation as the composition (the same product plan, one
addition per element in the composition's order), so values and every
gradient must agree bit for bit.  The reference's composition is
cppsrc/ops/matmul.cpp:11 + elementwise.cpp:8 and backward.cpp:17-36 (add_grads)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle as O
from conftest import TOL, assert_close
from devutil import Abi, dev, host
from test_linear_gpu import _split_count

pytestmark = pytest.mark.gpu
f32 = np.float32


def _bits_equal(got, want, what):
    for i, (g, w) in enumerate(zip(got, want)):
        assert g.shape == w.shape, (what, i, g.shape, w.shape)
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), f"{what}: output {i} differs"


# (leading dims of a, K, N)
LIN_CASES = [
    ((4, 64), 384, 384),     # the GPT block's output projection (256 rows)
    ((3, 50), 17, 65),       # unaligned: register path, scalar epilogue
    ((64,), 4096, 96),       # split-K forward, vector reduce applies the add
    ((33,), 4999, 7),        # split-K forward, scalar reduce
    ((16384,), 384, 65),     # a thin-kernel plan: the product, then the add
]


def test_residual_cases_take_their_paths():
    assert _split_count(1, 64, 96, 4096) > 1
    assert _split_count(1, 33, 7, 4999) > 1
    abi = Abi()
    cfg, sp = ctypes.c_int(), ctypes.c_int()
    abi.check(abi.L.aar_gemm_f32_plan(1, 16384, 65, 384, 0, ctypes.byref(cfg), ctypes.byref(sp)))
    n_tiles = 0
    while abi.L.aar_gemm_f32_tile_config(n_tiles, None, None, None) == 0:
        n_tiles += 1
    assert cfg.value == n_tiles  # the thin-output kernel's id follows the tile configurations


@pytest.mark.parametrize("lead,K,N", LIN_CASES)
def test_linear_residual_bit_identical_to_composition(gpu, lead, K, N):
    rng = np.random.default_rng(K * 3 + N * 7 + len(lead))
    r = rng.standard_normal(lead + (N,)).astype(f32)
    a = rng.standard_normal(lead + (K,)).astype(f32)
    w = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(f32)
    g = rng.standard_normal(lead + (N,)).astype(f32)
    runs = []
    for fused in (True, False):
        tr, ta, tw = dev(gpu, r, True), dev(gpu, a, True), dev(gpu, w, True)
        out = gpu._core._linear_residual(tr, ta, tw) if fused else gpu.add(tr, gpu.matmul_a_bt(ta, tw))
        out.backward(dev(gpu, g))
        runs.append([host(gpu, out)] + [host(gpu, t.grad) for t in (tr, ta, tw)])
    _bits_equal(runs[0], runs[1], f"linear_residual {lead} K={K} N={N}")
    A = a.reshape(-1, K).astype(np.float64)
    ref = r.reshape(-1, N) + A @ w.T.astype(np.float64)
    rows = np.arange(0, A.shape[0], max(1, A.shape[0] // 64))
    assert_close(runs[0][0].reshape(-1, N)[rows], ref[rows], 1e-4 * np.sqrt(K), "r + a W^T")


MLP_CASES = [
    ((4, 64), 384, 1536, 384),   # the GPT block's MLP (256 rows)
    ((3, 50), 17, 33, 65),       # unaligned everywhere
    ((64,), 4096, 96, 64),       # forward split-K, vector reduce
    ((33,), 16, 30, 4999),       # backward split-K, scalar reduce
]


@pytest.mark.parametrize("lead,d,H,N2", MLP_CASES)
def test_mlp_relu_residual_bit_identical_to_composition(gpu, lead, d, H, N2):
    rng = np.random.default_rng(d * 11 + H * 5 + N2)
    r = rng.standard_normal(lead + (N2,)).astype(f32)
    x = rng.standard_normal(lead + (d,)).astype(f32)
    w1 = (rng.standard_normal((H, d)) / np.sqrt(d)).astype(f32)
    b1 = (0.1 * rng.standard_normal(H)).astype(f32)
    w2 = (rng.standard_normal((N2, H)) / np.sqrt(H)).astype(f32)
    b2 = (0.1 * rng.standard_normal(N2)).astype(f32)
    g = rng.standard_normal(lead + (N2,)).astype(f32)
    runs = []
    for fused in (True, False):
        ts = [dev(gpu, t, True) for t in (r, x, w1, b1, w2, b2)]
        if fused:
            out = gpu._core._mlp_relu_residual(*ts)
        else:
            out = gpu.add(ts[0], gpu._core._mlp_relu(*ts[1:]))
        out.backward(dev(gpu, g))
        runs.append([host(gpu, out)] + [host(gpu, t.grad) for t in ts])
    _bits_equal(runs[0], runs[1], f"mlp_relu_residual {lead} {d} {H} {N2}")


def test_residual_op_errors_match_composition(gpu):
    a = dev(gpu, np.ones((4, 8), f32))
    w = dev(gpu, np.ones((6, 8), f32))
    with pytest.raises(ValueError):   # r of the wrong shape: the add's check
        gpu._core._linear_residual(dev(gpu, np.ones((4, 5), f32)), a, w)
    with pytest.raises(ValueError):   # contraction mismatch: matmul_a_bt's check
        gpu._core._linear_residual(dev(gpu, np.ones((4, 6), f32)), a, dev(gpu, np.ones((6, 7), f32)))
    x = dev(gpu, np.ones((4, 8), f32))
    w1, b1 = dev(gpu, np.ones((16, 8), f32)), dev(gpu, np.ones(16, f32))
    w2, b2 = dev(gpu, np.ones((6, 16), f32)), dev(gpu, np.ones(6, f32))
    with pytest.raises(ValueError):
        gpu._core._mlp_relu_residual(dev(gpu, np.ones((4, 7), f32)), x, w1, b1, w2, b2)


@pytest.mark.parametrize("shape", [(4, 64, 384), (300, 768), (16, 4096), (5, 10000), (64, 383)])
@pytest.mark.parametrize("leaf", [True, False])
def test_layernorm_fan_in_is_fused_and_exact(gpu, shape, leaf):
    """x + matmul_a_bt(LN(x), W): the add hands x its gradient G first, the
    layernorm's arrives second and is summed by the layernorm backward.  The
    result must equal G + (the layernorm path's gradient alone) in fp32, bit
    for bit, for a leaf x and for an x computed by another op."""
    C = shape[-1]
    rng = np.random.default_rng(sum(shape) + leaf)
    x = (3 * rng.standard_normal(shape)).astype(f32)
    w = (1 + 0.1 * rng.standard_normal(C)).astype(f32)
    b = (0.1 * rng.standard_normal(C)).astype(f32)
    W = (rng.standard_normal((C, C)) / np.sqrt(C)).astype(f32) if C <= 4096 else None
    G = rng.standard_normal(shape).astype(f32)

    def branch(t, tw, tb):
        y = gpu.layernorm(t, tw, tb, 1e-5)
        return gpu.matmul_a_bt(y, dev(gpu, W)) if W is not None else gpu.mul(y, y)

    def grad_of(fan_in):
        src = dev(gpu, x, True)
        t = src if leaf else gpu.mul(src, dev(gpu, np.ones(shape, f32)))
        tw, tb = dev(gpu, w, True), dev(gpu, b, True)
        out = gpu.add(t, branch(t, tw, tb)) if fan_in else branch(t, tw, tb)
        out.backward(dev(gpu, G))
        return host(gpu, src.grad), host(gpu, tw.grad), host(gpu, tb.grad)

    fused = grad_of(True)
    alone = grad_of(False)
    want = (G + alone[0]).astype(f32)  # add_grads(held = G, new = the layernorm gradient)
    _bits_equal([fused[0]], [want], f"x.grad {shape}")
    _bits_equal(list(fused[1:]), list(alone[1:]), f"dw/db {shape}")


@pytest.mark.parametrize("rows,cols,offset", [(4096, 384, 0), (300, 768, 0), (77, 4096, 0), (5, 10000, 0),
                                              (64, 383, 0), (100, 384, 1)])
def test_abi_layernorm_bwd_acc(gpu, rows, cols, offset):
    """aar_layernorm_bwd_acc_f32 against aar_layernorm_bwd_f32 then aar_add_f32,
    bit for bit, out of place and in place (dx_addend == dx); offset 1 makes
    every operand unaligned (the element-wise plan)."""
    rng = np.random.default_rng(rows + cols)
    x = (3 * rng.standard_normal((rows, cols))).astype(f32)
    gy = rng.standard_normal((rows, cols)).astype(f32)
    w = (1 + 0.02 * rng.standard_normal(cols)).astype(f32)
    b = (0.02 * rng.standard_normal(cols)).astype(f32)
    add = rng.standard_normal((rows, cols)).astype(f32)
    abi = Abi()
    L = abi.L
    vp, i64, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t
    L.aar_layernorm_bwd_acc_f32.argtypes = [vp] * 9 + [i64, i64, vp, sz, vp]
    try:
        px, pg, pw, pb = (abi.put(t, offset) for t in (x, gy, w, b))
        py, pm, pr = abi.empty(rows * cols, offset), abi.empty(rows), abi.empty(rows)
        abi.check(L.aar_layernorm_fwd_f32(px, pw, pb, py, pm, pr, rows, cols, ctypes.c_float(1e-5), None))
        wsb = L.aar_layernorm_bwd_workspace_bytes(rows, cols)
        ws = abi.alloc(wsb)
        pdx, pdw, pdb = abi.empty(rows * cols, offset), abi.empty(cols), abi.empty(cols)
        abi.check(L.aar_layernorm_bwd_f32(pg, px, pw, pm, pr, pdx, pdw, pdb, rows, cols, ws, wsb, None))
        padd = abi.put(add, offset)
        psum = abi.empty(rows * cols, offset)
        abi.check(L.aar_add_f32(padd, pdx, psum, rows * cols, None))
        want = [abi.get(psum, (rows, cols)), abi.get(pdw, cols), abi.get(pdb, cols)]
        # out of place
        pdx2, pdw2, pdb2 = abi.empty(rows * cols, offset), abi.empty(cols), abi.empty(cols)
        abi.check(L.aar_layernorm_bwd_acc_f32(pg, px, pw, pm, pr, padd, pdx2, pdw2, pdb2, rows, cols, ws, wsb, None))
        _bits_equal([abi.get(pdx2, (rows, cols)), abi.get(pdw2, cols), abi.get(pdb2, cols)], want, "out of place")
        # in place: the addend buffer receives the sum
        pin = abi.put(add, offset)
        abi.check(L.aar_layernorm_bwd_acc_f32(pg, px, pw, pm, pr, pin, pin, pdw2, pdb2, rows, cols, ws, wsb, None))
        _bits_equal([abi.get(pin, (rows, cols))], want[:1], "in place")
        # and the values against the oracle's layernorm backward plus the addend
        _, mean, rstd = O.layernorm(x, w, b, 1e-5, stats=True)
        ref_dx, _, _ = O.layernorm_backward(gy, x, w, mean, rstd)
        assert_close(want[0], add + ref_dx, TOL, "dx + addend vs oracle")
        assert L.aar_layernorm_bwd_acc_f32(pg, px, pw, pm, pr, None, pdx2, pdw2, pdb2, rows, cols, ws, wsb,
                                           None) == -1
    finally:
        abi.free()


@pytest.mark.parametrize("M,N,K,offset", [(256, 384, 384, 0), (50, 65, 17, 1), (64, 96, 4096, 0), (33, 7, 4999, 0),
                                          (16100, 384, 384, 0), (16100, 384, 1536, 0)])
def test_abi_gemm_add_epilogues(gpu, M, N, K, offset):
    """aar_gemm_f32_add / aar_gemm_f32_bias_add against aar_gemm_f32 /
    aar_gemm_f32_bias followed by aar_add_f32, bit for bit; other layouts are
    unsupported and a missing R is invalid.  16100 rows: the 8-wave 128 x 192
    tile with a ragged last row tile and the residual loaded in one batch."""
    rng = np.random.default_rng(M + N + K)
    a = rng.standard_normal((M, K)).astype(f32)
    w = rng.standard_normal((N, K)).astype(f32)
    bias = rng.standard_normal(N).astype(f32)
    r = rng.standard_normal((M, N)).astype(f32)
    abi = Abi()
    L = abi.L
    vp, i64, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t
    L.aar_gemm_f32_bias.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, vp, sz, vp]
    L.aar_gemm_f32_add.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, vp, sz, vp]
    L.aar_gemm_f32_bias_add.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, vp, vp, sz, vp]
    try:
        pa, pw, pbias, pr = (abi.put(t, offset) for t in (a, w, bias, r))
        wsb = L.aar_gemm_f32_workspace_bytes(1, M, N, K)
        ws = abi.alloc(wsb) if wsb else None
        pc, pc2, pfused = (abi.empty(M * N, offset) for _ in range(3))
        abi.check(L.aar_gemm_f32(1, M, N, K, pa, pw, pc, ws, wsb, None))
        abi.check(L.aar_add_f32(pr, pc, pc2, M * N, None))
        abi.check(L.aar_gemm_f32_add(1, M, N, K, pa, pw, pr, pfused, ws, wsb, None))
        _bits_equal([abi.get(pfused, (M, N))], [abi.get(pc2, (M, N))], "gemm + add")
        abi.check(L.aar_gemm_f32_bias(1, M, N, K, pa, pw, pbias, pc, ws, wsb, None))
        abi.check(L.aar_add_f32(pr, pc, pc2, M * N, None))
        abi.check(L.aar_gemm_f32_bias_add(1, M, N, K, pa, pw, pbias, pr, pfused, ws, wsb, None))
        _bits_equal([abi.get(pfused, (M, N))], [abi.get(pc2, (M, N))], "gemm + bias + add")
        assert L.aar_gemm_f32_add(0, M, N, K, pa, pw, pr, pfused, ws, wsb, None) == -3
        assert L.aar_gemm_f32_bias_add(2, M, N, K, pa, pw, pbias, pr, pfused, ws, wsb, None) == -3
        assert L.aar_gemm_f32_add(1, M, N, K, pa, pw, None, pfused, ws, wsb, None) == -1
    finally:
        abi.free()
