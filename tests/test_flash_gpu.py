"""Flash-attention parity on the GPU: forward O and lse, backward dQ/dK/dV,
against the oracle (the reference's CPU composite restated, and its float64
lse) at the reference tests' shapes, the golden vectors from the reference CPU
build, sampled heads of BASELINE config 4 and full-size checksum identities.
Tolerance 1e-4 on both error metrics."""
from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

import oracle as O
from conftest import TOL, assert_close
from devutil import Abi, abi_flash, dev, host

pytestmark = pytest.mark.gpu
f32 = np.float32
GOLDEN = O.HERE.parent / "tests" / "golden"


def run_flash(gpu, q, k, v, do, causal):
    tq, tk, tv = dev(gpu, q, True), dev(gpu, k, True), dev(gpu, v, True)
    o = gpu.flash_attention(tq, tk, tv, causal)
    o.backward(dev(gpu, do))
    return host(gpu, o), host(gpu, tq.grad), host(gpu, tk.grad), host(gpu, tv.grad)


def lse_of(gpu, q, k, v, causal):
    _, lse = gpu._core._flash_attention_fwd(dev(gpu, q), dev(gpu, k), dev(gpu, v), causal)
    return host(gpu, lse)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("T", [8, 32, 33, 64])
def test_reference_forward_shapes(gpu, causal, T):
    # tests/python/test_flash_attention.py:29-44 (B2 H4 d16), deterministic seed
    rng = np.random.default_rng(1000 + T + causal)
    q, k, v = (rng.standard_normal((2, 4, T, 16)).astype(f32) for _ in range(3))
    o = host(gpu, gpu.flash_attention(dev(gpu, q), dev(gpu, k), dev(gpu, v), causal))
    o_ref = O.attention(q, k, v, causal)
    np.testing.assert_allclose(o, o_ref, atol=1e-4)
    assert_close(o, o_ref, TOL, "O")
    assert_close(lse_of(gpu, q, k, v, causal), O.attention_lse(q, k, causal), TOL, "lse")


def test_reference_dq_case(gpu):
    # tests/python/test_flash_attention.py:47-77 (B1 H2 T4 d8, causal, loss = sum(out))
    rng = np.random.default_rng(7)
    q, k, v = (rng.standard_normal((1, 2, 4, 8)).astype(f32) for _ in range(3))
    ones = np.ones_like(q)
    _, dq, dk, dv = run_flash(gpu, q, k, v, ones, True)
    rq, rk, rv = O.attention_backward(q, k, v, ones, True)
    for got, ref, n in ((dq, rq, "dq"), (dk, rk, "dk"), (dv, rv, "dv")):
        assert_close(got, ref, TOL, n)


@pytest.mark.parametrize("causal", [0, 1])
def test_golden_cpu_gpu_parity(gpu, causal):
    # tests/python/test_flash_attention.py:80-112 inputs; outputs from the reference CPU build
    z = np.load(GOLDEN / "attention_b2h4t64d16.npz")
    o, dq, dk, dv = run_flash(gpu, z["q"], z["k"], z["v"], z["do"], bool(causal))
    np.testing.assert_allclose(o, z[f"o_{causal}"], atol=1e-4)
    for got, name in ((o, "o"), (dq, "dq"), (dk, "dk"), (dv, "dv")):
        assert_close(got, z[f"{name}_{causal}"], TOL, name)


@pytest.mark.parametrize("shape", [(1, 3, 100, 64), (2, 2, 257, 64), (1, 2, 130, 128), (1, 1, 70, 36),
                                   (3, 1, 1, 32), (1, 2, 96, 48)])
@pytest.mark.parametrize("causal", [False, True])
def test_shapes_vs_oracle(gpu, shape, causal):
    rng = np.random.default_rng(sum(shape) + causal)
    q, k, v, do = (rng.standard_normal(shape).astype(f32) for _ in range(4))
    o, dq, dk, dv = run_flash(gpu, q, k, v, do, causal)
    assert_close(o, O.attention(q, k, v, causal), TOL, "O")
    rq, rk, rv = O.attention_backward(q, k, v, do, causal)
    for got, ref, n in ((dq, rq, "dq"), (dk, rk, "dk"), (dv, rv, "dv")):
        assert_close(got, ref, TOL, n)
    assert_close(lse_of(gpu, q, k, v, causal), O.attention_lse(q, k, causal), TOL, "lse")


def _config4(T, seed):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal((8, 12, T, 64)).astype(f32) for _ in range(4)]


def _checksums(q, o, dk, dv, do):
    """Size-independent identities over every head: sum_j dV[j] = sum_i dO[i]
    (rows of P sum to 1) and sum_j dK[j] = 0 (rows of dS sum to 0)."""
    sdv = dv.astype(np.float64).sum(2)
    sdo = do.astype(np.float64).sum(2)
    assert_close(sdv, sdo, TOL, "sum dV = sum dO")
    sdk = np.abs(dk.astype(np.float64).sum(2)).max()
    scale = np.abs(dk.astype(np.float64)).sum(2).max()
    assert sdk <= TOL * scale, f"sum dK = {sdk:.3e} (scale {scale:.3e})"
    assert np.isfinite(o).all()


def test_config4_t1024_sampled_heads(gpu):
    q, k, v, do = _config4(1024, 0)
    o, dq, dk, dv = run_flash(gpu, q, k, v, do, True)
    lse = lse_of(gpu, q, k, v, True)
    for b, h in ((0, 0), (5, 7)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        assert_close(o[sl], O.attention(q[sl], k[sl], v[sl], True), TOL, "O")
        rq, rk, rv = O.attention_backward(q[sl], k[sl], v[sl], do[sl], True)
        assert_close(dq[sl], rq, TOL, "dq")
        assert_close(dk[sl], rk, TOL, "dk")
        assert_close(dv[sl], rv, TOL, "dv")
        assert_close(lse[sl], O.attention_lse(q[sl], k[sl], True), TOL, "lse")
    _checksums(q, o, dk, dv, do)


def _closed64(q, k, v, do):
    q, k, v, do = (t.astype(np.float64) for t in (q, k, v, do))
    T, d = q.shape[-2:]
    s = q @ k.T / math.sqrt(d)
    s = np.where(np.triu(np.ones((T, T), bool), 1), -np.inf, s)
    m = s.max(-1, keepdims=True)
    e = np.exp(s - m)
    l = e.sum(-1, keepdims=True)
    p = e / l
    dp = do @ v.T
    ds = p * (dp - (dp * p).sum(-1, keepdims=True))
    return p @ v, (m + np.log(l))[:, 0], ds @ k / math.sqrt(d), ds.T @ q / math.sqrt(d), p.T @ do


def test_config4_t4096_sampled_head(gpu):
    q, k, v, do = _config4(4096, 1)
    o, dq, dk, dv = run_flash(gpu, q, k, v, do, True)
    lse = lse_of(gpu, q, k, v, True)
    b, h = 3, 11
    ro, rl, rq, rk, rv = _closed64(q[b, h], k[b, h], v[b, h], do[b, h])
    for got, ref, n in ((o, ro, "O"), (lse, rl, "lse"), (dq, rq, "dq"), (dk, rk, "dk"), (dv, rv, "dv")):
        assert_close(got[b, h], ref, TOL, n)
    _checksums(q, o, dk, dv, do)


def test_backward_is_reproducible(gpu):
    rng = np.random.default_rng(2)
    q, k, v, do = (rng.standard_normal((2, 3, 300, 64)).astype(f32) for _ in range(4))
    r1 = run_flash(gpu, q, k, v, do, True)
    r2 = run_flash(gpu, q, k, v, do, True)
    for a, c in zip(r1, r2):
        np.testing.assert_array_equal(a, c)


def test_strided_views_like_mha(gpu):
    """nn.MultiHeadAttention feeds slice/squeeze/transpose views of qkv
    [B,T,3,H,d] (aargrad/nn.py:177-189); the kernels read them in place."""
    B, T, H, d = 2, 48, 3, 16
    rng = np.random.default_rng(9)
    qkv = rng.standard_normal((B, T, 3, H, d)).astype(f32)
    t = dev(gpu, qkv, True)

    def take(i):
        return gpu.transpose(gpu.squeeze(gpu.slice(t, 2, i, i + 1), 2), 1, 2)

    q, k, v = take(0), take(1), take(2)
    assert not q.is_contiguous()
    o = gpu.flash_attention(q, k, v, True)
    do = rng.standard_normal((B, H, T, d)).astype(f32)
    o.backward(dev(gpu, do))
    qn, kn, vn = (np.ascontiguousarray(qkv[:, :, i].transpose(0, 2, 1, 3)) for i in range(3))
    assert_close(host(gpu, o), O.attention(qn, kn, vn, True), TOL, "O")
    rq, rk, rv = O.attention_backward(qn, kn, vn, do, True)
    g = host(gpu, t.grad)
    for i, ref in enumerate((rq, rk, rv)):
        assert_close(g[:, :, i].transpose(0, 2, 1, 3), ref, TOL, f"d{'qkv'[i]}")


def test_abi_misaligned(gpu):
    bh, T, d = 3, 77, 64
    rng = np.random.default_rng(4)
    q, k, v, do = (rng.standard_normal((bh, T, d)).astype(f32) for _ in range(4))
    abi = Abi()
    try:
        pq, pk, pv, pdo = (abi.put(t, 1) for t in (q, k, v, do))
        po, pl = abi.empty(bh * T * d, 1), abi.empty(bh * T)
        s = 1.0 / math.sqrt(d)
        abi.check(abi.L.aar_flash_fwd_f32(pq, pk, pv, po, pl, bh, T, d, 1, s, None))
        assert_close(abi.get(po, (bh, T, d)), O.attention(q, k, v, True), TOL, "O")
        wsb = abi.L.aar_flash_bwd_workspace_bytes(bh, T, d)
        pdq, pdk, pdv = (abi.empty(bh * T * d, 1) for _ in range(3))
        assert abi.L.aar_flash_bwd_f32(pq, pk, pv, po, pl, pdo, pdq, pdk, pdv, bh, T, d, 1, s,
                                       None, 0, None) == -2
        abi.check(abi.L.aar_flash_bwd_f32(pq, pk, pv, po, pl, pdo, pdq, pdk, pdv, bh, T, d, 1, s,
                                          abi.alloc(wsb), wsb, None))
        rq, rk, rv = O.attention_backward(q, k, v, do, True)
        for p, ref, n in ((pdq, rq, "dq"), (pdk, rk, "dk"), (pdv, rv, "dv")):
            assert_close(abi.get(p, (bh, T, d)), ref, TOL, n)
    finally:
        abi.free()


def _paths_agree(fast, slow, bh, T, d, causal):
    """The stored-dS and recompute backward paths share the dK/dV kernel (bit
    for bit).  Their dQ passes run the key tiles in one order, except the
    paired dQ pass (planned with 64-key dK/dV blocks), which sums two key
    phases: then dQ agrees to rounding."""
    np.testing.assert_array_equal(fast[1], slow[1])
    np.testing.assert_array_equal(fast[2], slow[2])
    L = Abi().L
    L.aar_flash_bwd_plan.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                     ctypes.POINTER(ctypes.c_int)]
    kb = ctypes.c_int()
    assert L.aar_flash_bwd_plan(bh, T, d, int(causal), 1, ctypes.byref(kb)) == 0
    if kb.value == 128:
        np.testing.assert_array_equal(fast[0], slow[0])
    else:
        assert_close(fast[0], slow[0], 1e-5, "dq stored dS vs recompute")


def _abi_bwd_both_paths(q, k, v, do, causal):
    """(O, grads through the recompute path, grads through the stored-dS
    path) via the C ABI: the workspace size selects the path."""
    bh, T, d = q.shape
    abi = Abi()
    try:
        pq, pk, pv, pdo = (abi.put(t) for t in (q, k, v, do))
        po, pl = abi.empty(bh * T * d), abi.empty(bh * T)
        s = 1.0 / math.sqrt(d)
        abi.check(abi.L.aar_flash_fwd_f32(pq, pk, pv, po, pl, bh, T, d, int(causal), s, None))
        out = [abi.get(po, (bh, T, d))]
        small = abi.L.aar_flash_bwd_workspace_bytes(bh, T, d)
        big = abi.L.aar_flash_bwd_fast_workspace_bytes(bh, T, d, int(causal))
        assert big > small
        for wsb in (small, big):
            pdq, pdk, pdv = (abi.empty(bh * T * d) for _ in range(3))
            abi.check(abi.L.aar_flash_bwd_f32(pq, pk, pv, po, pl, pdo, pdq, pdk, pdv, bh, T, d, int(causal), s,
                                              abi.alloc(wsb), wsb, None))
            out.append([abi.get(p, (bh, T, d)) for p in (pdq, pdk, pdv)])
        return out
    finally:
        abi.free()


@pytest.mark.parametrize("bh,T,d,causal", [(3, 77, 64, True), (2, 45, 64, False), (2, 130, 100, True),
                                           (1, 33, 32, False), (2, 257, 128, True), (4, 64, 64, True),
                                           (2, 96, 128, False)])
def test_abi_stored_ds_path(gpu, bh, T, d, causal):
    """Both backward paths against the oracle, and against each other (see
    _paths_agree)."""
    rng = np.random.default_rng(bh * 1000 + T + d)
    q, k, v, do = (rng.standard_normal((bh, T, d)).astype(f32) for _ in range(4))
    o, slow, fast = _abi_bwd_both_paths(q, k, v, do, causal)
    assert_close(o, O.attention(q, k, v, causal), TOL, "O")
    ref = O.attention_backward(q, k, v, do, causal)
    for g, r, n in zip(fast, ref, ("dq", "dk", "dv")):
        assert_close(g, r, TOL, n + " (stored dS)")
    _paths_agree(fast, slow, bh, T, d, causal)


def test_stored_ds_padded_keys_with_extreme_lse(gpu):
    """Logits near -128 put lse below -88, where exp(-lse) overflows: the
    padded keys of the last tile (T = 45) must store dS = 0, not inf * 0."""
    bh, T, d = 2, 45, 64
    rng = np.random.default_rng(5)
    q = (4 + 0.1 * rng.standard_normal((bh, T, d))).astype(f32)
    k = (-4 + 0.1 * rng.standard_normal((bh, T, d))).astype(f32)
    v, do = (rng.standard_normal((bh, T, d)).astype(f32) for _ in range(2))
    assert O.attention_lse(q, k, False).max() < -88
    o, slow, fast = _abi_bwd_both_paths(q, k, v, do, False)
    for a in fast + slow:
        assert np.isfinite(a).all()
    _paths_agree(fast, slow, bh, T, d, False)
    # logits of magnitude 128 carry absolute rounding ~1e-5 into exp
    ref = O.attention_backward(q, k, v, do, False)
    for g, r, n in zip(fast, ref, ("dq", "dk", "dv")):
        assert_close(g, r, 1e-3, n)


def test_head_dim_limit(gpu):
    x = dev(gpu, np.zeros((1, 4, 136), f32))
    with pytest.raises(ValueError, match="D_MAX"):
        gpu.flash_attention(x, x, x, True)


def _packed_reference(qkv, H, causal, do):
    """Per-head q/k/v of a packed [B,T,3D] projection, oracle O [B,T,D] and
    the packed gradient for upstream dO [B,T,D]."""
    B, T, D3 = qkv.shape
    D = D3 // 3
    d = D // H
    heads = qkv.reshape(B, T, 3, H, d)
    q, k, v = (np.ascontiguousarray(heads[:, :, i].transpose(0, 2, 1, 3)).reshape(B * H, T, d) for i in range(3))
    o = O.attention(q, k, v, causal).reshape(B, H, T, d).transpose(0, 2, 1, 3).reshape(B, T, D)
    dob = np.ascontiguousarray(do.reshape(B, T, H, d).transpose(0, 2, 1, 3)).reshape(B * H, T, d)
    gq, gk, gv = O.attention_backward(q, k, v, dob, causal)
    g = np.stack([x.reshape(B, H, T, d).transpose(0, 2, 1, 3) for x in (gq, gk, gv)], axis=2)
    return o, g.reshape(B, T, 3 * D)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", [(2, 70, 3, 16), (1, 64, 2, 64), (2, 33, 2, 18)], ids=str)
def test_packed_qkv_attention(gpu, shape, causal):
    """_flash_attention_qkv (MultiHeadAttention's fused path) against the
    oracle on the per-head views, forward and the packed gradient; d = 18
    takes the element-wise (non-128-bit) path."""
    B, T, H, d = shape
    D = H * d
    rng = np.random.default_rng(B * T + H * d + causal)
    qkv = rng.standard_normal((B, T, 3 * D)).astype(f32)
    do = rng.standard_normal((B, T, D)).astype(f32)
    t = dev(gpu, qkv, True)
    o = gpu._core._flash_attention_qkv(t, H, causal)
    assert o.shape == [B, T, D] and o.is_contiguous()
    o.backward(dev(gpu, do))
    ro, rg = _packed_reference(qkv, H, causal, do)
    assert_close(host(gpu, o), ro, TOL, "O")
    assert_close(host(gpu, t.grad), rg, TOL, "dqkv")


def test_mha_fused_equals_views(gpu):
    """nn.MultiHeadAttention.forward (fused) and forward_views (the
    reference's literal composition) give the same output and gradients."""
    from aargrad import nn
    rng = np.random.default_rng(12)
    B, T, D, H = 2, 40, 48, 3
    mha = nn.MultiHeadAttention(D, H, causal=True, bias=True, rng=rng).to(gpu.Device.CUDA)
    x_np = rng.standard_normal((B, T, D)).astype(f32)
    g_np = rng.standard_normal((B, T, D)).astype(f32)
    outs, grads = [], []
    for fwd in (mha.forward, mha.forward_views):
        mha.zero_grad()
        x = dev(gpu, x_np, True)
        y = fwd(x)
        y.backward(dev(gpu, g_np))
        outs.append(host(gpu, y))
        grads.append([host(gpu, x.grad)] + [host(gpu, p.tensor.grad) for p in mha.parameters()])
    assert_close(outs[0], outs[1], TOL, "y")
    for a, b in zip(grads[0], grads[1]):
        assert_close(a, b, TOL, "grad")


def test_rank5_and_unfoldable_batch_views(gpu):
    """Leading dims fold into one batch stride when they nest; a view whose
    batch dims do not nest (swapped) is copied first.  Both match the oracle."""
    rng = np.random.default_rng(13)
    q, k, v = (rng.standard_normal((2, 3, 2, 40, 16)).astype(f32) for _ in range(3))
    o = host(gpu, gpu.flash_attention(dev(gpu, q), dev(gpu, k), dev(gpu, v), True))
    ref = O.attention(q.reshape(12, 40, 16), k.reshape(12, 40, 16), v.reshape(12, 40, 16), True)
    assert_close(o.reshape(12, 40, 16), ref, TOL, "rank5")
    tq, tk, tv = (gpu.transpose(dev(gpu, x), 0, 1) for x in (q, k, v))  # [3, 2, 2, T, d] views
    assert not tq.is_contiguous()
    o2 = host(gpu, gpu.flash_attention(tq, tk, tv, True))
    qs, ks, vs = (np.ascontiguousarray(x.transpose(1, 0, 2, 3, 4)).reshape(12, 40, 16) for x in (q, k, v))
    assert_close(o2.reshape(12, 40, 16), O.attention(qs, ks, vs, True), TOL, "swapped batch")


def test_abi_strided_output_layout(gpu):
    """aar_flash_fwd/bwd_strided_f32 with q/k/v read from a packed
    [B,T,3,H,d] buffer and O, dO, dq/dk/dv in [B,T,H,d] order."""
    B, T, H, d = 2, 50, 3, 32
    rng = np.random.default_rng(14)
    qkv = rng.standard_normal((B, T, 3, H, d)).astype(f32)
    do = rng.standard_normal((B, T, H, d)).astype(f32)
    abi = Abi()
    L = abi.L
    i64p = ctypes.POINTER(ctypes.c_int64)
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    L.aar_flash_fwd_strided_f32.argtypes = [vp] * 5 + [i64] * 4 + [i64p, ctypes.c_int, ctypes.c_float, vp,
                                                                  ctypes.c_size_t, vp]
    L.aar_flash_bwd_strided_f32.argtypes = [vp] * 9 + [i64] * 4 + [i64p, ctypes.c_int, ctypes.c_float, vp,
                                                                  ctypes.c_size_t, vp]
    try:
        px = abi.put(qkv)
        D = H * d
        pk = [T * 3 * D, d, 3 * D]
        po = [T * D, d, D]
        st = (ctypes.c_int64 * 24)(*(pk * 3 + po + po + [T * 3 * D, d, 3 * D] * 3))
        pq, pkk, pv = px, px + 4 * D, px + 8 * D
        pout, plse = abi.empty(B * T * D), abi.empty(B * H * T)
        s = 1.0 / math.sqrt(d)
        abi.check(L.aar_flash_fwd_strided_f32(pq, pkk, pv, pout, plse, B, H, T, d, st, 1, s, None, 0, None))
        ro, rg = _packed_reference(qkv.reshape(B, T, 3 * D), H, True, do.reshape(B, T, D))
        assert_close(abi.get(pout, (B, T, D)), ro, TOL, "O")
        pdo = abi.put(do)
        pg = abi.empty(B * T * 3 * D)
        wsb = L.aar_flash_bwd_workspace_bytes(B * H, T, d)
        abi.check(L.aar_flash_bwd_strided_f32(pq, pkk, pv, pout, plse, pdo, pg, pg + 4 * D, pg + 8 * D, B, H, T,
                                              d, st, 1, s, abi.alloc(wsb), wsb, None))
        assert_close(abi.get(pg, (B, T, 3 * D)), rg, TOL, "dqkv")
    finally:
        abi.free()


def _abi_forward(q, k, v, causal, split, offset=0):
    """(O, lse) of the strided forward with contiguous strides, with the split
    workspace (split=True) or none (every query block one workgroup)."""
    bh, T, d = q.shape
    abi = Abi()
    L = abi.L
    i64p = ctypes.POINTER(ctypes.c_int64)
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    L.aar_flash_fwd_strided_f32.argtypes = [vp] * 5 + [i64] * 4 + [i64p, ctypes.c_int, ctypes.c_float, vp,
                                                                  ctypes.c_size_t, vp]
    L.aar_flash_fwd_workspace_bytes.restype = ctypes.c_size_t
    L.aar_flash_fwd_workspace_bytes.argtypes = [i64] * 3 + [ctypes.c_int]
    try:
        pq, pk, pv = (abi.put(t, offset) for t in (q, k, v))
        po, pl = abi.empty(bh * T * d, offset), abi.empty(bh * T)
        st = (ctypes.c_int64 * 12)(*([bh * T * d, T * d, d] * 4))
        wsb = L.aar_flash_fwd_workspace_bytes(bh, T, d, int(causal)) if split else 0
        if split:
            assert wsb > 0
        ws = abi.alloc(wsb) if wsb else None
        abi.check(L.aar_flash_fwd_strided_f32(pq, pk, pv, po, pl, 1, bh, T, d, st, int(causal),
                                              1.0 / math.sqrt(d), ws, wsb, None))
        return abi.get(po, (bh, T, d)), abi.get(pl, (bh, T))
    finally:
        abi.free()


@pytest.mark.parametrize("bh,T,d,offset", [(2, 300, 64, 0), (3, 1000, 64, 0), (1, 257, 128, 0), (2, 256, 32, 0),
                                           (2, 300, 30, 0), (2, 390, 64, 1), (1, 2048, 64, 0)])
def test_abi_forward_key_range_split(gpu, bh, T, d, offset):
    """Causal forward with the key-range split (the longest half of the query
    blocks as two workgroups each, merged by the combine pass) against the
    oracle and against the unsplit launch.  offset=1 misaligns the operands,
    which takes the element-wise load path."""
    rng = np.random.default_rng(bh * 7919 + T + d)
    q, k, v = (rng.standard_normal((bh, T, d)).astype(f32) for _ in range(3))
    o_split, l_split = _abi_forward(q, k, v, True, True, offset)
    o_whole, l_whole = _abi_forward(q, k, v, True, False, offset)
    assert_close(o_split, O.attention(q, k, v, True), TOL, "O split")
    assert_close(l_split, O.attention_lse(q, k, True), TOL, "lse split")
    # same softmax over the same keys, merged from two halves: agreement far
    # below the tolerance
    assert_close(o_split, o_whole, 1e-5, "O split vs whole")
    assert_close(l_split, l_whole, 1e-5, "lse split vs whole")


def _flash_plans():
    L = Abi().L
    ip = ctypes.POINTER(ctypes.c_int)
    L.aar_flash_bwd_plan.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ip]
    L.aar_flash_fwd_plan.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_size_t, ip]
    L.aar_flash_fwd_workspace_bytes.restype = ctypes.c_size_t
    L.aar_flash_fwd_workspace_bytes.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int]
    L.aar_flash_fwd_query_block.argtypes = L.aar_flash_bwd_plan.argtypes
    return L


def _fwd_qb(L, bh, T, d, causal, vec=1):
    out = ctypes.c_int()
    assert L.aar_flash_fwd_query_block(bh, T, d, int(causal), vec, ctypes.byref(out)) == 0
    return out.value


def _bwd_plan(L, bh, T, d, causal, vec=1):
    out = ctypes.c_int()
    assert L.aar_flash_bwd_plan(bh, T, d, int(causal), vec, ctypes.byref(out)) == 0
    return out.value


def test_flash_plans(gpu):
    """The plan queries: the paired 64-key dK/dV kernel for grids of about one
    round with d = 64 on the 128-bit path, 128-key workgroups otherwise;
    the forward's key-range split for under-filled causal grids only."""
    L = _flash_plans()
    assert _bwd_plan(L, 384, 256, 64, True) == 64     # the GPT step's attention
    assert _bwd_plan(L, 96, 1024, 64, True) == 64     # BASELINE config 4, T = 1024
    assert _bwd_plan(L, 96, 4096, 64, True) == 128    # BASELINE config 4, T = 4096
    assert _bwd_plan(L, 8, 300, 64, False) == 64
    for d in (32, 48, 100, 128):                      # other head dims
        assert _bwd_plan(L, 8, 256, d, True) == 128
    assert _bwd_plan(L, 8, 256, 64, True, vec=0) == 128
    out = ctypes.c_int()
    assert L.aar_flash_bwd_plan(8, 256, 200, 1, 1, ctypes.byref(out)) == -1
    # forward split: with its workspace, a small causal grid splits, a full one does not
    for bh, T, want_split in ((2, 2048, True), (12, 1024, True), (96, 1024, True), (192, 512, False),
                              (96, 4096, False)):
        wsb = L.aar_flash_fwd_workspace_bytes(bh, T, 64, 1)
        assert L.aar_flash_fwd_plan(bh, T, 64, 1, 1, wsb, ctypes.byref(out)) == 0
        assert (out.value > 0) == want_split, (bh, T, out.value)
        assert L.aar_flash_fwd_plan(bh, T, 64, 1, 1, 0, ctypes.byref(out)) == 0 and out.value == 0
        assert L.aar_flash_fwd_plan(bh, T, 64, 0, 1, wsb, ctypes.byref(out)) == 0 and out.value == 0
    # forward query blocks: the paired 64-query kernel for causal d = 64 grids of up
    # to two rounds of 128-query workgroups (four for T <= 1024)
    assert _fwd_qb(L, 384, 256, 64, True) == 64      # the GPT step's attention
    assert _fwd_qb(L, 8, 100, 64, True) == 64
    assert _fwd_qb(L, 8, 512, 48, True) == 128       # the paired kernel's DMA layout is d = 64 exactly
    assert _fwd_qb(L, 96, 1024, 64, True) == 64      # BASELINE config 4, T = 1024
    assert _fwd_qb(L, 12, 4096, 64, True) == 64
    assert _fwd_qb(L, 96, 4096, 64, True) == 128     # four rounds at T = 4096
    assert _fwd_qb(L, 4096, 256, 64, True) == 128    # many rounds of 128-query workgroups
    assert _fwd_qb(L, 8, 256, 64, False) == 128
    for d in (32, 48, 63, 100, 128):
        assert _fwd_qb(L, 8, 256, d, True) == 128
    assert _fwd_qb(L, 8, 256, 64, True, vec=0) == 128
    assert L.aar_flash_fwd_query_block(8, 256, 200, 1, 1, ctypes.byref(out)) == -1


def test_forced_plan_is_per_call(gpu):
    """The plan entry points reject block sizes other than 0/64/128 before
    any launch, and forcing a plan for one call leaves the planner's answer
    (and so every later unforced call) unchanged: the library holds no plan
    state."""
    L = _flash_plans()
    bh, T, d = 4, 96, 64
    rng = np.random.default_rng(3)
    q, k, v, do = (rng.standard_normal((bh, T, d)).astype(f32) for _ in range(4))
    for bad in (96, -1, 1):
        with pytest.raises(RuntimeError):
            abi_flash(q, k, v, do, True, query_block=bad)
        with pytest.raises(RuntimeError):
            abi_flash(q, k, v, do, True, key_block=bad)
    before = (_fwd_qb(L, 384, 256, 64, True), _bwd_plan(L, 384, 256, 64, True))
    abi_flash(q, k, v, do, True, query_block=128, key_block=128)
    assert (_fwd_qb(L, 384, 256, 64, True), _bwd_plan(L, 384, 256, 64, True)) == before == (64, 64)


@pytest.mark.parametrize("query_block", [64, 128])
@pytest.mark.parametrize("bh,T,d", [(3, 77, 64), (1, 1, 64), (2, 33, 64), (2, 257, 64), (4, 64, 64),
                                    (2, 130, 48), (5, 31, 64), (3, 200, 64), (1, 511, 64), (2, 96, 64),
                                    (2, 448, 64), (1, 320, 64), (1, 1100, 64), (1, 2051, 64)])
def test_fwd_query_blocks_vs_oracle(gpu, query_block, bh, T, d):
    """Both causal forward decompositions (forced) against the oracle: O and
    lse, then the backward through the forward's lse.  The paired kernel
    merges two key phases per query tile in a fixed order, so a rerun is bit
    identical.  T > 1024 takes its double-buffered form, T <= 1024 the
    single-stage one."""
    L = _flash_plans()
    rng = np.random.default_rng(bh * 131 + T + d + query_block)
    q, k, v, do = (rng.standard_normal((bh, T, d)).astype(f32) for _ in range(4))
    assert _fwd_qb(L, bh, T, d, True) in (64, 128)
    o, lse, grads = abi_flash(q, k, v, do, True, query_block=query_block)
    o2, lse2, _ = abi_flash(q, k, v, do, True, query_block=query_block)
    np.testing.assert_array_equal(o, o2)
    np.testing.assert_array_equal(lse, lse2)
    assert_close(o, O.attention(q, k, v, True), TOL, f"O (query block {query_block})")
    assert_close(lse, O.attention_lse(q, k, True), TOL, f"lse (query block {query_block})")
    for g, r, n in zip(grads, O.attention_backward(q, k, v, do, True), ("dq", "dk", "dv")):
        assert_close(g, r, TOL, f"{n} (query block {query_block})")


@pytest.mark.parametrize("key_block", [64, 128])
@pytest.mark.parametrize("bh,T,d,causal", [(3, 77, 64, True), (2, 45, 64, False), (1, 1, 64, True),
                                           (2, 33, 64, True), (2, 257, 64, True), (4, 64, 64, True),
                                           (2, 96, 64, False), (1, 300, 64, False), (2, 130, 64, True),
                                           (5, 31, 64, True), (2, 65, 64, False), (3, 200, 64, True)])
def test_dkdv_key_blocks_vs_oracle(gpu, key_block, bh, T, d, causal):
    """Both backward decompositions (forced) against the oracle through both
    backward paths.  The two paths share the dK/dV kernel, so dK and dV agree
    bit for bit; with 128-key blocks both dQ passes also run the key tiles in
    one sequential order (bit for bit), while the paired dQ pass sums two key
    phases and agrees with the recompute pass to rounding."""
    rng = np.random.default_rng(bh * 977 + T + d + causal)
    q, k, v, do = (rng.standard_normal((bh, T, d)).astype(f32) for _ in range(4))
    o, _, fast = abi_flash(q, k, v, do, causal, key_block=key_block, fast=True)
    _, _, slow = abi_flash(q, k, v, do, causal, key_block=key_block, fast=False)
    assert_close(o, O.attention(q, k, v, causal), TOL, "O")
    ref = O.attention_backward(q, k, v, do, causal)
    for g, r, n in zip(fast, ref, ("dq", "dk", "dv")):
        assert_close(g, r, TOL, f"{n} (key block {key_block})")
    for g, r, n in zip(slow, ref, ("dq", "dk", "dv")):
        assert_close(g, r, TOL, f"{n} (key block {key_block}, recompute)")
    np.testing.assert_array_equal(fast[1], slow[1])
    np.testing.assert_array_equal(fast[2], slow[2])
    if key_block == 128:
        np.testing.assert_array_equal(fast[0], slow[0])
    else:
        assert_close(fast[0], slow[0], 1e-5, "dq paired vs recompute")


def test_paired_dkdv_at_config5_shape_and_reruns(gpu):
    """The paired kernel at the GPT step's attention shape (planned there), on
    the packed-qkv strided views, against the oracle on sampled heads and
    bit-identical on a rerun."""
    L = _flash_plans()
    B, T, H, d = 64, 256, 6, 64
    assert _bwd_plan(L, B * H, T, d, True) == 64
    rng = np.random.default_rng(12)
    D = H * d
    qkv = rng.standard_normal((B, T, 3 * D)).astype(f32)
    do = rng.standard_normal((B, T, D)).astype(f32)
    grads = []
    for _ in range(2):
        t = dev(gpu, qkv, True)
        gpu._core._flash_attention_qkv(t, H, True).backward(dev(gpu, do))
        grads.append(host(gpu, t.grad))
    np.testing.assert_array_equal(grads[0], grads[1])
    g = grads[0].reshape(B, T, 3, H, d)
    heads = qkv.reshape(B, T, 3, H, d)
    dob = do.reshape(B, T, H, d)
    for b, h in ((0, 0), (40, 5)):
        q, k, v = (np.ascontiguousarray(heads[b, :, i, h])[None] for i in range(3))
        rq, rk, rv = O.attention_backward(q, k, v, np.ascontiguousarray(dob[b, :, h])[None], True)
        for i, ref in enumerate((rq, rk, rv)):
            assert_close(g[b, :, i, h][None], ref, TOL, f"d{'qkv'[i]} ({b},{h})")
