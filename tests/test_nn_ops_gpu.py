"""GPU parity of the GPT-step ops against the oracle: elementwise family,
bias add/grad, sum_all, SGD/AdamW updates, embedding (one-hot MFMA backward)
and cross entropy, including ignore_index, deferred out-of-range errors and
bit-reproducible reductions.  Tolerance 1e-4 (both metrics) except where the
op is exact."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from conftest import TOL, assert_close
from devutil import dev, host

pytestmark = pytest.mark.gpu
f32 = np.float32


def ids_dev(gpu, ids):
    return gpu.from_numpy(np.ascontiguousarray(ids, np.int64)).to(gpu.Device.CUDA)


@pytest.mark.parametrize("n", [1, 7, 4096, 1_000_003])
def test_elementwise_family(gpu, n):
    rng = np.random.default_rng(n)
    a, b, g = (rng.standard_normal(n).astype(f32) for _ in range(3))
    ta, tb = dev(gpu, a, True), dev(gpu, b, True)
    np.testing.assert_array_equal(host(gpu, gpu.sub(ta, tb)), O.sub(a, b))
    np.testing.assert_array_equal(host(gpu, gpu.mul(ta, tb)), O.mul(a, b))
    np.testing.assert_array_equal(host(gpu, gpu.scale(ta, 0.37)), O.scale(a, 0.37))
    np.testing.assert_array_equal(host(gpu, gpu.relu(ta)), O.relu(a))
    assert_close(host(gpu, gpu.gelu(ta)), O.gelu(a), 1e-6, "gelu")
    # backward legs through autograd
    for name, fn, ref in (("relu", gpu.relu, O.relu_backward(g, a)), ("gelu", gpu.gelu, O.gelu_backward(g, a))):
        x = dev(gpu, a, True)
        fn(x).backward(dev(gpu, g))
        assert_close(host(gpu, x.grad), ref, 1e-6, f"{name} backward")
    x, y = dev(gpu, a, True), dev(gpu, b, True)
    gpu.mul(x, y).backward(dev(gpu, g))
    np.testing.assert_array_equal(host(gpu, x.grad), O.mul(g, b))
    np.testing.assert_array_equal(host(gpu, y.grad), O.mul(g, a))
    x, y = dev(gpu, a, True), dev(gpu, b, True)
    gpu.sub(x, y).backward(dev(gpu, g))
    np.testing.assert_array_equal(host(gpu, x.grad), g)
    np.testing.assert_array_equal(host(gpu, y.grad), -g)


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 5), (16384, 1536), (16384, 384), (1000, 65)])
def test_bias_add_and_grad(gpu, rows, cols):
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((rows, cols)).astype(f32)
    bias = rng.standard_normal(cols).astype(f32)
    g = rng.standard_normal((rows, cols)).astype(f32)
    tx, tb = dev(gpu, x, True), dev(gpu, bias, True)
    y = gpu.add_bias(tx, tb)
    y.backward(dev(gpu, g))
    np.testing.assert_array_equal(host(gpu, y), O.add_bias(x, bias))
    np.testing.assert_array_equal(host(gpu, tx.grad), g)
    assert_close(host(gpu, tb.grad), O.bias_grad(g, cols), TOL, "bias grad")


@pytest.mark.parametrize("n", [1, 10, 1000, 1 << 20, 3_000_001])
def test_sum_all_and_backward(gpu, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(f32)
    tx = dev(gpu, x, True)
    s = gpu.sum_all(tx)
    assert s.shape == []
    got = host(gpu, s)
    ref64 = x.astype(np.float64).sum()
    assert abs(float(got) - ref64) <= TOL * max(np.abs(x).sum(), 1.0)
    s.backward()
    np.testing.assert_array_equal(host(gpu, tx.grad), np.ones(n, f32))
    # reproducible
    assert host(gpu, gpu.sum_all(dev(gpu, x))) == got


def test_sum_all_reference_kat(gpu):
    # tests/cpp/test_autograd_ops.cpp:45-85: CUDA sum/mul fan-out, add_grads on device
    a = dev(gpu, np.array([1, 2, 3, 4], f32), True)
    gpu.sum_all(gpu.mul(a, a)).backward()
    np.testing.assert_array_equal(host(gpu, a.grad), [2, 4, 6, 8])


def test_sgd_and_adamw(gpu):
    rng = np.random.default_rng(3)
    p, g = rng.standard_normal(10001).astype(f32), rng.standard_normal(10001).astype(f32)
    tp = dev(gpu, p)
    gpu.scaled_add_inplace(tp, dev(gpu, g), -1e-3)
    # the device may fuse p + alpha*g into one fma: agreement to rounding
    assert_close(host(gpu, tp), O.scaled_add(p, g, -1e-3), 1e-6, "sgd")
    m, v = (0.1 * rng.standard_normal(10001)).astype(f32), np.abs(0.1 * rng.standard_normal(10001)).astype(f32)
    tp, tm, tv = dev(gpu, p), dev(gpu, m), dev(gpu, v)
    gpu.adamw_step(tp, dev(gpu, g), tm, tv, 1e-3, 0.9, 0.999, 1e-8, 0.01, 0.19, 0.002)
    rp, rm, rv = O.adamw(p, g, m, v, 1e-3, 0.9, 0.999, 1e-8, 0.01, 0.19, 0.002)
    assert_close(host(gpu, tm), rm, 1e-6, "m")
    assert_close(host(gpu, tv), rv, 1e-6, "v")
    assert_close(host(gpu, tp), rp, 1e-6, "p")


def test_multi_tensor_updates_bit_identical(gpu):
    # 100 tensors (three launches of at most 48), ragged sizes including empty
    # ones and chunk edges: the multi-tensor SGD / AdamW updates equal the
    # per-tensor ops bit for bit
    rng = np.random.default_rng(17)
    sizes = [int(s) for s in rng.choice([0, 1, 3, 4095, 4096, 4097, 12289, 70001], 100)]
    ps = [rng.standard_normal(n).astype(f32) for n in sizes]
    gs = [rng.standard_normal(n).astype(f32) for n in sizes]
    ms = [(0.1 * rng.standard_normal(n)).astype(f32) for n in sizes]
    vs = [np.abs(0.1 * rng.standard_normal(n)).astype(f32) for n in sizes]
    one = [dev(gpu, p) for p in ps]
    many = [dev(gpu, p) for p in ps]
    for t, g in zip(one, gs):
        gpu.scaled_add_inplace(t, dev(gpu, g), -3e-3)
    gpu._core._scaled_add_inplace_multi(many, [dev(gpu, g) for g in gs], -3e-3)
    for a, b in zip(one, many):
        np.testing.assert_array_equal(host(gpu, a), host(gpu, b))
    args = (1e-3, 0.9, 0.999, 1e-8, 0.01, 0.271, 0.00299)
    st1 = [(dev(gpu, p), dev(gpu, m), dev(gpu, v)) for p, m, v in zip(ps, ms, vs)]
    st2 = [(dev(gpu, p), dev(gpu, m), dev(gpu, v)) for p, m, v in zip(ps, ms, vs)]
    for (p, m, v), g in zip(st1, gs):
        gpu.adamw_step(p, dev(gpu, g), m, v, *args)
    gpu._core._adamw_step_multi([s[0] for s in st2], [dev(gpu, g) for g in gs], [s[1] for s in st2],
                                [s[2] for s in st2], *args)
    for a, b in zip(st1, st2):
        for x, y in zip(a, b):
            np.testing.assert_array_equal(host(gpu, x), host(gpu, y))
    # dst aliasing src: p += alpha * p
    t = dev(gpu, ps[0] if sizes[0] else np.ones(5, f32))
    ref = host(gpu, t)
    gpu._core._scaled_add_inplace_multi([t], [t], 0.5)
    np.testing.assert_array_equal(host(gpu, t), (ref + np.float32(0.5) * ref).astype(f32))
    with pytest.raises(ValueError, match="shape mismatch"):
        gpu._core._scaled_add_inplace_multi([dev(gpu, np.zeros(3, f32))], [dev(gpu, np.zeros(4, f32))], 1.0)


def test_multi_tensor_updates_with_repeated_parameters(gpu, ag):
    # A parameter listed twice (a shared module or a tied weight: Module.parameters()
    # does not de-duplicate) must be updated twice in list order, as the
    # reference's per-parameter loop does (aargrad/optim.py:13-18, :36-54); the
    # AdamW state is keyed by id(p), so both entries also share m and v.
    # Several repeats, an overlapping view and large tensors (many workgroups
    # per tensor) give concurrent updates every chance to race.
    rng = np.random.default_rng(23)
    sizes = [70001, 5, 300_000, 4097]
    init = [rng.standard_normal(n).astype(f32) for n in sizes]
    grads = [rng.standard_normal(n).astype(f32) for n in sizes]
    order = [0, 1, 0, 2, 3, 2, 0]
    # SGD: multi call vs sequential single-tensor calls
    multi = [dev(gpu, a) for a in init]
    seq = [dev(gpu, a) for a in init]
    gdev = [dev(gpu, g) for g in grads]
    gpu._core._scaled_add_inplace_multi([multi[i] for i in order], [gdev[i] for i in order], -0.25)
    for i in order:
        gpu.scaled_add_inplace(seq[i], gdev[i], -0.25)
    for a, b in zip(multi, seq):
        np.testing.assert_array_equal(host(gpu, a), host(gpu, b))
    # AdamW with shared m/v per repeated parameter
    args = (1e-2, 0.9, 0.999, 1e-8, 0.01, 0.1, 0.001)
    st_multi = [(dev(gpu, a), dev(gpu, np.zeros_like(a)), dev(gpu, np.zeros_like(a))) for a in init]
    st_seq = [(dev(gpu, a), dev(gpu, np.zeros_like(a)), dev(gpu, np.zeros_like(a))) for a in init]
    gpu._core._adamw_step_multi([st_multi[i][0] for i in order], [gdev[i] for i in order],
                                [st_multi[i][1] for i in order], [st_multi[i][2] for i in order], *args)
    for i in order:
        gpu.adamw_step(st_seq[i][0], gdev[i], st_seq[i][1], st_seq[i][2], *args)
    for a, b in zip(st_multi, st_seq):
        for x, y in zip(a, b):
            np.testing.assert_array_equal(host(gpu, x), host(gpu, y))
    # through optim.SGD with a module shared by two parents
    lin = ag.nn.Linear(6, 4)
    lin.to(gpu.Device.CUDA)
    params = list(lin.parameters()) + list(lin.parameters())
    x = dev(gpu, rng.standard_normal((3, 6)))
    gpu.sum_all(lin(x)).backward()
    before = [host(gpu, p.tensor) for p in lin.parameters()]
    grads_h = [host(gpu, p.tensor.grad) for p in lin.parameters()]
    ag.optim.SGD(params, lr=0.5).step()
    for p, b0, g in zip(lin.parameters(), before, grads_h):
        ref = b0 + np.float32(-0.5) * g
        ref = (ref + np.float32(-0.5) * g).astype(f32)
        np.testing.assert_array_equal(host(gpu, p.tensor), ref)


def test_optimizers_take_one_multi_tensor_step(gpu, ag):
    # optim.SGD / optim.AdamW (now one multi-tensor call per step) against the
    # reference optimizers' per-parameter loops (aargrad/optim.py:13-18, :36-54)
    rng = np.random.default_rng(5)
    shapes = [(8, 3), (3,), (0,), (5, 7)]
    for name in ("sgd", "adamw"):
        init = [rng.standard_normal(s).astype(f32) for s in shapes]
        grads = [rng.standard_normal(s).astype(f32) for s in shapes]
        params = [ag.nn.Parameter(dev(gpu, a)) for a in init]
        for p, g in zip(params, grads):
            gpu.sum_all(gpu.mul(p.tensor, dev(gpu, g))).backward()  # grad = g
        opt = ag.optim.SGD(params, lr=0.1) if name == "sgd" else ag.optim.AdamW(params, lr=1e-2)
        opt.step()
        opt.step()
        ref = [dev(gpu, a) for a in init]
        ms = [dev(gpu, np.zeros(s, f32)) for s in shapes]
        vs = [dev(gpu, np.zeros(s, f32)) for s in shapes]
        for t in (1, 2):
            for r, g, m, v in zip(ref, grads, ms, vs):
                if name == "sgd":
                    gpu.scaled_add_inplace(r, dev(gpu, g), -0.1)
                else:
                    gpu.adamw_step(r, dev(gpu, g), m, v, 1e-2, 0.9, 0.999, 1e-8, 0.01, 1 - 0.9 ** t, 1 - 0.999 ** t)
        for p, r in zip(params, ref):
            np.testing.assert_array_equal(host(gpu, p.tensor), host(gpu, r))


@pytest.mark.parametrize("vocab,dim,shape", [(7, 4, (2, 3)), (65, 384, (64, 256)), (256, 384, (64, 256)),
                                             (5, 3, (6,)), (3, 260, (5, 7)), (9, 4100, (3,))])
def test_embedding_fwd_bwd(gpu, vocab, dim, shape):
    rng = np.random.default_rng(vocab + dim)
    w = rng.standard_normal((vocab, dim)).astype(f32)
    ids = rng.integers(0, vocab, shape)
    g = rng.standard_normal(shape + (dim,)).astype(f32)
    tw = dev(gpu, w, True)
    y = gpu.embedding(tw, ids_dev(gpu, ids))
    assert y.shape == list(shape) + [dim]
    np.testing.assert_array_equal(host(gpu, y), O.embedding(w, ids))
    y.backward(dev(gpu, g))
    assert_close(host(gpu, tw.grad), O.embedding_backward(g, ids, vocab), TOL, "embedding dW")


@pytest.mark.parametrize("vocab,dim,B,T", [(256, 384, 64, 256), (260, 8, 3, 200), (300, 8, 2, 100)])
def test_embedding_backward_position_ids(gpu, vocab, dim, B, T):
    """Position ids (arange(T) per sequence, as the GPT step looks up its
    position table): in each 32-id tile only one 32-row block of the table
    occurs, and the short-M kernel skips the others; vocab 300 is past its
    260 rows and takes the one-hot GEMM path.  Rerun bit identical."""
    rng = np.random.default_rng(vocab + T)
    ids = np.tile(np.arange(T, dtype=np.int64), (B, 1))
    g = rng.standard_normal((B, T, dim)).astype(f32)
    outs = []
    for _ in range(2):
        tw = dev(gpu, rng.standard_normal((vocab, dim)).astype(f32), True)
        gpu.embedding(tw, ids_dev(gpu, ids)).backward(dev(gpu, g))
        outs.append(host(gpu, tw.grad))
    np.testing.assert_array_equal(outs[0], outs[1])
    assert_close(outs[0], O.embedding_backward(g, ids, vocab), TOL, "embedding dW at position ids")


@pytest.mark.parametrize("dim", [3, 8])  # the element-wise and the 128-bit row kernel
def test_embedding_out_of_range_is_reported(gpu, dim):
    w = dev(gpu, np.ones((5, dim), f32))
    y = gpu.embedding(w, ids_dev(gpu, np.array([1, 5, -1, 4], np.int64)))
    with pytest.raises(IndexError):
        host(gpu, y)
    w = dev(gpu, np.ones((5, 3), f32))
    y = gpu.embedding(w, ids_dev(gpu, np.array([1, 5], np.int64)))  # 5 is out of range
    with pytest.raises(IndexError):
        host(gpu, y)
    # the flag is cleared after reporting
    np.testing.assert_array_equal(host(gpu, gpu.embedding(w, ids_dev(gpu, np.array([0], np.int64)))),
                                  np.ones((1, 3), f32))


@pytest.mark.parametrize("dim,B,T", [(384, 64, 256), (8, 3, 50), (3, 2, 7)])  # 128-bit rows, element-wise
def test_embedding_add_matches_composition(gpu, dim, B, T):
    """_embedding_add (the GPT's token + position embeddings in one pass):
    output and both table gradients bit-identical to add(embedding, embedding),
    and against the oracle."""
    rng = np.random.default_rng(dim + T)
    tok, pos = rng.standard_normal((65, dim)).astype(f32), rng.standard_normal((T, dim)).astype(f32)
    ids = rng.integers(0, 65, (B, T))
    pids = np.tile(np.arange(T, dtype=np.int64), (B, 1))
    g = rng.standard_normal((B, T, dim)).astype(f32)
    res = []
    for fused in (True, False):
        tw, pw = dev(gpu, tok, True), dev(gpu, pos, True)
        a, b = ids_dev(gpu, ids), ids_dev(gpu, pids)
        if fused:
            y = gpu._core._embedding_add(tw, a, pw, b)
        else:
            y = gpu.add(gpu.embedding(tw, a), gpu.embedding(pw, b))
        y.backward(dev(gpu, g))
        res.append((host(gpu, y), host(gpu, tw.grad), host(gpu, pw.grad)))
    for x, y, name in zip(res[0], res[1], ("out", "d tok", "d pos")):
        np.testing.assert_array_equal(x, y, err_msg=name)
    np.testing.assert_array_equal(res[0][0], O.add(O.embedding(tok, ids), O.embedding(pos, pids)))
    # an id out of range is reported as by embedding; differing id shapes take the composition
    w = dev(gpu, np.ones((5, dim), f32))
    y = gpu._core._embedding_add(w, ids_dev(gpu, np.array([1, 5], np.int64)), w, ids_dev(gpu, np.array([0, 1])))
    with pytest.raises(IndexError):
        host(gpu, y)
    with pytest.raises(ValueError):
        gpu._core._embedding_add(w, ids_dev(gpu, np.array([1, 2], np.int64)), w, ids_dev(gpu, np.array([0])))


@pytest.mark.parametrize("N,V", [(6, 5), (4, 6), (16384, 65), (1000, 300)])
def test_cross_entropy_fwd_bwd(gpu, N, V):
    rng = np.random.default_rng(N + V)
    logits = (2 * rng.standard_normal((N, V))).astype(f32)
    t = rng.integers(0, V, N)
    t[::7] = -100
    tl = dev(gpu, logits, True)
    loss = gpu.cross_entropy(tl, ids_dev(gpu, t))
    assert loss.shape == []
    got = float(host(gpu, loss))
    ref = float(O.cross_entropy(logits, t))
    assert abs(got - ref) <= TOL * max(abs(ref), 1.0)
    go = np.array(1.7, f32)
    loss.backward(dev(gpu, go))
    assert_close(host(gpu, tl.grad), O.cross_entropy_backward(1.7, logits, t), TOL, "dlogits")


def test_cross_entropy_all_ignored_and_errors(gpu):
    logits = dev(gpu, np.zeros((3, 4), f32), True)
    loss = gpu.cross_entropy(logits, ids_dev(gpu, np.full(3, -100, np.int64)))
    assert float(host(gpu, loss)) == 0.0
    loss.backward()
    np.testing.assert_array_equal(host(gpu, logits.grad), np.zeros((3, 4), f32))
    bad = gpu.cross_entropy(dev(gpu, np.zeros((2, 4), f32)), ids_dev(gpu, np.array([0, 4], np.int64)))
    with pytest.raises(IndexError):
        host(gpu, bad)
    with pytest.raises(ValueError, match="targets must be Int64"):
        gpu.cross_entropy(logits, dev(gpu, np.zeros(3, f32)))


@pytest.mark.parametrize("rows,cols,offset", [(16384, 1536, 0), (300, 96, 0), (17, 4100, 0), (64, 30, 0),
                                              (100, 64, 1)])
def test_relu_bwd_colsum_matches_the_two_passes(gpu, rows, cols, offset):
    """aar_relu_bwd_colsum_f32 (the MLP backward's mask pass with db1's column
    sum) against aar_relu_bwd_f32 then aar_colsum_f32, bit for bit: the fused
    pass sums the same row chunks in the same order.  cols % 4 != 0 and an
    offset of one float take the two-pass fallback."""
    import ctypes
    from devutil import Abi
    rng = np.random.default_rng(rows + cols)
    g = rng.standard_normal((rows, cols)).astype(f32)
    x = rng.standard_normal((rows, cols)).astype(f32)
    abi = Abi()
    L = abi.L
    vp, i64, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t
    L.aar_relu_bwd_f32.argtypes = [vp, vp, vp, i64, vp]
    L.aar_colsum_workspace_bytes.restype = sz
    L.aar_colsum_workspace_bytes.argtypes = [i64, i64]
    L.aar_colsum_f32.argtypes = [vp, vp, i64, i64, vp, sz, vp]
    L.aar_relu_bwd_colsum_f32.argtypes = [vp, vp, vp, vp, i64, i64, vp, sz, vp]
    try:
        pg, px = abi.put(g, offset), abi.put(x, offset)
        wsb = L.aar_colsum_workspace_bytes(rows, cols)
        ws = abi.alloc(wsb)
        pdx, pcs = abi.empty(rows * cols, offset), abi.empty(cols)
        abi.check(L.aar_relu_bwd_f32(pg, px, pdx, rows * cols, None))
        abi.check(L.aar_colsum_f32(pdx, pcs, rows, cols, ws, wsb, None))
        pdx2, pcs2 = abi.empty(rows * cols, offset), abi.empty(cols)
        abi.check(L.aar_relu_bwd_colsum_f32(pg, px, pdx2, pcs2, rows, cols, ws, wsb, None))
        dx, cs = abi.get(pdx, (rows, cols)), abi.get(pcs, cols)
        np.testing.assert_array_equal(abi.get(pdx2, (rows, cols)).view(np.uint32), dx.view(np.uint32))
        np.testing.assert_array_equal(abi.get(pcs2, cols).view(np.uint32), cs.view(np.uint32))
        ref = np.where(x > 0, g, 0).astype(np.float64).sum(0)
        assert_close(cs, ref, TOL * np.sqrt(rows), "column sums of the masked gradient")
        assert L.aar_relu_bwd_colsum_f32(pg, px, pdx2, pcs2, rows, cols, ws, 4, None) == -2
    finally:
        abi.free()
