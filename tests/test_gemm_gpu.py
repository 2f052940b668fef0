"""GEMM parity on the GPU: matmul / matmul_a_bt / matmul_at_b through
aargrad._core (and the C ABI directly for alignment and workspace cases),
against the oracle at sizes it finishes in seconds and against float64
closed forms on sampled rows plus full-size checksums at the BASELINE sweep.
Tolerance: 1e-4*sqrt(K) for both error metrics (conftest.errs)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle as O
from conftest import assert_close, gemm_tol
from devutil import Abi, dev, host

pytestmark = pytest.mark.gpu
f32 = np.float32
OPFN = {"nn": "matmul", "nt": "matmul_a_bt", "tn": "matmul_at_b"}


def operands(op, M, N, K, rng, scale=1.0):
    a = (rng.standard_normal((M, K) if op != "tn" else (K, M)) * scale).astype(f32)
    b = (rng.standard_normal((K, N) if op != "nt" else (N, K)) * scale).astype(f32)
    return a, b


def logical(op, a, b):
    A = a.astype(np.float64) if op != "tn" else a.T.astype(np.float64)
    B = b.astype(np.float64) if op != "nt" else b.T.astype(np.float64)
    return A, B


@pytest.mark.parametrize("op", ["nn", "nt", "tn"])
def test_kat_on_device(gpu, op):
    # tests/cpp/test_matmul.cpp:21-36, :58-88, :96-117
    a = {"nn": [[1, 2, 3], [4, 5, 6]], "nt": [[1, 2, 3], [4, 5, 6]], "tn": [[1, 4], [2, 5], [3, 6]]}[op]
    b = {"nn": [[7, 8], [9, 10], [11, 12]], "nt": [[7, 9, 11], [8, 10, 12]],
         "tn": [[7, 8], [9, 10], [11, 12]]}[op]
    c = getattr(gpu, OPFN[op])(dev(gpu, np.array(a, f32)), dev(gpu, np.array(b, f32)))
    np.testing.assert_array_equal(host(gpu, c), [[58, 64], [139, 154]])


@pytest.mark.parametrize("op", ["nn", "nt", "tn"])
def test_golden_fill_64x96x48(gpu, op):
    # tests/cpp/test_matmul.cpp:119-140 fill; outputs from the reference CPU build
    z = np.load(O.HERE.parent / "tests" / "golden" / "gemm_64x96x48.npz")
    c = host(gpu, getattr(gpu, OPFN[op])(dev(gpu, z[f"{op}_a"]), dev(gpu, z[f"{op}_b"])))
    ref = z[f"{op}_c"]
    tol = 1e-5 * np.maximum(np.abs(ref), 1.0) + 1e-6  # the reference test's own bound
    assert np.all(np.abs(c - ref) <= tol)


@pytest.mark.parametrize("op", ["nn", "nt", "tn"])
def test_config1_1024_vs_oracle(gpu, op):
    # M=N=K=1024, A then B ~ N(0,1) from seed 0, forward only
    rng = np.random.default_rng(0)
    a, b = operands(op, 1024, 1024, 1024, rng)
    c = host(gpu, getattr(gpu, OPFN[op])(dev(gpu, a), dev(gpu, b)))
    assert_close(c, O.matmul(op, a, b), gemm_tol(1024), f"{op} 1024^3")


SWEEP = [(2048, 2048, 2048), (4096, 4096, 4096), (8192, 8192, 8192), (16384, 1536, 384), (16384, 384, 1536)]


# The reference bench's shapes beyond the BASELINE sweep (bench/bench_matmul.cu:
# 150-167): sq256, sq512, qkv_proj, vocab_head, big_ffn, tall, wide, tiny_M.
REF_BENCH = [(256, 256, 256), (512, 512, 512), (16384, 1152, 384), (16384, 65, 384), (8192, 4096, 1024),
             (16384, 256, 256), (256, 16384, 256), (128, 4096, 4096)]


@pytest.mark.parametrize("shape", SWEEP, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("op", ["nn", "nt", "tn"])
def test_config2_sweep_fwd_bwd(gpu, op, shape):
    """Forward plus both input-gradient GEMMs (through the autograd Functions)
    at the BASELINE sweep sizes.  Sampled output rows are compared with float64
    closed forms; every column is checked through the column-sum identity
    1^T (A B) = (1^T A) B, a size-independent checksum."""
    _fwd_bwd_sampled(gpu, op, shape)


@pytest.mark.parametrize("shape", REF_BENCH, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("op", ["nn", "nt", "tn"])
def test_reference_bench_shapes_fwd_bwd(gpu, op, shape):
    """The same checks at the reference bench's other shapes."""
    _fwd_bwd_sampled(gpu, op, shape)


@pytest.mark.parametrize("shape", REF_BENCH + [(1024, 1024, 1024), (4096, 4096, 4096), (16384, 384, 1536)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("op", ["nn", "nt", "tn"])
def test_reference_bench_inputs(gpu, op, shape):
    """The reference bench's inputs (A, B uniform in [0, 1), so every output
    is a sum of K positive terms near K/4) and its acceptance test: max abs
    error against an exact product within max(2e-3, 5e-3*sqrt(K)/32)
    (bench/bench_matmul.cu:97-99, :238-242), here against float64 on sampled
    rows, plus this build's 1e-4*sqrt(K) bound and the column-sum checksum."""
    M, N, K = shape
    rng = np.random.default_rng(M * 3 + N * 5 + K * 7 + ord(op[1]))
    a = rng.random((M, K) if op != "tn" else (K, M), dtype=f32)
    b = rng.random((K, N) if op != "nt" else (N, K), dtype=f32)
    c = host(gpu, getattr(gpu, OPFN[op])(dev(gpu, a), dev(gpu, b)))
    A, B = logical(op, a, b)
    rows = np.sort(rng.choice(M, min(M, 32), replace=False))
    ref = A[rows] @ B
    assert np.abs(c[rows] - ref).max() <= max(2e-3, 5e-3 * np.sqrt(K) / 32.0)
    assert_close(c[rows], ref, gemm_tol(K), f"{op} {shape} rows")
    assert_close(c.astype(np.float64).sum(0), A.sum(0) @ B, gemm_tol(K) * np.sqrt(M), f"{op} {shape} colsum")


def _fwd_bwd_sampled(gpu, op, shape):
    M, N, K = shape
    rng = np.random.default_rng(hash(shape) % 2**32 + ord(op[0]))
    a, b = operands(op, M, N, K, rng, 1.0 / np.sqrt(K))
    g = rng.standard_normal((M, N)).astype(f32)
    ta, tb = dev(gpu, a, True), dev(gpu, b, True)
    c = getattr(gpu, OPFN[op])(ta, tb)
    c.backward(dev(gpu, g))
    ch, da, db = host(gpu, c), host(gpu, ta.grad), host(gpu, tb.grad)
    A, B = logical(op, a, b)
    G = g.astype(np.float64)
    rows = np.sort(rng.choice(M, min(M, 48), replace=False))
    assert_close(ch[rows], A[rows] @ B, gemm_tol(K), f"{op} fwd rows")
    assert_close(ch.astype(np.float64).sum(0), A.sum(0) @ B, gemm_tol(K) * np.sqrt(M), f"{op} fwd colsum")
    # logical gradients: dA = G B^T (contraction N), dB = A^T G (contraction M)
    dA_rows = G[rows] @ B.T
    brow = np.sort(rng.choice(K, min(K, 48), replace=False))
    dB_rows = A[:, brow].T @ G
    dA_log = da if op != "tn" else da.T  # tn: a is A^T
    dB_log = db if op != "nt" else db.T  # nt: b is B^T
    assert_close(dA_log[rows], dA_rows, gemm_tol(N), f"{op} dA rows")
    assert_close(dB_log[brow], dB_rows, gemm_tol(M), f"{op} dB rows")


@pytest.mark.parametrize("op", ["nn", "nt", "tn"])
@pytest.mark.parametrize("shape", [(1, 1, 1), (1, 257, 3), (333, 65, 129), (65, 16384, 384),
                                   (384, 384, 16384), (17, 5, 1), (128, 128, 8)])
def test_edge_shapes_vs_oracle(gpu, op, shape):
    M, N, K = shape
    rng = np.random.default_rng(M + 7 * N + 13 * K)
    a, b = operands(op, M, N, K, rng)
    c = host(gpu, getattr(gpu, OPFN[op])(dev(gpu, a), dev(gpu, b)))
    if M * N * K <= 2**28:
        assert_close(c, O.matmul(op, a, b), gemm_tol(K), f"{op} {shape}")
    else:
        r = np.sort(rng.choice(M, 16, replace=False))
        A, B = logical(op, a, b)
        assert_close(c[r], A[r] @ B, gemm_tol(K), f"{op} {shape}")


def test_zero_contraction_writes_zeros(gpu):
    abi = Abi()
    try:
        c = abi.put(np.full((4, 5), 7.0, f32))
        abi.check(abi.L.aar_gemm_f32(0, 4, 5, 0, abi.alloc(16), abi.alloc(16), c, None, 0, None))
        np.testing.assert_array_equal(abi.get(c, (4, 5)), np.zeros((4, 5), f32))
    finally:
        abi.free()


@pytest.mark.parametrize("op", [0, 1, 2])
def test_abi_misaligned_and_no_workspace(gpu, op):
    """Pointers offset by one float take the scalar-load path; a missing
    workspace disables split-K.  Both must give the same parity."""
    M, N, K = 260, 132, 2052
    rng = np.random.default_rng(5 + op)
    name = ["nn", "nt", "tn"][op]
    a, b = operands(name, M, N, K, rng)
    ref = O.matmul(name, a, b)
    abi = Abi()
    try:
        pa, pb, pc = abi.put(a, 1), abi.put(b, 1), abi.empty(M * N, 1)
        abi.check(abi.L.aar_gemm_f32(op, M, N, K, pa, pb, pc, None, 0, None))
        assert_close(abi.get(pc, (M, N)), ref, gemm_tol(K), "misaligned")
        pa, pb, pc = abi.put(a), abi.put(b), abi.empty(M * N)
        wsb = abi.L.aar_gemm_f32_workspace_bytes(op, M, N, K)
        ws = abi.alloc(wsb) if wsb else None
        abi.check(abi.L.aar_gemm_f32(op, M, N, K, pa, pb, pc, ws, wsb, None))
        assert_close(abi.get(pc, (M, N)), ref, gemm_tol(K), "aligned")
    finally:
        abi.free()


def test_split_k_is_deterministic(gpu):
    rng = np.random.default_rng(11)
    a = rng.standard_normal((16384, 384)).astype(f32)
    g = rng.standard_normal((16384, 1152)).astype(f32)
    ta, tg = dev(gpu, a), dev(gpu, g)
    r1 = host(gpu, gpu.matmul_at_b(tg, ta))
    r2 = host(gpu, gpu.matmul_at_b(tg, ta))
    np.testing.assert_array_equal(r1, r2)
    rows = np.arange(0, 1152, 97)
    assert_close(r1[rows], g.astype(np.float64)[:, rows].T @ a.astype(np.float64), gemm_tol(16384), "dW")


def test_leading_dims_are_flattened(gpu):
    # matmul / matmul_a_bt accept rank>=2 LHS (cppsrc/ops/matmul.cpp:93-120)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 7, 24)).astype(f32)
    w = rng.standard_normal((24, 10)).astype(f32)
    y = gpu.matmul(dev(gpu, x), dev(gpu, w))
    assert y.shape == [4, 7, 10]
    assert_close(host(gpu, y), x.astype(np.float64) @ w, gemm_tol(24), "3-D matmul")
    wt = np.ascontiguousarray(w.T)
    y2 = gpu.matmul_a_bt(dev(gpu, x), dev(gpu, wt))
    assert_close(host(gpu, y2), x.astype(np.float64) @ w, gemm_tol(24), "3-D matmul_a_bt")


def test_linear_layer_grads_match_oracle(gpu):
    """nn.Linear's forward is matmul_a_bt; its backward runs matmul (dX) and
    matmul_at_b with 3-D operands flattened (dW) (cppsrc/ops/matmul.cpp:146-155)."""
    rng = np.random.default_rng(8)
    x = rng.standard_normal((2, 96, 64)).astype(f32)
    w = (0.1 * rng.standard_normal((48, 64))).astype(f32)
    g = rng.standard_normal((2, 96, 48)).astype(f32)
    tx, tw = dev(gpu, x, True), dev(gpu, w, True)
    y = gpu.matmul_a_bt(tx, tw)
    y.backward(dev(gpu, g))
    x2, g2 = x.reshape(-1, 64), g.reshape(-1, 48)
    assert_close(host(gpu, y).reshape(-1, 48), O.matmul("nt", x2, w), gemm_tol(64), "y")
    assert_close(host(gpu, tx.grad).reshape(-1, 64), O.matmul("nn", g2, w), gemm_tol(48), "dx")
    assert_close(host(gpu, tw.grad), O.matmul("tn", g2, x2), gemm_tol(192), "dw")


def gemm_configs(abi):
    out, c = [], 0
    m, n, k = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    while abi.L.aar_gemm_f32_tile_config(c, ctypes.byref(m), ctypes.byref(n), ctypes.byref(k)) == 0:
        out.append((c, m.value, n.value, k.value))
        c += 1
    return out


@pytest.mark.parametrize("op", [0, 1, 2])
def test_every_tile_config_vs_oracle(gpu, op):
    """Each tile configuration, forced through aar_gemm_f32_with_config, on
    ragged shapes: partial M/N tiles, a K tail shorter than the tile depth,
    the 128-bit path (aligned, extents % 4 == 0) and the predicated path
    (odd extents), with and without a forced split-K."""
    name = ["nn", "nt", "tn"][op]
    abi = Abi()
    try:
        cfgs = gemm_configs(abi)
        assert len(cfgs) >= 3
        for (M, N, K) in [(300, 260, 200), (77, 93, 45)]:
            rng = np.random.default_rng(M + N + K + op)
            a, b = operands(name, M, N, K, rng)
            ref = O.matmul(name, a, b)
            pa, pb = abi.put(a), abi.put(b)
            ws = abi.alloc(4 * 4 * M * N)
            vec = M % 4 == 0 and N % 4 == 0 and K % 4 == 0
            for (cfg, bm, bn, bk) in cfgs:
                # the 128-bit path stages a row-contiguous operand (A of TN, B of NN and TN)
                # with a layout that needs the tile extent to be a multiple of 64
                no_dma = vec and ((op == 2 and bm % 64) or (op in (0, 2) and bn % 64))
                for splits in (1, 3):
                    pc = abi.empty(M * N)
                    rc = abi.L.aar_gemm_f32_with_config(op, M, N, K, pa, pb, pc, ws, 16 * M * N, cfg, splits, None)
                    if no_dma:
                        assert rc == -3, (cfg, op, rc)
                        continue
                    abi.check(rc)
                    assert_close(abi.get(pc, (M, N)), ref, gemm_tol(K), f"{name} cfg {cfg} ({bm}x{bn}x{bk}) "
                                 f"splits {splits} shape {(M, N, K)}")
    finally:
        abi.free()



@pytest.mark.parametrize("op", [0, 1, 2])
def test_thin_output_kernel_vs_oracle(gpu, op):
    """The thin-output kernel (configuration id = the number of tile
    configurations), forced through aar_gemm_f32_with_config: N up to 128 in
    1..8 column blocks of 16 with ragged N and M (a last block of 1-4 columns
    goes through VALU FMAs), K a multiple of 16 up to 512
    (4 K parts per row slab, some of them empty), misaligned A (NN/NT), B
    rows that are not 16-byte aligned (N odd), B staged whole (flat) or row by
    row (padded).  A rerun is bit identical (fixed-order part sum); shapes
    outside its limits return AAR_EUNSUPPORTED; the plan takes it for the
    vocabulary head 16384 x 65 x 384 in all three layouts."""
    name = ["nn", "nt", "tn"][op]
    abi = Abi()
    try:
        thin = len(gemm_configs(abi))
        # N % 16 in 1..4 (65, 17, 33, 50, 20) takes the VALU tail-column form
        for (M, N, K) in [(300, 65, 384), (1000, 1, 16), (777, 128, 64), (64, 17, 512), (130, 96, 336),
                          (4097, 33, 48), (65, 80, 400), (16, 16, 32), (257, 50, 64), (300, 20, 128)]:
            if op == 1 and 16 * -(-N // 16) * 64 * -(-K // 64) > 32768:
                continue  # B^T in 64-deep chunks does not fit the kernel's LDS (checked below)
            if op != 1 and K * (16 * -(-N // 16) + 4) > 32768:
                continue
            rng = np.random.default_rng(M * 7 + N + K + op)
            a, b = operands(name, M, N, K, rng)
            ref = O.matmul(name, a, b)
            pa, pb = abi.put(a), abi.put(b)
            outs = []
            for _ in range(2):
                pc = abi.empty(M * N)
                abi.check(abi.L.aar_gemm_f32_with_config(op, M, N, K, pa, pb, pc, None, 0, thin, 1, None))
                outs.append(abi.get(pc, (M, N)))
            np.testing.assert_array_equal(outs[0], outs[1])
            assert_close(outs[0], ref, gemm_tol(K), f"{name} thin {(M, N, K)}")
        p = abi.alloc(4 << 20)
        for (M, N, K) in [(256, 129, 64), (256, 64, 100), (256, 64, 528), (256, 64, 8)]:
            assert abi.L.aar_gemm_f32_with_config(op, M, N, K, p, p, p, None, 0, thin, 1, None) == -3, (M, N, K)
        if op == 1:  # B^T as 128 columns x 5 chunks of 64 k exceeds the 128 KB of LDS
            assert abi.L.aar_gemm_f32_with_config(op, 256, 128, 272, p, p, p, None, 0, thin, 1, None) == -3
            # K = 256 fills it exactly
            rng = np.random.default_rng(9)
            a, b = operands(name, 256, 128, 256, rng)
            pa, pb, pc = abi.put(a), abi.put(b), abi.empty(256 * 128)
            abi.check(abi.L.aar_gemm_f32_with_config(op, 256, 128, 256, pa, pb, pc, None, 0, thin, 1, None))
            assert_close(abi.get(pc, (256, 128)), O.matmul(name, a, b), gemm_tol(256), "nt thin full LDS")
        if op != 2:  # 128-bit A rows need a 16-byte aligned A
            assert abi.L.aar_gemm_f32_with_config(op, 64, 65, 64, p + 4, p, p, None, 0, thin, 1, None) == -3
        assert abi.L.aar_gemm_f32_with_config(op, 64, 65, 64, p, p, p, None, 0, thin, 2, None) == -1
        cfg, sp = ctypes.c_int(-1), ctypes.c_int(-1)
        abi.check(abi.L.aar_gemm_f32_plan(op, 16384, 65, 384, 1 << 30, ctypes.byref(cfg), ctypes.byref(sp)))
        assert (cfg.value, sp.value) == (thin, 1)
        # NN/TN copy a contiguous, 16-byte aligned B into LDS whole (flat form); a B
        # one float off that alignment takes the padded row-by-row form
        if op != 1:
            for (M, N, K) in [(300, 65, 384), (130, 40, 96)]:
                rng = np.random.default_rng(M + N + K + 100 * op)
                a, b = operands(name, M, N, K, rng)
                pa, pb, pc = abi.put(a), abi.put(b, offset_floats=1), abi.empty(M * N)
                abi.check(abi.L.aar_gemm_f32_with_config(op, M, N, K, pa, pb, pc, None, 0, thin, 1, None))
                assert_close(abi.get(pc, (M, N)), O.matmul(name, a, b), gemm_tol(K), f"{name} thin padded B {(M, N, K)}")
        # At the vocabulary head's shape the plan (shape-only, aligned operands)
        # is the thin kernel; through aar_gemm_f32 an A one float off 16-byte
        # alignment, which the thin kernel's 128-bit A loads cannot take for
        # NN/NT, must fall back to a tile configuration and still match.
        if op != 2:
            rng = np.random.default_rng(5)
            M, N, K = 16384, 65, 384
            a, b = operands(name, M, N, K, rng)
            pa, pb, pc = abi.put(a, offset_floats=1), abi.put(b), abi.empty(M * N)
            abi.check(abi.L.aar_gemm_f32(op, M, N, K, pa, pb, pc, None, 0, None))
            assert_close(abi.get(pc, (M, N)), O.matmul(name, a, b), gemm_tol(K), f"{name} misaligned A at the head shape")
    finally:
        abi.free()


def test_plan_and_config_errors(gpu):
    abi = Abi()
    try:
        cfg, sp = ctypes.c_int(-1), ctypes.c_int(-1)
        abi.check(abi.L.aar_gemm_f32_plan(0, 4096, 4096, 4096, 0, ctypes.byref(cfg), ctypes.byref(sp)))
        assert cfg.value >= 0 and sp.value == 1
        n = len(gemm_configs(abi))
        p = abi.alloc(4096)
        # id n is the thin-output kernel (K = 8 is below its 16-deep k blocks); n + 1
        # the short-operand kernels (NN and TN only, NN unsplit); n + 2 is invalid
        assert abi.L.aar_gemm_f32_with_config(0, 8, 8, 8, p, p, p, None, 0, n, 1, None) == -3  # EUNSUPPORTED
        assert abi.L.aar_gemm_f32_with_config(1, 8, 8, 8, p, p, p, None, 0, n + 1, 1, None) == -3
        assert abi.L.aar_gemm_f32_with_config(0, 8, 8, 8, p, p, p, None, 0, n + 1, 2, None) == -1
        assert abi.L.aar_gemm_f32_with_config(0, 8, 8, 8, p, p, p, None, 0, n + 2, 1, None) == -1  # EINVAL
        assert abi.L.aar_gemm_f32_with_config(0, 8, 8, 8, p, p, p, None, 0, 0, 0, None) == -1
        # a forced split needs workspace
        assert abi.L.aar_gemm_f32_with_config(0, 64, 64, 4096, p, p, p, None, 0, 0, 4, None) == -2
    finally:
        abi.free()


def test_short_operand_kernels_vs_oracle(gpu):
    """The short-operand kernels (configuration id = tile configurations + 1):
    TN with at most 260 output rows split over K, NN with a contraction of at
    most 128, for operands whose rows are not 16-byte aligned (a vocabulary of
    65).  TN: MFMA over an even number of 32-row blocks plus up to 4 rows by
    VALU (65, 68, 130 rows) or padded blocks (1, 3, 100; past 6 blocks, and
    a misaligned A past 2, are refused and the plan falls back), N
    ragged against the 64-column workgroup tile, K ragged against the 32-row
    k tile, forced split counts 1, 3 and 17 and the planned one, A one float
    off 16-byte alignment (4-byte DMAs).  NN: K below one 8-step MFMA chunk
    (1, 7), K % 8 steps by VALU (65, 127), misaligned A.  Reruns are bit
    identical; the plan takes this kernel for the GPT head's TN and NN
    products, and aar_gemm_f32 runs them through it."""
    abi = Abi()
    try:
        short = len(gemm_configs(abi)) + 1
        tn_shapes = [(65, 384, 16384), (65, 388, 4099), (1, 4, 1024), (3, 64, 1000), (100, 100, 2048),
                     (68, 100, 2048), (130, 128, 1500), (200, 388, 1111), (257, 64, 3000), (260, 68, 777)]
        # (with_config is given pa as C where it must refuse before any launch)
        for (M, N, K) in tn_shapes:
            rng = np.random.default_rng(M + N + K)
            a, b = operands("tn", M, N, K, rng)
            ref = O.matmul("tn", a, b)
            for off in ((0, 1) if M in (65, 130, 257) else (0,)):
                pa, pb = abi.put(a, offset_floats=off), abi.put(b)
                ws_bytes = 64 * M * N * 4 + 4096
                ws = abi.alloc(ws_bytes)
                # more than 6 row blocks of a dense A do not fit two LDS stages,
                # and a misaligned A past 2 blocks needs more 4-byte DMAs than
                # one vmcnt counts: refused, and the plan falls back to the
                # tiled kernels
                supported = M <= 196 and (off == 0 or M <= 68)
                if not supported:
                    assert abi.L.aar_gemm_f32_with_config(2, M, N, K, pa, pb, pa, ws, ws_bytes, short, 3, None) == -3
                for splits in ((1, 3, 17) if supported else ()):
                    outs = []
                    for _ in range(2):
                        pc = abi.empty(M * N)
                        abi.check(abi.L.aar_gemm_f32_with_config(2, M, N, K, pa, pb, pc, ws, ws_bytes, short, splits,
                                                                 None))
                        outs.append(abi.get(pc, (M, N)))
                    np.testing.assert_array_equal(outs[0], outs[1])
                    assert_close(outs[0], ref, gemm_tol(K), f"tn short {(M, N, K)} splits {splits} off {off}")
                pc = abi.empty(M * N)
                abi.check(abi.L.aar_gemm_f32(2, M, N, K, pa, pb, pc, ws, ws_bytes, None))
                assert_close(abi.get(pc, (M, N)), ref, gemm_tol(K), f"tn planned {(M, N, K)} off {off}")
        for (M, N, K) in [(16384, 384, 65), (1000, 388, 7), (300, 100, 127), (77, 4, 1), (129, 260, 72)]:
            rng = np.random.default_rng(M + N + K + 1)
            a, b = operands("nn", M, N, K, rng)
            ref = O.matmul("nn", a, b)
            for off in (0, 1):
                pa, pb = abi.put(a, offset_floats=off), abi.put(b)
                outs = []
                for _ in range(2):
                    pc = abi.empty(M * N)
                    abi.check(abi.L.aar_gemm_f32_with_config(0, M, N, K, pa, pb, pc, None, 0, short, 1, None))
                    outs.append(abi.get(pc, (M, N)))
                np.testing.assert_array_equal(outs[0], outs[1])
                assert_close(outs[0], ref, gemm_tol(K), f"nn short {(M, N, K)} off {off}")
                pc = abi.empty(M * N)
                abi.check(abi.L.aar_gemm_f32(0, M, N, K, pa, pb, pc, None, 0, None))
                assert_close(abi.get(pc, (M, N)), ref, gemm_tol(K), f"nn planned {(M, N, K)} off {off}")
        cfg, sp = ctypes.c_int(-1), ctypes.c_int(-1)
        for op, (M, N, K) in ((2, (65, 384, 16384)), (0, (16384, 384, 65))):
            ws = abi.L.aar_gemm_f32_workspace_bytes(op, M, N, K)
            abi.check(abi.L.aar_gemm_f32_plan(op, M, N, K, ws, ctypes.byref(cfg), ctypes.byref(sp)))
            assert cfg.value == short, (op, M, N, K, cfg.value)
            assert sp.value >= (2 if op == 2 else 1)
            assert ws >= (sp.value * M * N * 4 if sp.value > 1 else 0)
        p = abi.alloc(4096)
        assert abi.L.aar_gemm_f32_with_config(2, 261, 64, 1024, p, p, p, None, 0, short, 1, None) == -3  # M > 260
        assert abi.L.aar_gemm_f32_with_config(0, 64, 64, 129, p, p, p, None, 0, short, 1, None) == -3  # K > 128
        assert abi.L.aar_gemm_f32_with_config(2, 65, 64, 4096, p, p, p, None, 0, short, 4, None) == -2  # workspace
    finally:
        abi.free()
