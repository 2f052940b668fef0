"""A linear layer's weight and bias gradients from one GEMM pass over G
(aar_gemm_f32_colsum_a, TN): C bit-identical to aar_gemm_f32 with the
workspace it asks for (the same plan, split or not), colsum bit-identical to
aar_colsum_f32 over A = G, and within the float64 bound of the exact sums.
The GPT block's shapes that take the path must take it (the MLP's two weight
gradients, split 7 ways);
the others return -3 having written nothing."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import assert_close
from devutil import Abi

pytestmark = pytest.mark.gpu
f32 = np.float32
vp, i64, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t
TN = 2


def _bind(L):
    L.aar_gemm_f32_colsum_a_workspace_bytes.restype = sz
    L.aar_gemm_f32_colsum_a_workspace_bytes.argtypes = [ctypes.c_int, i64, i64, i64]
    L.aar_gemm_f32_colsum_a.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, vp, sz, vp]
    L.aar_colsum_workspace_bytes.restype = sz
    L.aar_colsum_workspace_bytes.argtypes = [i64, i64]
    L.aar_colsum_f32.argtypes = [vp, vp, i64, i64, vp, sz, vp]


# (M, N, K, must_take): C[M, N] = A[K, M]^T B[K, N]
SHAPES = [
    (384, 1536, 16384, True),   # MLP output layer dW (7 splits)
    (1536, 384, 16384, True),   # MLP input layer dW
    (384, 384, 16384, False),   # attention out-projection dW (its plan has K groups)
    (1152, 384, 16384, False),  # qkv dW (its plan has K groups)
    (128, 256, 4096, False),
    (64, 64, 512, False),
    (96, 100, 1024, False),
]


@pytest.mark.parametrize("M,N,K,must", SHAPES)
def test_colsum_gemm_matches_product_and_colsum(gpu, M, N, K, must):
    rng = np.random.default_rng(M + 3 * N + 7 * K)
    a = rng.standard_normal((K, M)).astype(f32)
    b = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(f32)
    abi = Abi()
    L = abi.L
    _bind(L)
    try:
        pa, pb = abi.put(a), abi.put(b)
        wsb = L.aar_gemm_f32_workspace_bytes(TN, M, N, K)
        pc_ref = abi.empty(M * N)
        abi.check(L.aar_gemm_f32(TN, M, N, K, pa, pb, pc_ref, abi.alloc(wsb) if wsb else None, wsb, None))
        csb = L.aar_colsum_workspace_bytes(K, M)
        pcs_ref = abi.empty(M)
        abi.check(L.aar_colsum_f32(pa, pcs_ref, K, M, abi.alloc(csb), csb, None))
        c_ref, cs_ref = abi.get(pc_ref, (M, N)), abi.get(pcs_ref, (M,))

        wc = L.aar_gemm_f32_colsum_a_workspace_bytes(TN, M, N, K)
        assert wc >= K // 64 * M * 4
        pc, pcs = abi.put(np.full((M, N), 7.0, f32)), abi.put(np.full(M, 7.0, f32))
        rc = L.aar_gemm_f32_colsum_a(TN, M, N, K, pa, pb, pc, pcs, abi.alloc(wc), wc, None)
        assert rc in (0, -3), rc
        if rc == -3:
            assert not must, "this shape must take the fused path"
            assert (abi.get(pc, (M, N)) == 7.0).all() and (abi.get(pcs, (M,)) == 7.0).all()
            return
        np.testing.assert_array_equal(abi.get(pc, (M, N)), c_ref)
        np.testing.assert_array_equal(abi.get(pcs, (M,)), cs_ref)
        exact = a.astype(np.float64).sum(0)
        assert_close(cs_ref, exact, 1e-6 * np.sqrt(K) * (np.abs(a).sum(0).max() + 1), "colsum vs float64")
    finally:
        abi.free()


def test_colsum_gemm_refusals(gpu):
    """Other layouts, contractions that are not whole 64-row colsum chunks
    (or more than 256 of them) and a too-small workspace are refused before
    any launch."""
    abi = Abi()
    L = abi.L
    _bind(L)
    try:
        M, N = 128, 128
        pa, pb = abi.put(np.ones((16448, M), f32)), abi.put(np.ones((16448, N), f32))
        pc, pcs = abi.put(np.full((M, N), 7.0, f32)), abi.put(np.full(M, 7.0, f32))
        wc = L.aar_gemm_f32_colsum_a_workspace_bytes(TN, M, N, 16448)
        ws = abi.alloc(wc)
        for K in (1000, 16448):
            assert L.aar_gemm_f32_colsum_a(TN, M, N, K, pa, pb, pc, pcs, ws, wc, None) == -3
        for op in (0, 1):
            assert L.aar_gemm_f32_colsum_a(op, M, N, 4096, pa, pb, pc, pcs, ws, wc, None) == -3
        assert L.aar_gemm_f32_colsum_a(TN, M, N, 4096, pa, pb, pc, pcs, ws, 16, None) == -2
        assert (abi.get(pc, (M, N)) == 7.0).all() and (abi.get(pcs, (M,)) == 7.0).all()
    finally:
        abi.free()
