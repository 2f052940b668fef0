"""The MLP's relu carried as a bit mask between its GEMMs, through the C ABI:

* aar_gemm_f32_bias_relu_bits (NT): C bit-identical to aar_gemm_f32_bias_relu
  and the bits equal to C > 0 packed 32 rows a word (bit r % 32 of word
  (r / 32) * N + c, zero past M);
* aar_gemm_f32_mask_bits_colsum (NN): C bit-identical to aar_gemm_f32 then
  aar_relu_bwd_f32 against the forward's C, with column sums requested and
  without; and colsum bit-identical to aar_colsum_f32 of that C (its 64-row
  chunk partials come from the GEMM epilogue), and within the float64 bound
  of the exact column sums.

The GPT block's MLP shape (16384 rows, 384 -> 1536 -> 384) must take both
entry points; other shapes either take them (and are checked the same way) or
return -3 having written nothing.  The mask entry point also refuses row
counts whose colsum partials are not 64-row chunks."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import assert_close
from devutil import Abi

pytestmark = pytest.mark.gpu
f32 = np.float32
vp, i64, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t
NN, NT = 0, 1
SENTINEL = 0x5A5A5A5A


def _bind(L):
    L.aar_gemm_f32_bias_relu.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, vp, sz, vp]
    L.aar_gemm_f32_bias_relu_bits.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, vp, vp, sz, vp]
    L.aar_gemm_f32_mask_bits_colsum_workspace_bytes.restype = sz
    L.aar_gemm_f32_mask_bits_colsum_workspace_bytes.argtypes = [i64, i64]
    L.aar_gemm_f32_mask_bits_colsum.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, vp, vp, sz, vp]
    L.aar_relu_bwd_f32.argtypes = [vp, vp, vp, i64, vp]
    L.aar_colsum_workspace_bytes.restype = sz
    L.aar_colsum_workspace_bytes.argtypes = [i64, i64]
    L.aar_colsum_f32.argtypes = [vp, vp, i64, i64, vp, sz, vp]


def _pack(c):
    """bits[rb][col] bit b = c[32 rb + b][col] > 0 (zero past the last row)."""
    M, N = c.shape
    nb = (M + 31) // 32
    pos = np.zeros((nb * 32, N), bool)
    pos[:M] = c > 0
    pos = np.ascontiguousarray(pos.reshape(nb, 32, N).transpose(0, 2, 1))
    return np.packbits(pos, axis=2, bitorder="little").view("<u4").reshape(nb, N)


def _words(abi, p, shape):
    raw = abi.get(p, shape)
    return raw.view(np.uint32)


def _sentinel_words(abi, rows, cols):
    arr = np.full((rows, cols), SENTINEL, np.uint32).view(f32)
    return abi.put(arr)


# (M rows, H hidden, d in, N2 out): forward C[M,H] = X[M,d] W1[H,d]^T + b1,
# backward dh[M,H] = G[M,N2] W2[N2,H]
SHAPES = [
    (16384, 1536, 384, 384),  # GPT block (must be fused)
    (4096, 1536, 384, 384),
    (4004, 1536, 384, 384),   # forward on the 32-row wave tiles of configuration 16, a 4-row last word
    (2048, 960, 384, 128),
    (1000, 200, 64, 96),      # M not a multiple of 32: a partial last word (forward only)
    (1024, 200, 64, 96),      # N not a multiple of the tile width
    (512, 96, 64, 33),
    (128, 1536, 384, 384),
]


@pytest.mark.parametrize("M,H,d,N2", SHAPES)
def test_bits_forward_and_masked_backward(gpu, M, H, d, N2):
    rng = np.random.default_rng(M + 7 * H + 13 * d + N2)
    x = rng.standard_normal((M, d)).astype(f32)
    w1 = (rng.standard_normal((H, d)) / np.sqrt(d)).astype(f32)
    b1 = (0.1 * rng.standard_normal(H)).astype(f32)
    g = rng.standard_normal((M, N2)).astype(f32)
    w2 = (rng.standard_normal((N2, H)) / np.sqrt(N2)).astype(f32)
    nb = (M + 31) // 32
    abi = Abi()
    L = abi.L
    _bind(L)
    try:
        px, pw1, pb1, pg, pw2 = (abi.put(a) for a in (x, w1, b1, g, w2))
        wsf = L.aar_gemm_f32_workspace_bytes(NT, M, H, d)
        wf = abi.alloc(wsf) if wsf else None
        # forward: the plain bias + relu product, then the bits entry point
        ph_ref, ph = abi.empty(M * H), abi.put(np.full((M, H), 7.0, f32))
        pbits = _sentinel_words(abi, nb, H)
        abi.check(L.aar_gemm_f32_bias_relu(NT, M, H, d, px, pw1, pb1, ph_ref, wf, wsf, None))
        rc = L.aar_gemm_f32_bias_relu_bits(NT, M, H, d, px, pw1, pb1, ph, pbits, wf, wsf, None)
        assert rc in (0, -3), rc
        h_ref = abi.get(ph_ref, (M, H))
        assert 0.2 < np.mean(h_ref > 0) < 0.8  # both signs
        if rc == -3:
            assert M != 16384, "the GPT block shape must take the bits epilogue"
            assert (abi.get(ph, (M, H)) == 7.0).all()
            assert (_words(abi, pbits, (nb, H)) == SENTINEL).all()
            bits = _pack(h_ref)
            pbits = abi.put(bits.view(f32))
        else:
            np.testing.assert_array_equal(abi.get(ph, (M, H)), h_ref)
            bits = _words(abi, pbits, (nb, H))
            np.testing.assert_array_equal(bits, _pack(h_ref))

        # backward: the plain product, relu backward against h, colsum
        wsb = L.aar_gemm_f32_workspace_bytes(NN, M, H, N2)
        wb = abi.alloc(wsb) if wsb else None
        pp, pdh_ref = abi.empty(M * H), abi.empty(M * H)
        abi.check(L.aar_gemm_f32(NN, M, H, N2, pg, pw2, pp, wb, wsb, None))
        abi.check(L.aar_relu_bwd_f32(pp, ph_ref, pdh_ref, M * H, None))
        csb = L.aar_colsum_workspace_bytes(M, H)
        pcs_ref = abi.empty(H)
        abi.check(L.aar_colsum_f32(pdh_ref, pcs_ref, M, H, abi.alloc(csb), csb, None))
        dh_ref, cs_ref = abi.get(pdh_ref, (M, H)), abi.get(pcs_ref, (H,))

        # the mask only (no column sums, no workspace, any row count)
        pdh = abi.put(np.full((M, H), 7.0, f32))
        rc = L.aar_gemm_f32_mask_bits_colsum(NN, M, H, N2, pg, pw2, pbits, pdh, None, None, 0, None)
        assert rc in (0, -3), rc
        if rc == 0:
            np.testing.assert_array_equal(abi.get(pdh, (M, H)), dh_ref)
        else:
            assert M != 16384, "the GPT block shape must take the mask-bits epilogue"
            assert (abi.get(pdh, (M, H)) == 7.0).all()

        pdh, pcs = abi.put(np.full((M, H), 7.0, f32)), abi.put(np.full(H, 7.0, f32))
        wm = L.aar_gemm_f32_mask_bits_colsum_workspace_bytes(M, H)
        assert wm == (M + 63) // 64 * H * 4
        rc = L.aar_gemm_f32_mask_bits_colsum(NN, M, H, N2, pg, pw2, pbits, pdh, pcs, abi.alloc(wm), wm, None)
        assert rc in (0, -3), rc
        if rc == -3:
            assert M != 16384, "the GPT block shape must take the mask-bits epilogue"
            assert (abi.get(pdh, (M, H)) == 7.0).all() and (abi.get(pcs, (H,)) == 7.0).all()
            return
        np.testing.assert_array_equal(abi.get(pdh, (M, H)), dh_ref)
        np.testing.assert_array_equal(abi.get(pcs, (H,)), cs_ref)
        exact = dh_ref.astype(np.float64).sum(0)
        assert_close(cs_ref, exact, 1e-6 * np.sqrt(M) * (np.abs(dh_ref).sum(0).max() + 1), "colsum vs float64")
    finally:
        abi.free()


def test_mask_bits_refusals(gpu):
    """Row counts whose colsum partials are not 64-row chunks, the NT layout
    and a too-small workspace are refused before any launch; zero rows give
    zero column sums."""
    abi = Abi()
    L = abi.L
    _bind(L)
    try:
        H, N2 = 192, 64
        pg, pw2 = abi.put(np.ones((16448, N2), f32)), abi.put(np.ones((N2, H), f32))
        pbits = abi.put(np.zeros((16448 // 32, H), f32))
        pdh, pcs = abi.empty(16448 * H), abi.put(np.full(H, 7.0, f32))
        ws = abi.alloc(L.aar_gemm_f32_mask_bits_colsum_workspace_bytes(16448, H))
        wsb = L.aar_gemm_f32_mask_bits_colsum_workspace_bytes(16448, H)
        for M in (100, 16448):  # not a multiple of 64; more than 256 chunks
            assert L.aar_gemm_f32_mask_bits_colsum(NN, M, H, N2, pg, pw2, pbits, pdh, pcs, ws, wsb, None) == -3
        assert L.aar_gemm_f32_mask_bits_colsum(NT, 128, H, N2, pg, pw2, pbits, pdh, pcs, ws, wsb, None) == -3
        assert L.aar_gemm_f32_mask_bits_colsum(NN, 128, H, N2, pg, pw2, pbits, pdh, pcs, ws, 16, None) == -2
        assert (abi.get(pcs, (H,)) == 7.0).all()
        abi.check(L.aar_gemm_f32_mask_bits_colsum(NN, 0, H, N2, pg, pw2, pbits, pdh, pcs, ws, wsb, None))
        assert (abi.get(pcs, (H,)) == 0.0).all()
    finally:
        abi.free()
