"""The no-allocation layernorm backward (aar_layernorm_bwd_noalloc_f32: its
dgamma/dbeta partials live in a static per-GPU buffer, no workspace argument)
against the workspace entry point aar_layernorm_bwd_f32 through the C ABI.
The two share their kernels, so dx, dgamma and dbeta must agree bit for bit:
on two calls in a row, the second with a smaller input (the buffer keeps the
first call's contents), on both load paths, and for a shape that needs more
than the static buffer, which must be rejected before any launch."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from devutil import Abi

pytestmark = pytest.mark.gpu
f32 = np.float32
AAR_ESCRATCH = -5


def _setup(abi):
    L = abi.L
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    L.aar_layernorm_bwd_noalloc_f32.argtypes = [vp] * 8 + [i64, i64, vp]
    L.aar_layernorm_bwd_noalloc_max_bytes.restype = ctypes.c_size_t
    L.aar_layernorm_bwd_noalloc_max_bytes.argtypes = []
    return L


def _case(abi, rows, cols, seed, offset=0):
    """Run both entry points on one seeded input; return their (dx, dw, db)."""
    L = abi.L
    rng = np.random.default_rng(seed)
    x = (3 * rng.standard_normal((rows, cols))).astype(f32)
    w = (1 + 0.02 * rng.standard_normal(cols)).astype(f32)
    b = (0.02 * rng.standard_normal(cols)).astype(f32)
    gy = rng.standard_normal((rows, cols)).astype(f32)
    px, pw, pb, pg = abi.put(x, offset), abi.put(w, offset), abi.put(b, offset), abi.put(gy, offset)
    py, pm, pr = abi.empty(rows * cols, offset), abi.empty(rows), abi.empty(rows)
    abi.check(L.aar_layernorm_fwd_f32(px, pw, pb, py, pm, pr, rows, cols, ctypes.c_float(1e-5), None))
    outs = []
    for noalloc in (False, True):
        pdx, pdw, pdb = abi.empty(rows * cols, offset), abi.empty(cols), abi.empty(cols)
        if noalloc:
            abi.check(L.aar_layernorm_bwd_noalloc_f32(pg, px, pw, pm, pr, pdx, pdw, pdb, rows, cols, None))
        else:
            wsb = L.aar_layernorm_bwd_workspace_bytes(rows, cols)
            abi.check(L.aar_layernorm_bwd_f32(pg, px, pw, pm, pr, pdx, pdw, pdb, rows, cols,
                                              abi.alloc(wsb), wsb, None))
        outs.append((abi.get(pdx, (rows, cols)), abi.get(pdw, (cols,)), abi.get(pdb, (cols,))))
    return outs


@pytest.mark.parametrize("first,second", [((65536, 384), (4099, 384)), ((65536, 768), (300, 130)),
                                          ((65536, 4096), (1000, 4096)), ((2048, 257), (17, 257))])
def test_noalloc_matches_workspace_entry_point(gpu, first, second):
    abi = Abi()
    try:
        _setup(abi)
        for i, (rows, cols) in enumerate((first, second)):
            print(f"noalloc layernorm bwd rows={rows} cols={cols}", flush=True)
            (dx0, dw0, db0), (dx1, dw1, db1) = _case(abi, rows, cols, seed=rows + cols + i)
            assert np.isfinite(dx1).all() and np.isfinite(dw1).all() and np.isfinite(db1).all()
            np.testing.assert_array_equal(dx1, dx0)
            np.testing.assert_array_equal(dw1, dw0)
            np.testing.assert_array_equal(db1, db0)
    finally:
        abi.free()


def test_noalloc_misaligned_rows(gpu):
    # operands offset by one float take the element-wise load path
    abi = Abi()
    try:
        _setup(abi)
        for rows, cols in ((5000, 384), (77, 100)):
            (dx0, dw0, db0), (dx1, dw1, db1) = _case(abi, rows, cols, seed=3, offset=1)
            np.testing.assert_array_equal(dx1, dx0)
            np.testing.assert_array_equal(dw1, dw0)
            np.testing.assert_array_equal(db1, db0)
    finally:
        abi.free()


def test_noalloc_rejects_oversize_and_keeps_working(gpu):
    abi = Abi()
    try:
        L = _setup(abi)
        cap = L.aar_layernorm_bwd_noalloc_max_bytes()
        assert cap == 16 << 20
        # 16384 columns exceed every register-resident row plan, so the wide
        # plan keeps one partial row of 128 KB per workgroup (1024 of them):
        # 128 MiB.  The operands are NULL: the size check rejects the call
        # first, and were it to pass, the null checks would reject it before
        # any launch.  (Never hand undersized buffers to an entry point in the
        # hope that it rejects the shape.)
        rows, cols = 65536, 16384
        assert L.aar_layernorm_bwd_workspace_bytes(rows, cols) > 4 * cap
        rc = L.aar_layernorm_bwd_noalloc_f32(None, None, None, None, None, None, None, None, rows, cols, None)
        assert rc == AAR_ESCRATCH
        assert b"static scratch" in L.aar_error_string(rc)
        assert L.aar_layernorm_bwd_noalloc_f32(None, None, None, None, None, None, None, None, 4, 0, None) == -1
        (dx0, dw0, db0), (dx1, dw1, db1) = _case(abi, 1024, 384, seed=9)
        np.testing.assert_array_equal(dx1, dx0)
        np.testing.assert_array_equal(dw1, dw0)
        np.testing.assert_array_equal(db1, db0)
    finally:
        abi.free()


def _free_device_bytes():
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_noalloc_calls_allocate_nothing(gpu):
    """The defining property: after a first call (which loads the code object
    with its static buffer), further calls of several shapes leave the
    device's free memory unchanged, to the byte."""
    abi = Abi()
    try:
        L = _setup(abi)
        shapes = [(4096, 384), (300, 768), (1000, 4096), (77, 100)]
        bufs = {}
        for rows, cols in shapes:  # operands allocated up front, outside the measured window
            rng = np.random.default_rng(rows + cols)
            x = (3 * rng.standard_normal((rows, cols))).astype(f32)
            w = (1 + 0.02 * rng.standard_normal(cols)).astype(f32)
            b = np.zeros(cols, f32)
            gy = rng.standard_normal((rows, cols)).astype(f32)
            px, pw, pb, pg = abi.put(x), abi.put(w), abi.put(b), abi.put(gy)
            py, pm, pr = abi.empty(rows * cols), abi.empty(rows), abi.empty(rows)
            abi.check(L.aar_layernorm_fwd_f32(px, pw, pb, py, pm, pr, rows, cols, ctypes.c_float(1e-5), None))
            pdx, pdw, pdb = abi.empty(rows * cols), abi.empty(cols), abi.empty(cols)
            bufs[(rows, cols)] = (pg, px, pw, pm, pr, pdx, pdw, pdb)
        rows, cols = shapes[0]
        abi.check(L.aar_layernorm_bwd_noalloc_f32(*bufs[(rows, cols)], rows, cols, None))  # warm-up
        abi.check(L.aar_synchronize())
        before = _free_device_bytes()
        for _ in range(3):
            for rows, cols in shapes:
                abi.check(L.aar_layernorm_bwd_noalloc_f32(*bufs[(rows, cols)], rows, cols, None))
        abi.check(L.aar_synchronize())
        assert _free_device_bytes() == before
    finally:
        abi.free()
