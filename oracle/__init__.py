"""Parity oracle -- TEST INFRASTRUCTURE ONLY.

numpy front end over two CPU libraries:
  * ``_build/liboracle.so``: the plain-C restatement of the reference CPU path
    (``aar_oracle.c``), always available once ``make -C oracle`` has run;
  * ``_ref/libaar_ref.so``: the reference's own CPU implementation compiled from
    its sources (``ref_driver.cpp`` + the reference tree), present only where
    the reference tree was available at build time.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker: the product never uses it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"
REF_PATH = HERE / "_ref" / "libaar_ref.so"

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64

_lib = None
_ref = None


def build(reference: str | None = None) -> None:
    """Compile the oracle (and oracle/_ref when the reference tree exists)."""
    cmd = ["make", "-s", "-C", str(HERE), "-j8", "all"]
    if reference:
        cmd.append(f"REF={reference}")
    subprocess.run(cmd, check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        for name in ("orc_matmul_nn", "orc_matmul_nt", "orc_matmul_tn"):
            getattr(L, name).argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64]
            getattr(L, name).restype = None
        L.orc_softmax_fwd.argtypes = [_f32p, _f32p, _i64, _i64]
        L.orc_softmax_bwd.argtypes = [_f32p, _f32p, _f32p, _i64, _i64]
        L.orc_layernorm_fwd.argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_void_p, ctypes.c_void_p,
                                        _i64, _i64, ctypes.c_float]
        L.orc_layernorm_bwd.argtypes = [_f32p] * 8 + [_i64, _i64]
        L.orc_attention_fwd.argtypes = [_f32p] * 4 + [_i64, _i64, _i64, ctypes.c_int]
        L.orc_attention_fwd.restype = ctypes.c_int
        L.orc_attention_bwd.argtypes = [_f32p] * 7 + [_i64, _i64, _i64, ctypes.c_int]
        L.orc_attention_bwd.restype = ctypes.c_int
        L.orc_attention_lse.argtypes = [_f32p, _f32p, _f64p, _i64, _i64, _i64, ctypes.c_int]
        L.orc_add.argtypes = [_f32p, _f32p, _f32p, _i64]
        _lib = L
    return _lib


def ref_available() -> bool:
    return REF_PATH.exists()


def ref():
    """The reference's own CPU build, or None when it was not built here."""
    global _ref
    if _ref is None and REF_PATH.exists():
        R = ctypes.CDLL(str(REF_PATH))
        vp = ctypes.c_void_p
        R.ref_matmul.argtypes = [ctypes.c_int, _f32p, _f32p, _f32p, _i64, _i64, _i64]
        R.ref_softmax.argtypes = [_f32p, vp, _f32p, vp, _i64, _i64]
        R.ref_layernorm.argtypes = [_f32p, _f32p, _f32p, vp, _f32p, vp, vp, vp, _i64, _i64, ctypes.c_float]
        R.ref_attention.argtypes = [_f32p, _f32p, _f32p, vp, _f32p, vp, vp, vp, _i64, _i64, _i64, ctypes.c_int]
        for f in (R.ref_matmul, R.ref_softmax, R.ref_layernorm, R.ref_attention):
            f.restype = ctypes.c_int
        _ref = R
    return _ref


def _c(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ------------------------------------------------------------------ GEMM
OPS = ("nn", "nt", "tn")


def gemm_shapes(op: str, a: np.ndarray, b: np.ndarray):
    if op == "nn":
        (M, K), N = a.shape, b.shape[1]
    elif op == "nt":
        (M, K), N = a.shape, b.shape[0]
    else:
        (K, M), N = a.shape, b.shape[1]
    return M, N, K


def matmul(op: str, a, b, rows: tuple[int, int] | None = None) -> np.ndarray:
    """C (or rows [r0, r1) of C, other rows zero) for op in nn / nt / tn."""
    a, b = _c(a), _c(b)
    M, N, K = gemm_shapes(op, a, b)
    r0, r1 = rows if rows is not None else (0, M)
    c = np.zeros((M, N), np.float32)
    getattr(lib(), f"orc_matmul_{op}")(a, b, c, M, N, K, r0, r1)
    return c


def softmax(x) -> np.ndarray:
    x = _c(x)
    y = np.empty_like(x)
    lib().orc_softmax_fwd(x, y, x.size // x.shape[-1], x.shape[-1])
    return y


def softmax_backward(g, y) -> np.ndarray:
    g, y = _c(g), _c(y)
    dx = np.empty_like(g)
    lib().orc_softmax_bwd(g, y, dx, g.size // g.shape[-1], g.shape[-1])
    return dx


def layernorm(x, w, b, eps: float = 1e-5, stats: bool = False):
    x, w, b = _c(x), _c(w), _c(b)
    rows, cols = x.size // x.shape[-1], x.shape[-1]
    y = np.empty_like(x)
    mean = np.empty(rows, np.float32)
    rstd = np.empty(rows, np.float32)
    lib().orc_layernorm_fwd(x, w, b, y, _ptr(mean), _ptr(rstd), rows, cols, eps)
    return (y, mean, rstd) if stats else y


def layernorm_backward(gy, x, w, mean, rstd):
    gy, x, w, mean, rstd = map(_c, (gy, x, w, mean, rstd))
    rows, cols = x.size // x.shape[-1], x.shape[-1]
    dx = np.empty_like(x)
    dw = np.empty(cols, np.float32)
    db = np.empty(cols, np.float32)
    lib().orc_layernorm_bwd(gy, x, w, mean, rstd, dx, dw, db, rows, cols)
    return dx, dw, db


def _bhtd(q):
    T, d = q.shape[-2], q.shape[-1]
    return q.size // (T * d), T, d


def attention(q, k, v, causal: bool) -> np.ndarray:
    q, k, v = _c(q), _c(k), _c(v)
    bh, T, d = _bhtd(q)
    o = np.empty_like(q)
    if lib().orc_attention_fwd(q, k, v, o, bh, T, d, int(causal)) != 0:
        raise MemoryError("oracle attention scratch")
    return o


def attention_backward(q, k, v, dout, causal: bool):
    q, k, v, dout = _c(q), _c(k), _c(v), _c(dout)
    bh, T, d = _bhtd(q)
    dq, dk, dv = np.empty_like(q), np.empty_like(q), np.empty_like(q)
    if lib().orc_attention_bwd(q, k, v, dout, dq, dk, dv, bh, T, d, int(causal)) != 0:
        raise MemoryError("oracle attention scratch")
    return dq, dk, dv


def attention_lse(q, k, causal: bool) -> np.ndarray:
    q, k = _c(q), _c(k)
    bh, T, d = _bhtd(q)
    out = np.empty(bh * T, np.float64)
    lib().orc_attention_lse(q, k, out, bh, T, d, int(causal))
    return out.reshape(q.shape[:-1])


def add(a, b) -> np.ndarray:
    a, b = _c(a), _c(b)
    c = np.empty_like(a)
    lib().orc_add(a, b, c, a.size)
    return c


# --------------------------------------------------- reference CPU build
def ref_matmul(op: str, a, b) -> np.ndarray:
    a, b = _c(a), _c(b)
    M, N, K = gemm_shapes(op, a, b)
    c = np.empty((M, N), np.float32)
    if ref().ref_matmul(OPS.index(op), a, b, c, M, N, K) != 0:
        raise RuntimeError("reference matmul failed")
    return c


def ref_softmax(x, g=None):
    x = _c(x)
    rows, cols = x.size // x.shape[-1], x.shape[-1]
    y = np.empty_like(x)
    dx = np.empty_like(x) if g is not None else None
    g = _c(g) if g is not None else None
    if ref().ref_softmax(x, _ptr(g), y, _ptr(dx), rows, cols) != 0:
        raise RuntimeError("reference softmax failed")
    return (y, dx) if g is not None else y


def ref_layernorm(x, w, b, eps=1e-5, gy=None):
    x, w, b = _c(x), _c(w), _c(b)
    rows, cols = x.size // x.shape[-1], x.shape[-1]
    y = np.empty_like(x)
    if gy is None:
        rc = ref().ref_layernorm(x, w, b, None, y, None, None, None, rows, cols, eps)
        if rc != 0:
            raise RuntimeError("reference layernorm failed")
        return y
    gy = _c(gy)
    dx, dw, db = np.empty_like(x), np.empty(cols, np.float32), np.empty(cols, np.float32)
    rc = ref().ref_layernorm(x, w, b, _ptr(gy), y, _ptr(dx), _ptr(dw), _ptr(db), rows, cols, eps)
    if rc != 0:
        raise RuntimeError("reference layernorm failed")
    return y, dx, dw, db


def ref_attention(q, k, v, causal, dout=None):
    q, k, v = _c(q), _c(k), _c(v)
    bh, T, d = _bhtd(q)
    o = np.empty_like(q)
    if dout is None:
        if ref().ref_attention(q, k, v, None, o, None, None, None, bh, T, d, int(causal)) != 0:
            raise RuntimeError("reference attention failed")
        return o
    dout = _c(dout)
    dq, dk, dv = np.empty_like(q), np.empty_like(q), np.empty_like(q)
    rc = ref().ref_attention(q, k, v, _ptr(dout), o, _ptr(dq), _ptr(dk), _ptr(dv), bh, T, d, int(causal))
    if rc != 0:
        raise RuntimeError("reference attention failed")
    return o, dq, dk, dv
