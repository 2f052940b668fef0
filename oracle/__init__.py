"""Parity oracle -- TEST INFRASTRUCTURE ONLY.

numpy front end over two CPU libraries:
  * ``_build/liboracle.so``: the plain-C restatement of the reference CPU path
    (``aar_oracle.c``), always available once ``make -C oracle`` has run;
  * ``_ref/libaar_ref.so``: the reference's own CPU implementation compiled from
    its sources (``ref_driver.cpp`` + the reference tree), present only where
    the reference tree was available at build time;
  * ``_ref/libaar_glue.so``: the same reference sources and driver with the
    reference's device entry points bound to libaar_hip.so (``hip_backend.cpp``).
    Inside ``reference_on_device()`` the ``ref_*`` wrappers call it, so the
    reference's own C++ runs its ops on the GPU; it checks the integration
    boundary, and the CPU build stays the checker.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker: the product never uses it.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"
REF_PATH = HERE / "_ref" / "libaar_ref.so"
GLUE_PATH = HERE / "_ref" / "libaar_glue.so"

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64

_lib = None
_ref = None
_glue = None
_front = None  # the library the ref_* wrappers call inside reference_on_device()


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
        for name in ("orc_sub", "orc_mul"):
            getattr(L, name).argtypes = [_f32p, _f32p, _f32p, _i64]
        L.orc_scale.argtypes = [_f32p, _f32p, ctypes.c_float, _i64]
        for name in ("orc_relu", "orc_gelu"):
            getattr(L, name).argtypes = [_f32p, _f32p, _i64]
        for name in ("orc_relu_bwd", "orc_gelu_bwd"):
            getattr(L, name).argtypes = [_f32p, _f32p, _f32p, _i64]
        L.orc_add_bias.argtypes = [_f32p, _f32p, _f32p, _i64, _i64]
        L.orc_bias_grad.argtypes = [_f32p, _f32p, _i64, _i64]
        L.orc_sum_all.argtypes = [_f32p, _i64]
        L.orc_sum_all.restype = ctypes.c_float
        L.orc_scaled_add.argtypes = [_f32p, _f32p, ctypes.c_float, _i64]
        L.orc_embedding_fwd.argtypes = [_f32p, _i64p, _f32p, _i64, _i64, _i64]
        L.orc_embedding_fwd.restype = ctypes.c_int
        L.orc_embedding_bwd.argtypes = [_f32p, _i64p, _f32p, _i64, _i64, _i64]
        L.orc_cross_entropy_fwd.argtypes = [_f32p, _i64p, ctypes.POINTER(ctypes.c_float), _i64, _i64, _i64]
        L.orc_cross_entropy_fwd.restype = ctypes.c_int
        L.orc_cross_entropy_bwd.argtypes = [ctypes.c_float, _f32p, _i64p, _f32p, _i64, _i64, _i64]
        L.orc_adamw.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64] + [ctypes.c_float] * 7
        _u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
        L.orc_philox4x32_10.argtypes = [_u32p, _u32p, _u32p]
        L.orc_philox_uniform.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.orc_philox_uniform.restype = ctypes.c_float
        L.orc_dropout.argtypes = [_f32p, _f32p, _f32p, _i64, ctypes.c_float, ctypes.c_uint64]
        L.orc_causal_mask.argtypes = [_f32p, _f32p, _i64, _i64, ctypes.c_float]
        _lib = L
    return _lib


def ref_available() -> bool:
    return REF_PATH.exists()


def glue_available() -> bool:
    return GLUE_PATH.exists()


def ref():
    """The library the ref_* wrappers call: the reference's own CPU build (None
    when it was not built here), or libaar_glue.so inside reference_on_device()."""
    global _ref
    if _front is not None:
        return _front
    if _ref is None and REF_PATH.exists():
        _ref = _bind_driver(ctypes.CDLL(str(REF_PATH)))
    return _ref


@contextlib.contextmanager
def reference_on_device():
    """Within the block the ref_* wrappers run the reference's ops, autograd and
    optimizer steps with every operand on Device::CUDA: libaar_glue.so, the
    reference's C++ with its device entry points bound to libaar_hip.so."""
    global _glue, _front
    if _glue is None:
        if not GLUE_PATH.exists():
            raise RuntimeError(f"{GLUE_PATH} is not built")
        _glue = _bind_driver(ctypes.CDLL(str(GLUE_PATH)))
    prev, _front = _front, _glue
    try:
        yield
    finally:
        _front = prev


def _bind_driver(R):
    """Argument types of ref_driver.cpp's entry points (both builds)."""
    vp = ctypes.c_void_p
    R.ref_matmul.argtypes = [ctypes.c_int, _f32p, _f32p, _f32p, _i64, _i64, _i64]
    R.ref_softmax.argtypes = [_f32p, vp, _f32p, vp, _i64, _i64]
    R.ref_layernorm.argtypes = [_f32p, _f32p, _f32p, vp, _f32p, vp, vp, vp, _i64, _i64, ctypes.c_float]
    R.ref_attention.argtypes = [_f32p, _f32p, _f32p, vp, _f32p, vp, vp, vp, _i64, _i64, _i64, ctypes.c_int]
    R.ref_elementwise.argtypes = [ctypes.c_int, _f32p, vp, ctypes.c_float, vp, _f32p, vp, _i64]
    R.ref_add_bias.argtypes = [_f32p, _f32p, vp, _f32p, vp, _i64, _i64]
    R.ref_sum_all.argtypes = [_f32p, _i64, ctypes.POINTER(ctypes.c_float)]
    R.ref_embedding.argtypes = [_f32p, _i64p, vp, _f32p, vp, _i64, _i64, _i64]
    R.ref_cross_entropy.argtypes = [_f32p, _i64p, _i64, _i64, _i64, ctypes.c_float,
                                    ctypes.POINTER(ctypes.c_float), vp]
    R.ref_adamw.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64] + [ctypes.c_float] * 7
    R.ref_gpt_step.argtypes = [_i64] * 6 + [ctypes.POINTER(ctypes.c_void_p), _i64p, _i64p, ctypes.c_float,
                                             ctypes.POINTER(ctypes.c_float)]
    R.ref_gpt_step.restype = ctypes.c_int
    pp = ctypes.POINTER(ctypes.c_void_p)
    R.ref_lm_step.argtypes = [_i64] * 6 + [ctypes.c_float, _i64, pp, pp, pp, _i64p, _i64p] + \
        [ctypes.c_float] * 7 + [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p]
    R.ref_lm_step.restype = ctypes.c_int
    R.ref_philox_uniform.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
    R.ref_philox_uniform.restype = ctypes.c_float
    R.ref_dropout.argtypes = [_f32p, _f32p, vp, _i64, ctypes.c_float, ctypes.c_uint64]
    R.ref_causal_mask.argtypes = [_f32p, vp, _f32p, vp, _i64, _i64]
    R.ref_bmm.argtypes = [ctypes.c_int, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64]
    R.ref_fanin_graph.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64]
    for f in (R.ref_dropout, R.ref_causal_mask, R.ref_bmm, R.ref_fanin_graph):
        f.restype = ctypes.c_int
    for f in (R.ref_matmul, R.ref_softmax, R.ref_layernorm, R.ref_attention, R.ref_elementwise,
              R.ref_add_bias, R.ref_sum_all, R.ref_embedding, R.ref_cross_entropy, R.ref_adamw):
        f.restype = ctypes.c_int
    return R


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


def philox4x32_10(counter, key) -> np.ndarray:
    """One Philox-4x32-10 block: uint32[4] counter, uint32[2] key -> uint32[4]."""
    c = np.ascontiguousarray(counter, np.uint32)
    k = np.ascontiguousarray(key, np.uint32)
    out = np.empty(4, np.uint32)
    lib().orc_philox4x32_10(c, k, out)
    return out


def philox_uniform(seed: int, idx: int) -> float:
    return float(np.float32(lib().orc_philox_uniform(seed, idx)))


def dropout(x, p: float, seed: int):
    """(out, mask) of dropout over the flattened x with stream `seed`."""
    x = _c(x)
    o, m = np.empty_like(x), np.empty_like(x)
    lib().orc_dropout(x, o, m, x.size, p, seed)
    return o, m


def causal_mask(x, fill: float = float("-inf")) -> np.ndarray:
    """x [..., T, T] with entries above the diagonal replaced by `fill`."""
    x = _c(x)
    T = x.shape[-1]
    y = np.empty_like(x)
    lib().orc_causal_mask(x, y, x.size // (T * T), T, fill)
    return y


BMM_OPS = ("bmm", "bmm_a_bt", "bmm_at_b")


def bmm(op: str, a, b) -> np.ndarray:
    """Batched product over the leading dimension: per batch, matmul with op
    nn (bmm), nt (bmm_a_bt) or tn (bmm_at_b)."""
    a, b = _c(a), _c(b)
    g = {"bmm": "nn", "bmm_a_bt": "nt", "bmm_at_b": "tn"}[op]
    M, N, _ = gemm_shapes(g, a[0] if a.shape[0] else np.empty(a.shape[1:], np.float32),
                          b[0] if b.shape[0] else np.empty(b.shape[1:], np.float32))
    c = np.empty((a.shape[0], M, N), np.float32)
    for i in range(a.shape[0]):
        c[i] = matmul(g, a[i], b[i])
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


# ------------------------------------------------------ GPT-step ops (next row)
def sub(a, b):
    a, b = _c(a), _c(b)
    c = np.empty_like(a)
    lib().orc_sub(a, b, c, a.size)
    return c


def mul(a, b):
    a, b = _c(a), _c(b)
    c = np.empty_like(a)
    lib().orc_mul(a, b, c, a.size)
    return c


def scale(x, alpha):
    x = _c(x)
    y = np.empty_like(x)
    lib().orc_scale(x, y, alpha, x.size)
    return y


def relu(x):
    x = _c(x)
    y = np.empty_like(x)
    lib().orc_relu(x, y, x.size)
    return y


def relu_backward(g, x):
    g, x = _c(g), _c(x)
    d = np.empty_like(x)
    lib().orc_relu_bwd(g, x, d, x.size)
    return d


def gelu(x):
    x = _c(x)
    y = np.empty_like(x)
    lib().orc_gelu(x, y, x.size)
    return y


def gelu_backward(g, x):
    g, x = _c(g), _c(x)
    d = np.empty_like(x)
    lib().orc_gelu_bwd(g, x, d, x.size)
    return d


def add_bias(x, bias):
    x, bias = _c(x), _c(bias)
    y = np.empty_like(x)
    lib().orc_add_bias(x, bias, y, x.size, bias.size)
    return y


def bias_grad(g, D):
    g = _c(g)
    db = np.empty(D, np.float32)
    lib().orc_bias_grad(g, db, g.size, D)
    return db


def sum_all(x):
    x = _c(x)
    return np.float32(lib().orc_sum_all(x, x.size))


def scaled_add(dst, src, alpha):
    dst = _c(dst).copy()
    lib().orc_scaled_add(dst, _c(src), alpha, dst.size)
    return dst


def embedding(w, ids):
    w = _c(w)
    ids = np.ascontiguousarray(ids, np.int64)
    V, D = w.shape
    out = np.empty(ids.shape + (D,), np.float32)
    if lib().orc_embedding_fwd(w, ids.reshape(-1), out.reshape(-1, D), ids.size, V, D) != 0:
        raise IndexError("embedding: id out of range [0, vocab_size)")
    return out


def embedding_backward(g, ids, vocab):
    ids = np.ascontiguousarray(ids, np.int64).reshape(-1)
    g = _c(g).reshape(ids.size, -1)
    dw = np.empty((vocab, g.shape[1]), np.float32)
    lib().orc_embedding_bwd(g, ids, dw, ids.size, vocab, g.shape[1])
    return dw


def cross_entropy(logits, targets, ignore_index=-100):
    logits = _c(logits)
    targets = np.ascontiguousarray(targets, np.int64)
    N, V = logits.shape
    out = ctypes.c_float()
    if lib().orc_cross_entropy_fwd(logits, targets, ctypes.byref(out), N, V, ignore_index) != 0:
        raise IndexError("cross_entropy: target out of range [0, V)")
    return np.float32(out.value)


def cross_entropy_backward(go, logits, targets, ignore_index=-100):
    logits = _c(logits)
    targets = np.ascontiguousarray(targets, np.int64)
    N, V = logits.shape
    d = np.empty_like(logits)
    lib().orc_cross_entropy_bwd(go, logits, targets, d, N, V, ignore_index)
    return d


def adamw(p, g, m, v, lr, b1, b2, eps, wd, bc1, bc2):
    p, m, v = _c(p).copy(), _c(m).copy(), _c(v).copy()
    lib().orc_adamw(p, _c(g), m, v, p.size, lr, b1, b2, eps, wd, bc1, bc2)
    return p, m, v


def ref_elementwise(op, a, b=None, alpha=0.0, g=None):
    a = _c(a)
    b = _c(b) if b is not None else None
    g = _c(g) if g is not None else None
    y = np.empty_like(a)
    da = np.empty_like(a) if g is not None else None
    code = {"sub": 0, "mul": 1, "scale": 2, "relu": 3, "gelu": 4}[op]
    if ref().ref_elementwise(code, a, _ptr(b), alpha, _ptr(g), y, _ptr(da), a.size) != 0:
        raise RuntimeError("reference elementwise failed")
    return (y, da) if g is not None else y


def ref_add_bias(x, bias, g=None):
    x, bias = _c(x), _c(bias)
    y = np.empty_like(x)
    db = np.empty_like(bias) if g is not None else None
    g = _c(g) if g is not None else None
    if ref().ref_add_bias(x, bias, _ptr(g), y, _ptr(db), x.size // bias.size, bias.size) != 0:
        raise RuntimeError("reference add_bias failed")
    return (y, db) if g is not None else y


def ref_sum_all(x):
    x = _c(x)
    r = ctypes.c_float()
    if ref().ref_sum_all(x, x.size, ctypes.byref(r)) != 0:
        raise RuntimeError("reference sum_all failed")
    return np.float32(r.value)


def ref_embedding(w, ids, g=None):
    w = _c(w)
    ids = np.ascontiguousarray(ids, np.int64).reshape(-1)
    V, D = w.shape
    y = np.empty((ids.size, D), np.float32)
    dw = np.empty_like(w) if g is not None else None
    g = _c(g) if g is not None else None
    if ref().ref_embedding(w, ids, _ptr(g), y, _ptr(dw), ids.size, V, D) != 0:
        raise RuntimeError("reference embedding failed")
    return (y, dw) if g is not None else y


def ref_cross_entropy(logits, targets, ignore_index=-100, go=None):
    logits = _c(logits)
    targets = np.ascontiguousarray(targets, np.int64)
    N, V = logits.shape
    loss = ctypes.c_float()
    d = np.empty_like(logits) if go is not None else None
    if ref().ref_cross_entropy(logits, targets, N, V, ignore_index, go or 0.0, ctypes.byref(loss), _ptr(d)) != 0:
        raise RuntimeError("reference cross_entropy failed")
    return (np.float32(loss.value), d) if go is not None else np.float32(loss.value)


def ref_adamw(p, g, m, v, lr, b1, b2, eps, wd, bc1, bc2):
    p, m, v = _c(p).copy(), _c(m).copy(), _c(v).copy()
    if ref().ref_adamw(p, _c(g), m, v, p.size, lr, b1, b2, eps, wd, bc1, bc2) != 0:
        raise RuntimeError("reference adamw failed")
    return p, m, v


def ref_gpt_step(cfg, params, ids, targets, lr):
    """One SGD step of the config-5 GPT on the reference CPU path.  Returns
    (loss before the update, updated parameter arrays)."""
    ps = [np.ascontiguousarray(p, np.float32).copy() for p in params]
    ptrs = (ctypes.c_void_p * len(ps))(*[p.ctypes.data for p in ps])
    ids = np.ascontiguousarray(ids, np.int64)
    targets = np.ascontiguousarray(targets, np.int64).reshape(-1)
    loss = ctypes.c_float()
    rc = ref().ref_gpt_step(cfg["vocab"], cfg["ctx"], cfg["layers"], cfg["d_model"], cfg["heads"], ids.shape[0],
                            ptrs, ids.reshape(-1), targets, lr, ctypes.byref(loss))
    if rc != 0:
        raise RuntimeError("reference gpt step failed")
    return float(loss.value), ps


def ref_philox_uniform(seed: int, idx: int) -> float:
    return float(np.float32(ref().ref_philox_uniform(seed, idx)))


def ref_dropout(x, p: float, seed: int, grad: bool = False):
    """vlm::manual_seed(seed); vlm::dropout(x, p) on the reference CPU path.
    With grad, also d(sum(out))/dx (the mask)."""
    x = _c(x).reshape(-1)
    y = np.empty_like(x)
    dx = np.empty_like(x) if grad else None
    if ref().ref_dropout(x, y, _ptr(dx), x.size, p, seed) != 0:
        raise RuntimeError("reference dropout failed")
    return (y, dx) if grad else y


def ref_causal_mask(x, g=None):
    x = _c(x)
    T = x.shape[-1]
    y = np.empty_like(x)
    g = None if g is None else _c(g)
    dx = np.empty_like(x) if g is not None else None
    if ref().ref_causal_mask(x, _ptr(g), y, _ptr(dx), x.size // (T * T), T) != 0:
        raise RuntimeError("reference apply_causal_mask failed")
    return (y, dx) if g is not None else y


def ref_bmm(op: str, a, b) -> np.ndarray:
    a, b = _c(a), _c(b)
    Bn = a.shape[0]
    if op == "bmm":
        M, K, N = a.shape[1], a.shape[2], b.shape[2]
    elif op == "bmm_a_bt":
        M, K, N = a.shape[1], a.shape[2], b.shape[1]
    else:
        K, M, N = a.shape[1], a.shape[2], b.shape[2]
    c = np.empty((Bn, M, N), np.float32)
    if ref().ref_bmm(BMM_OPS.index(op), a, b, c, Bn, M, N, K) != 0:
        raise RuntimeError("reference bmm failed")
    return c


def ref_fanin_graph(x, w, g):
    """x.grad of the reference driver's fan-in graph (h = x*w0; u = h*w1;
    v = 0.75*h; z = h*w2; t = x*w3; root = ((u+v)+z)+t) through the
    reference's own autograd; w is [4, n]."""
    x, w, g = _c(x), _c(w), _c(g)
    n = x.size
    assert w.shape == (4, n) and g.size == n
    dx = np.empty_like(x)
    if ref().ref_fanin_graph(x, w, g, dx, n) != 0:
        raise RuntimeError("reference fan-in graph failed")
    return dx


def ref_lm_step(cfg, params, m, v, ids, targets, *, dropout, seed, lr, betas, eps, wd, t, grads=False):
    """One AdamW training step of the reference Shakespeare GPT on the
    reference CPU path.  params, m and v are updated in place; returns the
    loss before the update (and the gradients when grads is set).  seed >= 0
    reseeds the dropout stream, a negative seed continues it."""
    def ptrs(arrs):
        return (ctypes.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
    for a in list(params) + list(m) + list(v):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    g = [np.empty_like(p) for p in params] if grads else None
    ids = np.ascontiguousarray(ids, np.int64)
    targets = np.ascontiguousarray(targets, np.int64).reshape(-1)
    b1, b2 = betas
    bc1, bc2 = 1.0 - b1 ** t, 1.0 - b2 ** t  # AdamW.step, in double as the Python optimizer
    loss = ctypes.c_float()
    rc = ref().ref_lm_step(cfg["vocab"], cfg["ctx"], cfg["layers"], cfg["d_model"], cfg["heads"], ids.shape[0],
                           dropout, seed, ptrs(params), ptrs(m), ptrs(v), ids.reshape(-1), targets, lr, b1, b2, eps,
                           wd, bc1, bc2, ctypes.byref(loss), ptrs(g) if grads else None)
    if rc != 0:
        raise RuntimeError("reference lm step failed")
    return (float(loss.value), g) if grads else float(loss.value)
