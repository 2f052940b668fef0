"""Helpers for the GPU tests: move arrays through aargrad._core, and a thin
ctypes wrapper over the C ABI (include/aar_hip.h) for direct calls."""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB = Path(__file__).resolve().parent.parent / "aar-vlm_amd" / "aargrad" / "libaar_hip.so"


def dev(ag, arr, requires_grad=False):
    # np.array (not ascontiguousarray) keeps 0-d arrays 0-d
    t = ag.from_numpy(np.array(arr, dtype=np.float32, order="C")).to(ag.Device.CUDA)
    if requires_grad:
        t.requires_grad = True
    return t


def host(ag, t):
    return ag.to_numpy(t.to(ag.Device.CPU))


class Abi:
    """Direct C-ABI access with device buffers owned by this object."""

    def __init__(self):
        L = ctypes.CDLL(str(LIB))
        vp, i64, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t
        L.aar_error_string.restype = ctypes.c_char_p
        L.aar_malloc.argtypes = [ctypes.POINTER(vp), sz]
        L.aar_free.argtypes = [vp]
        L.aar_memcpy.argtypes = [vp, vp, sz, ctypes.c_int, vp]
        L.aar_memset_zero.argtypes = [vp, sz, vp]
        L.aar_gemm_f32.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, sz, vp]
        L.aar_gemm_f32_workspace_bytes.restype = sz
        L.aar_gemm_f32_workspace_bytes.argtypes = [ctypes.c_int, i64, i64, i64]
        ip = ctypes.POINTER(ctypes.c_int)
        L.aar_gemm_f32_tile_config.argtypes = [ctypes.c_int, ip, ip, ip]
        L.aar_gemm_f32_plan.argtypes = [ctypes.c_int, i64, i64, i64, sz, ip, ip]
        L.aar_gemm_f32_with_config.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, sz, ctypes.c_int,
                                               ctypes.c_int, vp]
        L.aar_softmax_fwd_f32.argtypes = [vp, vp, i64, i64, vp]
        L.aar_softmax_bwd_f32.argtypes = [vp, vp, vp, i64, i64, vp]
        L.aar_layernorm_fwd_f32.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, ctypes.c_float, vp]
        L.aar_layernorm_bwd_workspace_bytes.restype = sz
        L.aar_layernorm_bwd_workspace_bytes.argtypes = [i64, i64]
        L.aar_layernorm_bwd_f32.argtypes = [vp] * 8 + [i64, i64, vp, sz, vp]
        L.aar_flash_fwd_f32.argtypes = [vp] * 5 + [i64, i64, i64, ctypes.c_int, ctypes.c_float, vp]
        L.aar_flash_bwd_workspace_bytes.restype = sz
        L.aar_flash_bwd_workspace_bytes.argtypes = [i64, i64, i64]
        L.aar_flash_bwd_f32.argtypes = [vp] * 9 + [i64, i64, i64, ctypes.c_int, ctypes.c_float, vp, sz, vp]
        L.aar_flash_bwd_fast_workspace_bytes.restype = sz
        L.aar_flash_bwd_fast_workspace_bytes.argtypes = [i64, i64, i64, ctypes.c_int]
        L.aar_flash_fwd_workspace_bytes.restype = sz
        L.aar_flash_fwd_workspace_bytes.argtypes = [i64, i64, i64, ctypes.c_int]
        pi64 = ctypes.POINTER(i64)
        L.aar_flash_fwd_strided_plan_f32.argtypes = [vp] * 5 + [i64] * 4 + [pi64, ctypes.c_int, ctypes.c_float,
                                                                            ctypes.c_int, vp, sz, vp]
        L.aar_flash_bwd_strided_plan_f32.argtypes = [vp] * 9 + [i64] * 4 + [pi64, ctypes.c_int, ctypes.c_float,
                                                                            ctypes.c_int, vp, sz, vp]
        L.aar_add_f32.argtypes = [vp, vp, vp, i64, vp]
        L.aar_strided_copy_f32.argtypes = [vp, vp, ctypes.c_int, ctypes.POINTER(i64), ctypes.POINTER(i64),
                                           ctypes.POINTER(i64), vp]
        L.aar_synchronize.restype = ctypes.c_int
        self.L = L
        self._bufs = []

    def check(self, rc):
        if rc != 0:
            raise RuntimeError(self.L.aar_error_string(rc).decode())

    def alloc(self, nbytes):
        p = ctypes.c_void_p()
        self.check(self.L.aar_malloc(ctypes.byref(p), max(int(nbytes), 16)))
        self._bufs.append(p)
        return p.value

    def put(self, arr, offset_floats=0):
        """Upload into a fresh buffer, optionally at a float offset (misaligned)."""
        arr = np.ascontiguousarray(arr, np.float32)
        base = self.alloc(arr.nbytes + 4 * offset_floats + 16)
        p = base + 4 * offset_floats
        self.check(self.L.aar_memcpy(p, arr.ctypes.data, arr.nbytes, 1, None))
        return p

    def empty(self, n_floats, offset_floats=0):
        return self.alloc(4 * (n_floats + offset_floats) + 16) + 4 * offset_floats

    def get(self, p, shape):
        out = np.empty(shape, np.float32)
        self.check(self.L.aar_memcpy(out.ctypes.data, p, out.nbytes, 2, None))
        return out

    def free(self):
        self.L.aar_synchronize()
        for p in self._bufs:
            self.L.aar_free(p)
        self._bufs.clear()


def abi_flash(q, k, v, do, causal, query_block=0, key_block=0, fast=True, abi=None):
    """Forward (O, lse) and backward (dq, dk, dv) of [bh, T, d] operands
    through the C ABI's per-call plan entry points: query_block / key_block
    64 or 128 force the forward's / backward's decomposition for these calls
    only (0: the planner's).  The forward gets its split workspace; `fast`
    gives the backward the stored-dS workspace, else the minimum (recompute
    path)."""
    bh, T, d = q.shape
    own = abi is None
    abi = abi if abi is not None else Abi()
    L = abi.L
    try:
        pq, pk, pv, pdo = (abi.put(t) for t in (q, k, v, do))
        po, pl = abi.empty(bh * T * d), abi.empty(bh * T)
        s = 1.0 / float(np.sqrt(d))
        st = (ctypes.c_int64 * 24)(*([bh * T * d, T * d, d] * 8))
        fw = L.aar_flash_fwd_workspace_bytes(bh, T, d, int(causal))
        abi.check(L.aar_flash_fwd_strided_plan_f32(pq, pk, pv, po, pl, 1, bh, T, d, st, int(causal), s, query_block,
                                                   abi.alloc(fw) if fw else None, fw, None))
        o, lse = abi.get(po, (bh, T, d)), abi.get(pl, (bh, T))
        wsb = (L.aar_flash_bwd_fast_workspace_bytes(bh, T, d, int(causal)) if fast
               else L.aar_flash_bwd_workspace_bytes(bh, T, d))
        pdq, pdk, pdv = (abi.empty(bh * T * d) for _ in range(3))
        abi.check(L.aar_flash_bwd_strided_plan_f32(pq, pk, pv, po, pl, pdo, pdq, pdk, pdv, 1, bh, T, d, st,
                                                   int(causal), s, key_block, abi.alloc(wsb), wsb, None))
        return o, lse, [abi.get(p, (bh, T, d)) for p in (pdq, pdk, pdv)]
    finally:
        if own:
            abi.free()
