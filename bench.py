#!/usr/bin/env python3
"""Benchmark of the MI355X aargrad backend on BASELINE.json's headline metric:
fp32 matmul TFLOPS at 4096^3 (fraction of the 157.3 TFLOP/s fp32 MFMA peak),
plus causal flash-attention fwd+bwd TFLOPS (B8 H12 T4096 d64).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one C = A.B at M=N=K=4096 (BASELINE config 2's square 4096 point,
A, B ~ N(0,1)/sqrt(K), synthetic, resident in HBM), issued through the product
path: aargrad.matmul -> aargrad._core -> aar_gemm_f32 (C ABI) -> the gfx950
MFMA kernel, all ordered on the null stream.  W untimed steps, then exactly K
timed steps bracketed by device synchronisation; HIP events recorded on that
same stream time the region, one per step boundary, so the median and p99
step times are reported beside the mean.  One GPU only: --gpus N > 1 exits
with a message.

Prints ONE JSON line on stdout; a human-readable summary goes to stderr.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "aar-vlm_amd"))

PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 matrix peak
# The reference's published fp32 matmul figure at 4096^3 (its shipping v4 kernel, A100 80GB PCIe).
REF_PUBLISHED_TFLOPS = 16.02
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Events:
    """HIP events through the C ABI, recorded on the null stream (the stream
    every aargrad op is enqueued on)."""

    def __init__(self):
        self.L = ctypes.CDLL(str(REPO / "aar-vlm_amd" / "aargrad" / "libaar_hip.so"))
        vp = ctypes.c_void_p
        self.L.aar_event_create.argtypes = [ctypes.POINTER(vp)]
        self.L.aar_event_record.argtypes = [vp, vp]
        self.L.aar_event_elapsed_ms.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        self.L.aar_event_destroy.argtypes = [vp]
        self.a, self.b = vp(), vp()
        assert self.L.aar_event_create(ctypes.byref(self.a)) == 0
        assert self.L.aar_event_create(ctypes.byref(self.b)) == 0

    def start(self):
        self.L.aar_event_record(self.a, None)

    def stop_ms(self):
        self.L.aar_event_record(self.b, None)
        ms = ctypes.c_float()
        assert self.L.aar_event_elapsed_ms(ctypes.byref(ms), self.a, self.b) == 0
        return float(ms.value)


class StepTimer:
    """One HIP event per step boundary on the null stream, for per-step
    times (median and p99, the reference bench's protocol) beside the
    whole-run mean.  Recording an event enqueues a marker only: no sync."""

    def __init__(self, ev: Events, steps: int):
        self.L = ev.L
        self.evs = []
        for _ in range(steps + 1):
            e = ctypes.c_void_p()
            assert self.L.aar_event_create(ctypes.byref(e)) == 0
            self.evs.append(e)
        self.i = 0

    def mark(self):
        self.L.aar_event_record(self.evs[self.i], None)
        self.i += 1

    def _ms(self, a, b):
        ms = ctypes.c_float()
        assert self.L.aar_event_elapsed_ms(ctypes.byref(ms), a, b) == 0
        return float(ms.value)

    def result(self):
        """(total ms, {median, p99} per step in ms); call after a synchronize."""
        assert self.i == len(self.evs), "one mark per step boundary"
        per = np.array([self._ms(self.evs[k], self.evs[k + 1]) for k in range(len(self.evs) - 1)])
        total = self._ms(self.evs[0], self.evs[-1])
        for e in self.evs:
            self.L.aar_event_destroy(e)
        self.evs = []
        return total, {"median_ms": round(float(np.median(per)), 5),
                       "p99_ms": round(float(np.percentile(per, 99)), 5)}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def load_traffic(name: str):
    """L2-to-fabric bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE
    + WRITE_SIZE count L2 misses and write-backs, scaled by the copy-kernel
    calibration), committed under profiles/ as JSON; None when not
    measured."""
    p = REPO / "profiles" / f"{name}_traffic.json"
    if not p.exists():
        return None
    try:
        return float(json.loads(p.read_text())["l2_fabric_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def matmul_inputs(ag, n: int = 4096):
    """The headline step's operands, uploaded once (resident in HBM before
    any timing starts)."""
    rng = np.random.default_rng(0)
    a = (rng.standard_normal((n, n)) / np.sqrt(n)).astype(np.float32)
    b = (rng.standard_normal((n, n)) / np.sqrt(n)).astype(np.float32)
    return a, b, ag.from_numpy(a).to(ag.Device.CUDA), ag.from_numpy(b).to(ag.Device.CUDA)


def bench_matmul(ag, steps: int, warmup: int, ev: Events, inputs=None):
    a, b, ta, tb = inputs if inputs is not None else matmul_inputs(ag)
    n = a.shape[0]
    rng = np.random.default_rng(1)
    for _ in range(warmup):
        ag.matmul(ta, tb)
    ag.cuda_synchronize()
    st = StepTimer(ev, steps)
    t0 = time.perf_counter()
    st.mark()
    for _ in range(steps):
        c = ag.matmul(ta, tb)
        st.mark()
    ag.cuda_synchronize()
    wall = time.perf_counter() - t0
    ms, dist = st.result()
    # spot-check the timed output (rows sampled, float64 closed form)
    ch = ag.to_numpy(c.to(ag.Device.CPU))
    rows = rng.choice(n, 8, replace=False)
    ref = a[rows].astype(np.float64) @ b.astype(np.float64)
    err = float(np.abs(ch[rows] - ref).max() / max(np.abs(ref).max(), 1.0))
    if not err <= 1e-4 * np.sqrt(n):
        raise SystemExit(f"bench: matmul result check failed (err {err:.3e})")
    return ms / steps, wall, err, (a, b), dist


def bench_flash(ag, steps: int, warmup: int, ev: Events, T: int = 4096, B: int = 8, H: int = 12):
    d = 64
    rng = np.random.default_rng(0)
    q, k, v, do = (rng.standard_normal((B, H, T, d)).astype(np.float32) for _ in range(4))
    tq, tk, tv = (ag.from_numpy(x).to(ag.Device.CUDA) for x in (q, k, v))
    tdo = ag.from_numpy(do).to(ag.Device.CUDA)
    for t in (tq, tk, tv):
        t.requires_grad = True

    def step():
        o = ag.flash_attention(tq, tk, tv, True)
        o.backward(tdo)
        for t in (tq, tk, tv):
            t.zero_grad()
        return o

    for _ in range(warmup):
        step()
    ag.cuda_synchronize()
    st = StepTimer(ev, steps)
    st.mark()
    for _ in range(steps):
        step()
        st.mark()
    ag.cuda_synchronize()
    ms, dist = st.result()
    fwd_flops = 4.0 * B * H * T * T * d / 2.0
    return ms / steps, 3.5 * fwd_flops, dist


class Abi:
    """Direct C-ABI calls with preallocated buffers (kernel-level timing)."""

    def __init__(self, L):
        vp, i64, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t
        L.aar_malloc.argtypes = [ctypes.POINTER(vp), sz]
        L.aar_free.argtypes = [vp]
        L.aar_memcpy.argtypes = [vp, vp, sz, ctypes.c_int, vp]
        L.aar_softmax_fwd_f32.argtypes = [vp, vp, i64, i64, vp]
        L.aar_softmax_bwd_f32.argtypes = [vp, vp, vp, i64, i64, vp]
        L.aar_layernorm_fwd_f32.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, ctypes.c_float, vp]
        L.aar_layernorm_bwd_workspace_bytes.restype = sz
        L.aar_layernorm_bwd_workspace_bytes.argtypes = [i64, i64]
        L.aar_layernorm_bwd_f32.argtypes = [vp] * 8 + [i64, i64, vp, sz, vp]
        L.aar_add_f32.argtypes = [vp, vp, vp, i64, vp]
        self.L = L
        self.bufs = []

    def alloc(self, nbytes):
        p = ctypes.c_void_p()
        if self.L.aar_malloc(ctypes.byref(p), max(int(nbytes), 256)) != 0:
            raise MemoryError(nbytes)
        self.bufs.append(p)
        return p.value

    def put(self, arr):
        p = self.alloc(arr.nbytes)
        assert self.L.aar_memcpy(p, arr.ctypes.data, arr.nbytes, 1, None) == 0
        return p

    def free(self):
        self.L.aar_synchronize()
        for p in self.bufs:
            self.L.aar_free(p)
        self.bufs.clear()


def bench_rowwise(ev: Events, iters: int = 20, min_set_bytes: float = 1.2e9):
    """Softmax / layernorm fwd+bwd at BASELINE config 3 (rows 65536,
    cols 384/768/4096), rotating over enough buffer sets (>= 1.2 GB of
    operands) that the 256 MB Infinity Cache cannot serve them.  Algorithmic
    bytes: softmax fwd 8RC, bwd 12RC; layernorm fwd-with-stats 8RC+8C+8R,
    bwd 12RC+12C+8R (dgamma/dbeta partials excluded)."""
    abi = Abi(ev.L)
    rows = 65536
    out = {}
    rng = np.random.default_rng(0)
    try:
        for cols in (384, 768, 4096):
            rc_bytes = rows * cols * 4
            nsets = max(1, int(np.ceil(min_set_bytes / (3 * rc_bytes))))
            x = (3 * rng.standard_normal((rows, cols))).astype(np.float32)
            w = (1 + 0.02 * rng.standard_normal(cols)).astype(np.float32)
            b = (0.02 * rng.standard_normal(cols)).astype(np.float32)
            sets = [(abi.put(x), abi.alloc(rc_bytes), abi.put(x)) for _ in range(nsets)]  # x, y, g
            pw, pb = abi.put(w), abi.put(b)
            pm, pr = abi.alloc(rows * 4), abi.alloc(rows * 4)
            pdw, pdb = abi.alloc(cols * 4), abi.alloc(cols * 4)
            wsb = ev.L.aar_layernorm_bwd_workspace_bytes(rows, cols)
            pws = abi.alloc(wsb)
            L = ev.L
            cases = {
                "softmax_fwd": (8.0 * rows * cols, lambda s: L.aar_softmax_fwd_f32(s[0], s[1], rows, cols, None)),
                "softmax_bwd": (12.0 * rows * cols,
                                lambda s: L.aar_softmax_bwd_f32(s[2], s[1], s[0], rows, cols, None)),
                "layernorm_fwd": (8.0 * rows * cols + 8 * cols + 8 * rows,
                                  lambda s: L.aar_layernorm_fwd_f32(s[0], pw, pb, s[1], pm, pr, rows, cols,
                                                                    ctypes.c_float(1e-5), None)),
                "layernorm_bwd": (12.0 * rows * cols + 12 * cols + 8 * rows,
                                  lambda s: L.aar_layernorm_bwd_f32(s[2], s[0], pw, pm, pr, s[1], pdw, pdb, rows,
                                                                    cols, pws, wsb, None)),
            }
            for name, (nbytes, fn) in cases.items():
                for i in range(3):
                    assert fn(sets[i % nsets]) == 0
                ev.start()
                for i in range(iters):
                    assert fn(sets[i % nsets]) == 0
                ms = ev.stop_ms() / iters
                out[f"{name}_c{cols}"] = {"ms": round(ms, 4), "GB_s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                          "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                                          "buffer_sets": nsets}
            abi.free()
    finally:
        abi.free()
    return out


def bench_extra(ev: Events, iters: int = 10):
    """The non-flash attention ops, dropout and the token-window gather
    through the C ABI.  dropout
    over 2^26 floats (algorithmic 12 B/element: x in, out and mask out);
    causal mask over [96, 1024, 1024] (8 B/element); bmm_a_bt scores
    (96 x 1024x1024x64, the unfused attention of B8 H12 T1024 d64) and a
    square batched NN product (8 x 2048^3), counted as 2*B*M*N*K flops."""
    abi = Abi(ev.L)
    L = ev.L
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    L.aar_dropout_f32.argtypes = [vp, vp, vp, i64, ctypes.c_float, ctypes.c_uint64, vp]
    L.aar_causal_mask_f32.argtypes = [vp, vp, i64, i64, ctypes.c_float, vp]
    L.aar_gemm_f32_batched.argtypes = [ctypes.c_int] + [i64] * 4 + [vp, i64, i64, vp, i64, i64, vp, i64, i64, vp]
    out = {}
    rng = np.random.default_rng(0)

    def timed(fn):
        for _ in range(2):
            assert fn() == 0
        ev.start()
        for _ in range(iters):
            assert fn() == 0
        return ev.stop_ms() / iters

    try:
        n = 1 << 26
        px, po, pm = abi.put(rng.standard_normal(n).astype(np.float32)), abi.alloc(4 * n), abi.alloc(4 * n)
        ms = timed(lambda: L.aar_dropout_f32(px, po, pm, n, ctypes.c_float(0.1), 1234, None))
        out["dropout_n2^26"] = {"ms": round(ms, 4), "GB_s": round(12 * n / (ms * 1e-3) / 1e9, 1),
                                "frac_of_hbm_peak": round(12 * n / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
        abi.free()
        mats, T = 96, 1024
        px, py = abi.put(rng.standard_normal(mats * T * T).astype(np.float32)), abi.alloc(4 * mats * T * T)
        ms = timed(lambda: L.aar_causal_mask_f32(px, py, mats, T, ctypes.c_float(float("-inf")), None))
        nb = 8 * mats * T * T
        out["causal_mask_96x1024x1024"] = {"ms": round(ms, 4), "GB_s": round(nb / (ms * 1e-3) / 1e9, 1),
                                           "frac_of_hbm_peak": round(nb / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
        abi.free()
        # token-window batch gather from an HBM-resident stream: batch 512 x
        # 1024 windows of int64 (algorithmic 16 B per token position written,
        # 8 B read: x and y reads overlap)
        L.aar_token_windows_i64.argtypes = [vp, i64, vp, i64, i64, vp, vp, vp, vp]
        n_tok, bsz, T = 1 << 24, 512, 1024
        ptok = abi.put(rng.integers(0, 65, n_tok))
        pst = abi.put(rng.integers(0, n_tok - T - 1, bsz))
        px, py = abi.alloc(8 * bsz * T), abi.alloc(8 * bsz * T)
        ms = timed(lambda: L.aar_token_windows_i64(ptok, n_tok, pst, bsz, T, px, py, None, None))
        nb = 24 * bsz * T
        out["token_windows_512x1024"] = {"ms": round(ms, 4), "GB_s": round(nb / (ms * 1e-3) / 1e9, 1),
                                         "frac_of_hbm_peak": round(nb / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
        abi.free()
        for name, (op, Bn, M, N, K) in {"bmm_a_bt_96x1024x1024x64": (1, 96, 1024, 1024, 64),
                                        "bmm_8x2048x2048x2048": (0, 8, 2048, 2048, 2048)}.items():
            pa = abi.put(rng.standard_normal(Bn * M * K).astype(np.float32))
            pb = abi.put(rng.standard_normal(Bn * N * K).astype(np.float32))
            pc = abi.alloc(4 * Bn * M * N)
            ldb = K if op == 1 else N
            ms = timed(lambda: L.aar_gemm_f32_batched(op, Bn, M, N, K, pa, K, M * K, pb, ldb, N * K, pc, N, M * N,
                                                      None))
            tf = 2.0 * Bn * M * N * K / (ms * 1e-3) / 1e12
            out[name] = {"ms": round(ms, 4), "TFLOPS": round(tf, 2),
                         "pct_of_fp32_mfma_peak": round(100 * tf / PEAK_FP32_MFMA_TFLOPS, 2),
                         "min_hbm_GB_s": round(4 * Bn * (M * K + N * K + M * N) / (ms * 1e-3) / 1e9, 1)}
            abi.free()
    finally:
        abi.free()
    return out


def bench_copy(ev: Events, iters: int = 5, n: int = 1 << 26):
    """Calibration kernel for the HBM byte counters: c = a + b over n floats
    (reads 8n bytes, writes 4n bytes per launch)."""
    abi = Abi(ev.L)
    try:
        a = np.ones(n, np.float32)
        pa, pb, pc = abi.put(a), abi.put(a), abi.alloc(4 * n)
        for _ in range(2):
            ev.L.aar_add_f32(pa, pb, pc, n, None)
        ev.start()
        for _ in range(iters):
            assert ev.L.aar_add_f32(pa, pb, pc, n, None) == 0
        ms = ev.stop_ms() / iters
    finally:
        abi.free()
    return {"n": n, "read_bytes": 8 * n, "write_bytes": 4 * n, "ms": ms, "GB_s": 12 * n / (ms * 1e-3) / 1e9}


def bench_gemm_sweep(ev: Events, iters: int = 20):
    """BASELINE config 1 and 2 shapes and the reference bench's shapes in all
    three layouts through the C ABI (kernel-level timing of back-to-back
    launches, workspace preallocated)."""
    abi = Abi(ev.L)
    L = ev.L
    vp, i64, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t
    L.aar_gemm_f32.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, sz, vp]
    L.aar_gemm_f32_workspace_bytes.restype = sz
    L.aar_gemm_f32_workspace_bytes.argtypes = [ctypes.c_int, i64, i64, i64]
    shapes = [(1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096), (8192, 8192, 8192),
              (16384, 1536, 384), (16384, 384, 1536), (1536, 384, 16384), (384, 1536, 16384),
              (16384, 1152, 384), (16384, 65, 384), (1152, 384, 16384),
              # the rest of the reference bench's shapes (bench/bench_matmul.cu:150-167)
              (256, 256, 256), (512, 512, 512), (8192, 4096, 1024), (16384, 256, 256), (256, 16384, 256),
              (128, 4096, 4096)]
    out = {}
    rng = np.random.default_rng(0)
    try:
        for (M, N, K) in shapes:
            a = rng.standard_normal(max(M * K, 1)).astype(np.float32)
            b = rng.standard_normal(max(K * N, 1)).astype(np.float32)
            pa, pb, pc = abi.put(a), abi.put(b), abi.alloc(4 * M * N)
            for op, name in ((0, "nn"), (1, "nt"), (2, "tn")):
                wsb = L.aar_gemm_f32_workspace_bytes(op, M, N, K)
                ws = abi.alloc(wsb) if wsb else None
                flop = 2.0 * M * N * K
                n_it = iters if flop < 2e11 else max(3, iters // 4)
                # 30-40 ms of warm-up per layout so the clock has ramped before
                # timing (launches of a 1024^3 product take ~22 us each: a cap
                # of 200 left it timing the ramp)
                n_warm = int(min(2000, max(3, 4e12 / max(flop, 1.0))))
                for _ in range(n_warm):
                    assert L.aar_gemm_f32(op, M, N, K, pa, pb, pc, ws, wsb, None) == 0
                ev.start()
                for _ in range(n_it):
                    L.aar_gemm_f32(op, M, N, K, pa, pb, pc, ws, wsb, None)
                ms = ev.stop_ms() / n_it
                out[f"{name}_{M}x{N}x{K}"] = round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 2)
            abi.free()
    finally:
        abi.free()
    return out


# The reference bench's shapes, in its groups (bench/bench_matmul.cu:146-167),
# and its published rows for its shipping matmul kernel v4 (A = [M,K] times
# B = [K,N], i.e. our NN layout), NVIDIA A100 80GB PCIe, as (ms_med, TFLOPS)
# from bench/baselines/matmul_a100_80gb.csv (lines 7, 13, ..., 85: every sixth
# line from 7, in this order).  Other hardware: a reported yardstick only.
REF_SHAPES = [
    ("square", "sq256", 256, 256, 256), ("square", "sq512", 512, 512, 512),
    ("square", "sq1024", 1024, 1024, 1024), ("square", "sq2048", 2048, 2048, 2048),
    ("square", "sq4096", 4096, 4096, 4096), ("square", "sq8192", 8192, 8192, 8192),
    ("transformer", "qkv_proj", 16384, 1152, 384), ("transformer", "ffn_up", 16384, 1536, 384),
    ("transformer", "ffn_down", 16384, 384, 1536), ("transformer", "vocab_head", 16384, 65, 384),
    ("transformer", "big_ffn", 8192, 4096, 1024),
    ("skinny", "tall", 16384, 256, 256), ("skinny", "wide", 256, 16384, 256), ("skinny", "tiny_M", 128, 4096, 4096),
]
REF_A100_V4 = {
    "sq256": (0.0156, 2.15), "sq512": (0.0444, 6.05), "sq1024": (0.1867, 11.50), "sq2048": (1.3702, 12.54),
    "sq4096": (8.5775, 16.02), "sq8192": (63.7034, 17.26), "qkv_proj": (1.0287, 14.09), "ffn_up": (1.3594, 14.22),
    "ffn_down": (1.2375, 15.62), "vocab_head": (0.1452, 5.63), "big_ffn": (4.2348, 16.23), "tall": (0.1488, 14.44),
    "wide": (0.1478, 14.53), "tiny_M": (0.5338, 8.05),
}
LAYOUTS = {"nn": 0, "nt": 1, "tn": 2}


def _quantile(v, q):
    """The reference bench's quantile: the sorted sample at floor(n*q),
    clamped to the last (bench/bench_matmul.cu:60-64)."""
    v = sorted(v)
    return v[min(len(v) - 1, int(len(v) * q))]


def bench_reference_shapes(ev: Events, shapes, layouts=("nn", "nt", "tn"), warmup: int = 10, iters: int = 50,
                           seed: int = 0xC0FFEE, min_warm_ms: float = 30.0, csv_path=None, table=None):
    """The reference bench's GEMM protocol (bench/bench_matmul.cu:66-89,
    :203-274) through the C ABI: per shape, A and B uniform in [0, 1) from
    `seed`; per layout, `warmup` launches (and at least `min_warm_ms` of GPU
    time, so the clock has ramped), then `iters` launches each timed alone
    between two events with a synchronisation (median and p99 of those, the
    reference's figures), plus the back-to-back rate of `iters` pipelined
    launches.  The result is checked on sampled rows against float64 with
    the reference's tolerance max(2e-3, 5e-3*sqrt(K)/32) on the max abs
    error.  NN entries carry the reference's published A100 v4 figure."""
    abi = Abi(ev.L)
    L = ev.L
    vp, i64, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t
    L.aar_gemm_f32.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, sz, vp]
    L.aar_gemm_f32_workspace_bytes.restype = sz
    L.aar_gemm_f32_workspace_bytes.argtypes = [ctypes.c_int, i64, i64, i64]
    rng = np.random.default_rng(seed)
    check_rng = np.random.default_rng(seed + 1)
    gpu_name = device_name(L)
    out = {}
    csv_rows = []
    try:
        for group, tag, M, N, K in shapes:
            a = rng.random(M * K, dtype=np.float32)
            b = rng.random(K * N, dtype=np.float32)
            pa, pb, pc = abi.put(a), abi.put(b), abi.alloc(4 * M * N)
            flop = 2.0 * M * N * K
            for op in layouts:
                opi = LAYOUTS[op]
                wsb = L.aar_gemm_f32_workspace_bytes(opi, M, N, K)
                ws = abi.alloc(wsb) if wsb else None

                def call():
                    return L.aar_gemm_f32(opi, M, N, K, pa, pb, pc, ws, wsb, None)

                assert call() == 0
                L.aar_synchronize()
                rows = check_rng.choice(M, min(M, 16), replace=False)
                A = a.reshape(M, K) if op != "tn" else a.reshape(K, M).T
                B = b.reshape(K, N) if op != "nt" else b.reshape(N, K).T
                ref = A[rows].astype(np.float64) @ B.astype(np.float64)
                got = np.empty((len(rows), N), np.float32)
                for i, r in enumerate(rows):
                    assert L.aar_memcpy(got[i].ctypes.data, pc + 4 * int(r) * N, 4 * N, 2, None) == 0
                err = float(np.abs(got - ref).max())
                tol = max(2e-3, 5e-3 * np.sqrt(K) / 32.0)
                if not err <= tol:
                    raise SystemExit(f"bench: {op} {tag} check failed (max abs err {err:.3e} > {tol:.3e})")
                n_warm = int(max(warmup, min(5000, min_warm_ms * 1e-3 / max(flop / 150e12, 1e-7))))
                for _ in range(n_warm):
                    call()
                L.aar_synchronize()
                ts = []
                for _ in range(iters):
                    ev.start()
                    call()
                    ts.append(ev.stop_ms())
                ev.start()
                for _ in range(iters):
                    call()
                pipe = ev.stop_ms() / iters
                med, p99 = _quantile(ts, 0.5), _quantile(ts, 0.99)
                e = {"tag": tag, "M": M, "N": N, "K": K, "ms_med": round(med, 5), "ms_p99": round(p99, 5),
                     "tflops": round(flop / (med * 1e-3) / 1e12, 2),
                     "tflops_pipelined": round(flop / (pipe * 1e-3) / 1e12, 2), "max_abs_err": err}
                if op == "nn" and tag in REF_A100_V4:
                    pub = REF_A100_V4[tag][1]
                    e["a100_v4_published_tflops"] = pub
                    e["ratio_vs_a100_v4"] = round(e["tflops"] / pub, 2)
                out[f"{op}_{tag}"] = e
                csv_rows.append(f"{gpu_name},aar_{op},{tag},{M},{N},{K},{iters},{med:.4f},{p99:.4f},"
                                f"{e['tflops']:.2f},,,{err:.4g}")
                if table is not None:
                    pub = f"{e['ratio_vs_a100_v4']:9.2f}" if "ratio_vs_a100_v4" in e else f"{'-':>9s}"
                    print(f"{'aar_' + op:<14s} {tag:<12s} {M:6d} {N:6d} {K:6d} {med:10.4f} {p99:10.4f} "
                          f"{e['tflops']:9.2f} {e['tflops_pipelined']:9.2f} {pub}", file=table, flush=True)
            abi.free()
    finally:
        abi.free()
    if csv_path:
        path = Path(csv_path)
        if path.parent != Path(""):
            path.parent.mkdir(parents=True, exist_ok=True)
        new = not path.exists()
        with open(path, "a") as f:
            if new:
                f.write("gpu,kernel,tag,M,N,K,iters,ms_med,ms_p99,tflops,vs_sgemm_pct,vs_tf32_pct,max_abs_err\n")
            f.write("\n".join(csv_rows) + "\n")
    return out


def device_name(L) -> str:
    cu, clk, lds = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    arch = ctypes.create_string_buffer(64)
    L.aar_device_info.argtypes = [ctypes.POINTER(ctypes.c_int)] * 3 + [ctypes.c_char_p, ctypes.c_int]
    if L.aar_device_info(ctypes.byref(cu), ctypes.byref(clk), ctypes.byref(lds), arch, 64) != 0:
        return "AMD GPU"
    return f"AMD {arch.value.decode()} ({cu.value} CUs)"


# ----------------------------------------------------------------- GPT step
# decoder-only char GPT, 6 layers, d_model 384, 6 heads,
# context 256, batch 64, vocab 65, pre-LN, 4x ReLU MLP (biased), bias-free
# attention, final LN, bias-free head, mean cross entropy, SGD lr 1e-3;
# weights N(0, 0.02), LN gamma 1 / beta 0, biases 0; ids uniform in [0, 65).
GPT5 = dict(vocab=65, ctx=256, layers=6, d_model=384, heads=6, batch=64)


def gpt_param_shapes(vocab, ctx, layers, d_model, **_):
    """Parameter shapes in Module.parameters() order (tok_emb, pos_emb, then per
    block ln1 w/b, qkv W, out W, ln2 w/b, fc1 W/b, fc2 W/b; ln_f w/b; head W)."""
    d, f = d_model, 4 * d_model
    shapes = [("tok_emb", (vocab, d)), ("pos_emb", (ctx, d))]
    for i in range(layers):
        shapes += [(f"b{i}.ln1.w", (d,)), (f"b{i}.ln1.b", (d,)), (f"b{i}.qkv", (3 * d, d)),
                   (f"b{i}.out", (d, d)), (f"b{i}.ln2.w", (d,)), (f"b{i}.ln2.b", (d,)),
                   (f"b{i}.fc1.w", (f, d)), (f"b{i}.fc1.b", (f,)), (f"b{i}.fc2.w", (d, f)), (f"b{i}.fc2.b", (d,))]
    shapes += [("ln_f.w", (d,)), ("ln_f.b", (d,)), ("head", (vocab, d))]
    return shapes


def gpt_init_params(cfg, seed=0):
    rng = np.random.default_rng(seed)
    out = []
    for name, shape in gpt_param_shapes(**cfg):
        if name.endswith((".ln1.w", ".ln2.w")) or name == "ln_f.w":
            out.append(np.ones(shape, np.float32))
        elif name.endswith((".ln1.b", ".ln2.b", ".fc1.b", ".fc2.b")) or name == "ln_f.b":
            out.append(np.zeros(shape, np.float32))
        else:
            out.append((0.02 * rng.standard_normal(shape)).astype(np.float32))
    return out


def gpt_tokens(cfg, batch, seed=1):
    ids = np.random.default_rng(seed).integers(0, cfg["vocab"], (batch, cfg["ctx"] + 1)).astype(np.int64)
    return np.ascontiguousarray(ids[:, :-1]), np.ascontiguousarray(ids[:, 1:])


class GPT:
    """Config-5 GPT on aargrad (same composition as the reference's
    python/shakespeare/scripts/model.py with ReLU and no dropout)."""

    def __init__(self, ag, cfg, params):
        self.ag, self.cfg = ag, cfg
        self.p = []
        for arr in params:
            t = ag.from_numpy(arr).to(ag.Device.CUDA)
            t.requires_grad = True
            self.p.append(t)

    def forward(self, ids, pos):
        ag, c, p = self.ag, self.cfg, self.p
        B, T = ids.shape
        d, H = c["d_model"], c["heads"]
        # add(embedding(tok), embedding(pos)) as one lookup-and-add pass
        x = ag._core._embedding_add(p[0], ids, p[1], pos)
        for i in range(c["layers"]):
            (l1w, l1b, wqkv, wout, l2w, l2b, f1w, f1b, f2w, f2b) = p[2 + 10 * i: 12 + 10 * i]
            h = ag.layernorm(x, l1w, l1b, 1e-5)
            # nn.MultiHeadAttention's composition (per-head views of the packed
            # projection, causal flash attention, heads merged) as one fused op
            a = ag._core._flash_attention_qkv(ag.matmul_a_bt(h, wqkv), H, True)
            # x + out_proj(a), the residual add in the projection GEMM's epilogue
            x = ag._core._linear_residual(x, a, wout)
            h = ag.layernorm(x, l2w, l2b, 1e-5)
            # x + (the MLP linear -> relu -> linear, nn.Linear with bias) as one
            # fused op: bias and relu in the first GEMM's epilogue, the second
            # bias and the residual add in its GEMM's epilogue
            x = ag._core._mlp_relu_residual(x, h, f1w, f1b, f2w, f2b)
        x = ag.layernorm(x, p[-3], p[-2], 1e-5)
        return ag.matmul_a_bt(x, p[-1])

    def step(self, ids, pos, targets, lr):
        ag = self.ag
        logits = self.forward(ids, pos)
        B, T = ids.shape
        loss = ag.cross_entropy(ag.reshape(logits, [B * T, self.cfg["vocab"]]), targets, -100)
        for t in self.p:
            t.zero_grad()
        loss.backward()
        # SGD step as aargrad.optim.SGD takes it: one multi-tensor update
        ag._core._scaled_add_inplace_multi(self.p, [t.grad for t in self.p], -lr)
        return loss


def gpt_steps(ag, n: int = 5, cfg=GPT5):
    """n config-5 steps, each synchronised and logged, with no event timing:
    the mode counter passes (rocprofv3 --pmc) run, one line per step."""
    B, T = cfg["batch"], cfg["ctx"]
    model = GPT(ag, cfg, gpt_init_params(cfg))
    ids_np, tgt_np = gpt_tokens(cfg, B)
    ids = ag.from_numpy(ids_np).to(ag.Device.CUDA)
    tgt = ag.from_numpy(tgt_np.reshape(-1)).to(ag.Device.CUDA)
    pos = ag.from_numpy(np.tile(np.arange(T, dtype=np.int64), (B, 1))).to(ag.Device.CUDA)
    for i in range(n):
        t0 = time.time()
        model.step(ids, pos, tgt, 1e-3)
        ag.cuda_synchronize()
        log(f"gpt step {i}: {(time.time() - t0) * 1e3:.1f} ms (synchronised)")


def gpt_flops_per_step(cfg, batch):
    d, L, T, V, H = cfg["d_model"], cfg["layers"], cfg["ctx"], cfg["vocab"], cfg["heads"]
    linear_weights = L * (3 * d * d + d * d + 2 * 4 * d * d) + V * d
    gemm = 6.0 * linear_weights * batch * T
    attn = L * 7.0 * batch * H * T * T * (d // H)  # causal fwd (2) + bwd (5), halved by the mask
    return gemm + attn


def bench_gpt(ag, ev: Events, steps: int = 50, warmup: int = 10, cfg=GPT5):
    B, T = cfg["batch"], cfg["ctx"]
    params = gpt_init_params(cfg)
    model = GPT(ag, cfg, params)
    ids_np, tgt_np = gpt_tokens(cfg, B)
    ids = ag.from_numpy(ids_np).to(ag.Device.CUDA)
    tgt = ag.from_numpy(tgt_np.reshape(-1)).to(ag.Device.CUDA)
    pos = ag.from_numpy(np.tile(np.arange(T, dtype=np.int64), (B, 1))).to(ag.Device.CUDA)
    for _ in range(warmup):
        model.step(ids, pos, tgt, 1e-3)
    ag.cuda_synchronize()
    st = StepTimer(ev, steps)
    st.mark()
    for _ in range(steps):
        loss = model.step(ids, pos, tgt, 1e-3)
        st.mark()
    ag.cuda_synchronize()
    ms, dist = st.result()
    ms /= steps
    last = float(ag.to_numpy(loss.to(ag.Device.CPU)))
    tokens = B * T
    return {"tokens_per_s": round(tokens / (ms * 1e-3), 1), "ms_per_step": round(ms, 3), "steps": steps,
            "step_ms_median": dist["median_ms"], "step_ms_p99": dist["p99_ms"],
            "implied_tflops": round(gpt_flops_per_step(cfg, B) / (ms * 1e-3) / 1e12, 2),
            "loss_after_steps": round(last, 5), "batch": B, "ctx": T,
            "config": "6 layers, d_model 384, 6 heads, ctx 256, batch 64, vocab 65, ReLU MLP, SGD lr 1e-3"}


def cpu_pin():
    """Pin the calling thread (the one that runs the reference CPU code) to one
    host core: the last core this process may use.  Returns (core, cores the
    process may use, previous affinity)."""
    allowed = sorted(os.sched_getaffinity(0))
    core = allowed[-1]
    os.sched_setaffinity(0, {core})
    return core, len(allowed), set(allowed)


def cpu_host_note(core: int, n_allowed: int) -> str:
    return f"host {cpu_model()}, nproc {os.cpu_count()} ({n_allowed} usable), pinned to core {core}"


def cpu_baseline_gpt(cfg=GPT5, batch: int = 2):
    """The reference's own CPU GPT step (oracle/_ref, built from its sources)
    on one core at a reduced batch: tokens/s = batch*ctx / t_step."""
    import oracle

    if not oracle.ref_available():
        return None
    params = gpt_init_params(cfg)
    ids, tgt = gpt_tokens(cfg, batch)
    t0 = time.perf_counter()
    oracle.ref_gpt_step(cfg, params, ids, tgt, 1e-3)
    t = time.perf_counter() - t0
    return {"tokens_per_s": round(batch * cfg["ctx"] / t, 2), "s_per_step": round(t, 2), "batch": batch,
            "cores": 1, "kind": "reference"}


def cpu_baseline_matmul(ab, budget_s: float = 12.0):
    """The reference CPU path (oracle/_ref: the reference's own matmul built
    from its sources; else the C restatement) on one core, on a row band of
    the same 4096^3 product, extrapolated to the full product."""
    import oracle

    a, b = ab
    n = a.shape[0]
    use_ref = oracle.ref_available()
    kind = "reference" if use_ref else "port"

    def run(rows):
        if use_ref:
            oracle.ref_matmul("nn", np.ascontiguousarray(a[:rows]), b)
        else:
            oracle.matmul("nn", a, b, rows=(0, rows))

    run(2)  # warm caches / page in
    t0 = time.perf_counter()
    run(4)
    per_row = (time.perf_counter() - t0) / 4
    rows = int(max(8, min(n, budget_s / max(per_row, 1e-6))))
    t0 = time.perf_counter()
    run(rows)
    t = time.perf_counter() - t0
    tflops = 2.0 * rows * n * n / t / 1e12
    return {
        "value": tflops,
        "unit": "TFLOPS",
        "cores": 1,
        "kind": kind,
        "sample": f"{rows}-row band of the 4096^3 fp32 matmul (naive i-j-k reference loop, {t:.1f} s; "
                  f"full product extrapolates to {t * n / rows:.0f} s)",
    }


def _ratio(cpu_ms, gpu_ms):
    return round(cpu_ms / gpu_ms, 1) if gpu_ms else None


def cpu_baselines_configs(sweep, rowwise, flash):
    """The reference's own CPU path (oracle/_ref) for BASELINE configs 1, 3 and
    4 on one pinned core, beside the GPU figures of the same run.
      config 1: matmul / matmul_a_bt / matmul_at_b at 1024^3, in full
                (cppsrc/ops/matmul.cpp:24-91);
      config 3: softmax and layernorm fwd and fwd+bwd (autograd) at
                rows 65536 x cols 384/768 in full; cols 4096 on an 8192-row
                band x 8, labelled extrapolated (softmax.cpp:15-63,
                layernorm.cpp:20-157);
      config 4: the causal attention composite fwd+bwd (flash_attention.cpp:
                40-45 with bmm/scale/mask/softmax and autograd) on (b,h)
                slices, x 96 slices, labelled extrapolated: 2 slices at
                T=1024, 1 at T=4096.
    Each reference call includes copying its inputs into reference Tensors
    and its outputs out (memcpy-rate work, small beside the arithmetic).
    The backward figures are fwd+bwd time minus the forward time."""
    import oracle

    if not oracle.ref_available():
        return None
    rng = np.random.default_rng(0)
    out = {}
    # config 1
    a = rng.standard_normal((1024, 1024)).astype(np.float32)
    b = rng.standard_normal((1024, 1024)).astype(np.float32)
    c1 = {}
    for op in ("nn", "nt", "tn"):
        t0 = time.perf_counter()
        oracle.ref_matmul(op, a, b)
        t = time.perf_counter() - t0
        gpu_tf = sweep.get(f"{op}_1024x1024x1024")
        gpu_ms = 2.0 * 1024 ** 3 / (gpu_tf * 1e12) * 1e3 if gpu_tf else None
        c1[op] = {"cpu_ms": round(t * 1e3, 1), "cpu_GFLOPS": round(2.0 * 1024 ** 3 / t / 1e9, 3),
                  "gpu_ms": round(gpu_ms, 4) if gpu_ms else None, "gpu_over_cpu": _ratio(t * 1e3, gpu_ms)}
    out["config1_gemm_1024"] = c1
    # config 3
    rows = 65536
    c3 = {}
    for cols in (384, 768, 4096):
        band = rows if cols < 4096 else 8192
        x = (3 * rng.standard_normal((band, cols))).astype(np.float32)
        w = (1 + 0.02 * rng.standard_normal(cols)).astype(np.float32)
        bb = (0.02 * rng.standard_normal(cols)).astype(np.float32)
        g = rng.standard_normal((band, cols)).astype(np.float32)
        calls = {"softmax_fwd": lambda: oracle.ref_softmax(x),
                 "softmax_bwd": lambda: oracle.ref_softmax(x, g),
                 "layernorm_fwd": lambda: oracle.ref_layernorm(x, w, bb),
                 "layernorm_bwd": lambda: oracle.ref_layernorm(x, w, bb, 1e-5, g)}
        tm = {}
        for name, fn in calls.items():  # best of two (the first run also faults in fresh pages)
            best = None
            for _ in range(2):
                t0 = time.perf_counter()
                fn()
                t = time.perf_counter() - t0
                best = t if best is None else min(best, t)
            tm[name] = best
        tm["softmax_bwd"] = max(tm["softmax_bwd"] - tm["softmax_fwd"], 1e-9)
        tm["layernorm_bwd"] = max(tm["layernorm_bwd"] - tm["layernorm_fwd"], 1e-9)
        nbytes = {"softmax_fwd": 8.0 * rows * cols, "softmax_bwd": 12.0 * rows * cols,
                  "layernorm_fwd": 8.0 * rows * cols + 8 * cols + 8 * rows,
                  "layernorm_bwd": 12.0 * rows * cols + 12 * cols + 8 * rows}
        for name, t in tm.items():
            t_full = t * rows / band
            gpu_ms = rowwise.get(f"{name}_c{cols}", {}).get("ms")
            c3[f"{name}_c{cols}"] = {"cpu_ms": round(t_full * 1e3, 1),
                                     "cpu_GB_s": round(nbytes[name] / t_full / 1e9, 3),
                                     "gpu_ms": gpu_ms, "gpu_over_cpu": _ratio(t_full * 1e3, gpu_ms),
                                     "sample": "full" if band == rows else f"{band}-row band x {rows // band}, extrapolated"}
    out["config3_rowwise_65536"] = c3
    # config 4
    c4 = {}
    for T, n_sl in ((1024, 2), (4096, 1)):
        q, k, v, do = (rng.standard_normal((n_sl, T, 64)).astype(np.float32) for _ in range(4))
        t0 = time.perf_counter()
        oracle.ref_attention(q, k, v, True, do)
        t = (time.perf_counter() - t0) * 96 / n_sl
        flops = 3.5 * 4.0 * 96 * T * T * 64 / 2.0
        gpu_ms = flash.get(T)
        c4[f"t{T}"] = {"cpu_ms": round(t * 1e3, 1), "cpu_GFLOPS": round(flops / t / 1e9, 3),
                       "gpu_ms": gpu_ms, "gpu_over_cpu": _ratio(t * 1e3, gpu_ms),
                       "sample": f"{n_sl} of 96 (b,h) slices x {96 // n_sl}, extrapolated",
                       "flops": "3.5 * 4*B*H*T^2*d/2 (algorithmic, causal)"}
    out["config4_flash_b8h12d64"] = c4
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=60)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--flash-steps", type=int, default=50)
    ap.add_argument("--flash-t", type=int, default=4096, choices=[256, 1024, 4096],
                    help="sequence length of the --only flash run (BASELINE config 4 has 1024 and 4096 at "
                         "B8 H12; 256 is config 5's attention, B64 H6)")
    ap.add_argument("--only", choices=["all", "gemm", "flash", "rowwise", "extra", "copy", "gpt", "gpt-steps", "sweep"],
                    default="all",
                    help="run one part (profiling runs); the JSON line is printed for 'all'")
    # The reference bench's command line (bench/bench_matmul.cu:101-136): with
    # --shape or --shapes, run its GEMM table protocol only, print the table
    # and, with --csv, append rows in its CSV format.
    ap.add_argument("--shape", default=None, help="one GEMM shape MxNxK (reference bench protocol)")
    ap.add_argument("--shapes", default=None, choices=["all", "square", "transformer", "skinny"],
                    help="a group of the reference bench's shapes (reference bench protocol)")
    ap.add_argument("--iters", type=int, default=50, help="timed launches per shape and layout (table mode)")
    ap.add_argument("--seed", type=lambda v: int(v, 0), default=0xC0FFEE, help="input seed (table mode)")
    ap.add_argument("--csv", default=None, help="append the table's rows to this CSV (table mode)")
    ap.add_argument("--kernel", default="all", choices=["all", "nn", "nt", "tn"],
                    help="layout(s) to time in table mode: nn = matmul, nt = matmul_a_bt, tn = matmul_at_b")
    args = ap.parse_args()
    warmup_given = any(a == "--warmup" or a.startswith("--warmup=") for a in sys.argv[1:])
    if args.gpus != 1:
        print(f"bench.py: this build targets one GPU; --gpus {args.gpus} is not supported "
              "(every kernel here runs on one GPU's share; no collectives are built)", file=sys.stderr)
        return 2

    import aargrad as ag

    if not ag.device_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    ev = Events()
    n = 4096
    flops = 2.0 * n ** 3

    if args.shape or args.shapes:
        if args.shape:
            try:
                M, N, K = (int(t) for t in args.shape.lower().split("x"))
            except ValueError:
                print(f"bad shape {args.shape} (want MxNxK)", file=sys.stderr)
                return 1
            shapes = [("single", "custom", M, N, K)]
        else:
            shapes = [s for s in REF_SHAPES if args.shapes in ("all", s[0])]
        layouts = ("nn", "nt", "tn") if args.kernel == "all" else (args.kernel,)
        print(f"# GPU={device_name(ev.L)} iters={args.iters} warmup={args.warmup if warmup_given else 10} "
              f"seed={args.seed:#x}")
        print(f"{'kernel':<14s} {'tag':<12s} {'M':>6s} {'N':>6s} {'K':>6s} {'ms_med':>10s} {'ms_p99':>10s} "
              f"{'TFLOPS':>9s} {'TF_pipe':>9s} {'vs_A100v4':>9s}", flush=True)
        res = bench_reference_shapes(ev, shapes, layouts, warmup=args.warmup if warmup_given else 10,
                                     iters=args.iters, seed=args.seed, csv_path=args.csv, table=sys.stdout)
        log(json.dumps(res))
        return 0

    if args.only == "copy":
        log("copy calibration:", bench_copy(ev))
        return 0
    if args.only == "rowwise":
        log(json.dumps(bench_rowwise(ev)))
        return 0
    if args.only == "extra":
        log(json.dumps(bench_extra(ev)))
        return 0
    if args.only == "sweep":
        log(json.dumps(bench_gemm_sweep(ev)))
        return 0
    if args.only == "gpt-steps":
        gpt_steps(ag)
        return 0
    if args.only == "gpt":
        log(json.dumps(bench_gpt(ag, ev)))
        return 0
    if args.only == "flash":
        bh = (64, 6) if args.flash_t == 256 else (8, 12)
        fa_ms, fa_flops, fa_dist = bench_flash(ag, args.flash_steps, 10, ev, T=args.flash_t, B=bh[0], H=bh[1])
        log(f"flash T={args.flash_t} fwd+bwd {fa_ms:.3f} ms {fa_flops / (fa_ms * 1e-3) / 1e12:.2f} TFLOPS {fa_dist}")
        return 0

    if args.only == "gemm":
        step_ms, wall, err, ab, mm_dist = bench_matmul(ag, args.steps, args.warmup, ev)
        tflops = flops / (step_ms * 1e-3) / 1e12
        log(f"matmul 4096^3: {step_ms:.4f} ms/step, {tflops:.2f} TFLOPS")
        return 0

    # The other GPU legs run first, so the headline's W warm-up steps start on
    # a GPU whose clocks have already ramped; its operands are uploaded before
    # them, so no host-to-device copy idles the GPU right before it.
    mm_inputs = matmul_inputs(ag)
    fa_ms, fa_flops, fa_dist = bench_flash(ag, args.flash_steps, 10, ev)
    fa_tflops = fa_flops / (fa_ms * 1e-3) / 1e12
    log(f"flash causal B8 H12 T4096 d64 fwd+bwd: {fa_ms:.3f} ms, {fa_tflops:.2f} TFLOPS "
        f"({100 * fa_tflops / PEAK_FP32_MFMA_TFLOPS:.1f}%)")
    fa1_ms, fa1_flops, fa1_dist = bench_flash(ag, args.flash_steps, 10, ev, T=1024)
    fa1_tflops = fa1_flops / (fa1_ms * 1e-3) / 1e12
    log(f"flash causal B8 H12 T1024 d64 fwd+bwd: {fa1_ms:.3f} ms, {fa1_tflops:.2f} TFLOPS "
        f"({100 * fa1_tflops / PEAK_FP32_MFMA_TFLOPS:.1f}%)")

    fa5_ms, fa5_flops, fa5_dist = bench_flash(ag, args.flash_steps, 10, ev, T=256, B=64, H=6)
    fa5_tflops = fa5_flops / (fa5_ms * 1e-3) / 1e12
    log(f"flash causal B64 H6 T256 d64 (config 5 attention) fwd+bwd: {fa5_ms:.4f} ms, {fa5_tflops:.2f} TFLOPS "
        f"({100 * fa5_tflops / PEAK_FP32_MFMA_TFLOPS:.1f}%)")

    sweep = bench_gemm_sweep(ev)
    log("GEMM sweep TFLOPS: " + ", ".join(f"{k} {v}" for k, v in sweep.items()))

    ref_table = bench_reference_shapes(ev, REF_SHAPES)
    log("reference bench shapes (its protocol: median of single timed launches), TFLOPS: " +
        ", ".join(f"{k} {v['tflops']}" + (f" ({v['ratio_vs_a100_v4']}x A100 v4)" if "ratio_vs_a100_v4" in v else "")
                  for k, v in ref_table.items()))

    rowwise = bench_rowwise(ev)
    for k, v in rowwise.items():
        log(f"{k}: {v['GB_s']} GB/s ({100 * v['frac_of_hbm_peak']:.1f}% of HBM peak)")

    extra = bench_extra(ev)
    for k, v in extra.items():
        log(f"{k}: " + ", ".join(f"{a} {b}" for a, b in v.items()))

    gpt = bench_gpt(ag, ev)
    log(f"GPT step (config 5): {gpt['tokens_per_s']:.0f} tokens/s, {gpt['ms_per_step']} ms/step, "
        f"{gpt['implied_tflops']} TFLOPS implied")

    step_ms, wall, err, ab, mm_dist = bench_matmul(ag, args.steps, args.warmup, ev, mm_inputs)
    tflops = flops / (step_ms * 1e-3) / 1e12
    log(f"matmul 4096^3: {step_ms:.4f} ms/step, {tflops:.2f} TFLOPS "
        f"({100 * tflops / PEAK_FP32_MFMA_TFLOPS:.1f}% of fp32 MFMA peak), check err {err:.2e}")
    ag.cuda_synchronize()

    # Reference CPU legs, after all GPU work, on one pinned host core.
    cpu = None
    cpu_configs = None
    if not args.no_cpu_baseline:
        core, n_allowed, prev = cpu_pin()
        try:
            note = cpu_host_note(core, n_allowed)
            cpu = cpu_baseline_matmul(ab)
            cpu["sample"] += "; " + note
            log(f"cpu baseline ({cpu['kind']}): {cpu['value'] * 1e3:.3f} GFLOPS on 1 core ({note})")
            gpt["cpu_baseline"] = cpu_baseline_gpt()
            if gpt["cpu_baseline"]:
                gpt["cpu_baseline"]["host"] = note
                log(f"GPT step reference CPU (batch 2, 1 core): {gpt['cpu_baseline']['tokens_per_s']} tokens/s")
            cpu_configs = cpu_baselines_configs(sweep, rowwise, {4096: round(fa_ms, 4), 1024: round(fa1_ms, 4)})
            if cpu_configs is not None:
                cpu_configs["host"] = note
                cpu_configs["kind"] = "reference"
                cpu_configs["cores"] = 1
                log("reference CPU per config: " + json.dumps(cpu_configs))
        finally:
            os.sched_setaffinity(0, prev)

    out = {
        "metric": "fp32 matmul TFLOPS @4096^3 (% of FP32 MFMA peak) + flash-attn fwd+bwd TFLOPS",
        "value": round(tflops, 3),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "ms_per_step_median": mm_dist["median_ms"],
        "ms_per_step_p99": mm_dist["p99_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(tflops / REF_PUBLISHED_TFLOPS, 3),
        "baseline": {"value": REF_PUBLISHED_TFLOPS, "unit": "TFLOPS",
                     "source": "reference matmul_tiled_kernel_v4, M=N=K=4096, NVIDIA A100 80GB PCIe "
                               "(bench/baselines/matmul_a100_80gb.csv:31); other hardware"},
        "dtype": "f32",
        "data": "synthetic (A, B ~ N(0,1)/sqrt(K) from seed 0, resident in HBM)",
        "config": {
            "workload": "fp32 matmul C=A.B, M=N=K=4096 (BASELINE config 2 square point)",
            "op": "matmul (NN)",
            "M": n, "N": n, "K": n,
            "flops_per_step": flops,
        },
        "pct_of_fp32_mfma_peak": round(100 * tflops / PEAK_FP32_MFMA_TFLOPS, 2),
        "flash_attn_fwd_bwd": {
            "tflops": round(fa_tflops, 3),
            "pct_of_fp32_mfma_peak": round(100 * fa_tflops / PEAK_FP32_MFMA_TFLOPS, 2),
            "ms_per_step": round(fa_ms, 4),
            "steps": args.flash_steps,
            "ms_per_step_median": fa_dist["median_ms"],
            "ms_per_step_p99": fa_dist["p99_ms"],
            "config": "causal, B8 H12 T4096 d64, fwd+bwd, flops = 3.5 * 4*B*H*T^2*d/2",
        },
        "flash_attn_fwd_bwd_t1024": {
            "tflops": round(fa1_tflops, 3),
            "pct_of_fp32_mfma_peak": round(100 * fa1_tflops / PEAK_FP32_MFMA_TFLOPS, 2),
            "ms_per_step": round(fa1_ms, 4),
            "ms_per_step_median": fa1_dist["median_ms"],
            "ms_per_step_p99": fa1_dist["p99_ms"],
            "config": "causal, B8 H12 T1024 d64, fwd+bwd",
        },
        "flash_attn_fwd_bwd_config5_t256": {
            "tflops": round(fa5_tflops, 3),
            "pct_of_fp32_mfma_peak": round(100 * fa5_tflops / PEAK_FP32_MFMA_TFLOPS, 2),
            "ms_per_step": round(fa5_ms, 4),
            "ms_per_step_median": fa5_dist["median_ms"],
            "ms_per_step_p99": fa5_dist["p99_ms"],
            "config": "causal, B64 H6 T256 d64 (one GPT-step layer's attention), fwd+bwd",
        },
        "gemm_sweep_tflops": sweep,
        "gemm_reference_bench_table": ref_table,
        "rowwise_hbm": rowwise,
        "attention_ops_and_dropout": extra,
        "gpt_train_step": gpt,
        "cpu_baselines_per_config": cpu_configs,
        "roofline": {
            "bound": "mfma",
            "achieved": round(tflops, 3),
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / PEAK_FP32_MFMA_TFLOPS, 4),
            "traffic": load_traffic("gemm_f32_nn_4096"),
            "traffic_counts": "L2-to-fabric bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated); "
                              "HBM bytes proper are not counted separately",
            "kernel": "gemm_f32_dma_kernel<256, 256, 32, 64, 128, 2, 2, true, false, 0, 1> (NN, plain epilogue; "
                      "one launch per step)",
            "algorithmic_flops_per_launch": flops,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
