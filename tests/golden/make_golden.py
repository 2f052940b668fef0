"""Writes tests/golden/*.npz: input/output vectors produced by the reference's
own CPU implementation (AARONKANG04/aar-vlm cppsrc/, compiled from its sources
into oracle/_ref/libaar_ref.so by oracle/Makefile).

Run in the container that holds the reference tree:
    make -C oracle && python tests/golden/make_golden.py

Inputs follow the reference tests' deterministic fills where they have one:
  gemm       64x96x48, a = i*0.013 - 0.4, b = i*0.007 + 0.1
             (tests/cpp/test_matmul.cpp:119-140), all three layouts
  softmax    32x257, x = sin(i*0.13)*5 + (i%7)*0.5 (tests/cpp/test_softmax.cpp:76-82),
             upstream grad from default_rng(1)
  layernorm  32x257, same x, w = 1 + 0.1 cos(0.2 j), b = 0.05 j
             (tests/cpp/test_layernorm.cpp:118-132), upstream grad default_rng(2)
  attention  B2 H4 T64 d16 from default_rng(11) (tests/python/test_flash_attention.py:80-87),
             causal and not, upstream grad default_rng(12)
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

import oracle  # noqa: E402


def main() -> None:
    if not oracle.ref_available():
        raise SystemExit("oracle/_ref/libaar_ref.so is not built (needs the reference tree)")
    f32 = np.float32
    i = np.arange(64 * 96, dtype=f32)
    a_fill = i * f32(0.013) - f32(0.4)
    j = np.arange(96 * 48, dtype=f32)
    b_fill = j * f32(0.007) + f32(0.1)
    out = {}
    # nn: A[64,96] B[96,48]; nt: A[64,96] B[48,96]; tn: A[96,64] B[96,48]
    out["nn_a"], out["nn_b"] = a_fill.reshape(64, 96), b_fill.reshape(96, 48)
    out["nt_a"], out["nt_b"] = a_fill.reshape(64, 96), b_fill.reshape(48, 96)
    out["tn_a"], out["tn_b"] = a_fill.reshape(96, 64), b_fill.reshape(96, 48)
    for op in oracle.OPS:
        out[f"{op}_c"] = oracle.ref_matmul(op, out[f"{op}_a"], out[f"{op}_b"])
    np.savez(HERE / "gemm_64x96x48.npz", **out)

    k = np.arange(32 * 257, dtype=f32)
    x = (np.sin(k * f32(0.13)) * f32(5.0) + (np.arange(32 * 257) % 7).astype(f32) * f32(0.5)).astype(f32)
    x = x.reshape(32, 257)
    g = np.random.default_rng(1).standard_normal((32, 257)).astype(f32)
    y, dx = oracle.ref_softmax(x, g)
    np.savez(HERE / "softmax_32x257.npz", x=x, g=g, y=y, dx=dx)

    col = np.arange(257, dtype=f32)
    w = (f32(1.0) + f32(0.1) * np.cos(col * f32(0.2))).astype(f32)
    b = (f32(0.05) * col).astype(f32)
    gy = np.random.default_rng(2).standard_normal((32, 257)).astype(f32)
    y, dx, dw, db = oracle.ref_layernorm(x, w, b, 1e-5, gy)
    np.savez(HERE / "layernorm_32x257.npz", x=x, w=w, b=b, gy=gy, y=y, dx=dx, dw=dw, db=db, eps=np.float32(1e-5))

    rng = np.random.default_rng(11)
    q = rng.standard_normal((2, 4, 64, 16)).astype(f32)
    kk = rng.standard_normal((2, 4, 64, 16)).astype(f32)
    v = rng.standard_normal((2, 4, 64, 16)).astype(f32)
    do = np.random.default_rng(12).standard_normal((2, 4, 64, 16)).astype(f32)
    att = {"q": q, "k": kk, "v": v, "do": do}
    for causal in (0, 1):
        o, dq, dk, dv = oracle.ref_attention(q, kk, v, causal, do)
        att.update({f"o_{causal}": o, f"dq_{causal}": dq, f"dk_{causal}": dk, f"dv_{causal}": dv})
    np.savez(HERE / "attention_b2h4t64d16.npz", **att)
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
