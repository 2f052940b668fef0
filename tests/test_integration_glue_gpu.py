"""The reference's own C++ running on the MI355X kernels.

oracle/_ref/libaar_glue.so is the reference's CPU sources (its Tensor,
autograd, ops frontends and optimizer steps) with its device entry points bound
to libaar_hip.so by oracle/hip_backend.cpp, the glue a maintainer adds to the
reference.  Inside ``oracle.reference_on_device()`` the ``ref_*`` wrappers run
that build with every operand on Device::CUDA; each result is compared with the
same call on the reference's CPU build (oracle/_ref/libaar_ref.so).

Tolerances: a GEMM output of contraction length K within 1e-4*sqrt(K); softmax,
layernorm and attention outputs and gradients within 1e-4; a parameter update
of a training step, a GEMM gradient over the B*T tokens, within
1e-4*sqrt(B*T).  Elementwise ops, the fan-in gradient sums of the reference's
autograd, dropout and the causal mask are bit-identical.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from conftest import TOL, assert_close, gemm_tol

sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
import bench  # noqa: E402  (the config-5 workload definition lives with the benchmark)

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not (O.glue_available() and O.ref_available()),
                                 reason="oracle/_ref glue or reference build absent (no reference tree at build time)")]
f32 = np.float32


def on_device(fn, *args, **kw):
    with O.reference_on_device():
        return fn(*args, **kw)


@pytest.mark.parametrize("op", ["nn", "nt", "tn"])
@pytest.mark.parametrize("M,N,K", [(131, 77, 96), (512, 1152, 384)])
def test_glue_matmul(gpu, op, M, N, K):
    rng = np.random.default_rng(M + N + K)
    a = rng.standard_normal((M, K) if op != "tn" else (K, M)).astype(f32)
    b = rng.standard_normal((K, N) if op != "nt" else (N, K)).astype(f32)
    assert_close(on_device(O.ref_matmul, op, a, b), O.ref_matmul(op, a, b), gemm_tol(K), f"matmul {op}")


def test_glue_softmax_and_layernorm(gpu):
    rng = np.random.default_rng(1)
    x = (3 * rng.standard_normal((257, 384))).astype(f32)
    g = rng.standard_normal(x.shape).astype(f32)
    for got, ref, name in zip(on_device(O.ref_softmax, x, g), O.ref_softmax(x, g), ("y", "dx")):
        assert_close(got, ref, TOL, f"softmax {name}")
    w = (1 + 0.1 * rng.standard_normal(384)).astype(f32)
    b = (0.1 * rng.standard_normal(384)).astype(f32)
    for got, ref, name in zip(on_device(O.ref_layernorm, x, w, b, 1e-5, g), O.ref_layernorm(x, w, b, 1e-5, g),
                              ("y", "dx", "dw", "db")):
        assert_close(got, ref, TOL if name in ("y", "dx") else gemm_tol(x.shape[0]), f"layernorm {name}")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("bh,T,d", [(6, 256, 64), (3, 100, 32)])
def test_glue_flash_attention(gpu, causal, bh, T, d):
    rng = np.random.default_rng(T + d + causal)
    q, k, v, do = (rng.standard_normal((bh, T, d)).astype(f32) for _ in range(4))
    got = on_device(O.ref_attention, q, k, v, causal, do)
    ref = O.ref_attention(q, k, v, causal, do)
    for g, r, name in zip(got, ref, ("o", "dq", "dk", "dv")):
        assert_close(g, r, TOL, f"attention {name}")


def test_glue_autograd_fanin_is_bit_identical(gpu):
    rng = np.random.default_rng(3)
    n = 4099
    x, g = rng.standard_normal(n).astype(f32), rng.standard_normal(n).astype(f32)
    w = rng.standard_normal((4, n)).astype(f32)
    assert np.array_equal(on_device(O.ref_fanin_graph, x, w, g), O.ref_fanin_graph(x, w, g))


def test_glue_step_ops(gpu):
    rng = np.random.default_rng(4)
    a, b, g = (rng.standard_normal(3001).astype(f32) for _ in range(3))
    for op in ("sub", "mul", "relu"):
        for got, ref in zip(on_device(O.ref_elementwise, op, a, b, 0.0, g), O.ref_elementwise(op, a, b, 0.0, g)):
            assert np.array_equal(got, ref), op
    for got, ref in zip(on_device(O.ref_elementwise, "gelu", a, None, 0.0, g), O.ref_elementwise("gelu", a, None, 0.0, g)):
        assert_close(got, ref, 1e-6, "gelu")
    x = rng.standard_normal((300, 96)).astype(f32)
    bias = rng.standard_normal(96).astype(f32)
    gy = rng.standard_normal(x.shape).astype(f32)
    y, db = on_device(O.ref_add_bias, x, bias, gy)
    y_ref, db_ref = O.ref_add_bias(x, bias, gy)
    assert np.array_equal(y, y_ref)
    assert_close(db, db_ref, gemm_tol(300), "bias grad")
    assert abs(on_device(O.ref_sum_all, a) - O.ref_sum_all(a)) <= 1e-4 * max(1.0, float(np.abs(a).sum()))
    ids = rng.integers(0, 65, 500)
    w = rng.standard_normal((65, 48)).astype(f32)
    ge = rng.standard_normal((500, 48)).astype(f32)
    ye, dwe = on_device(O.ref_embedding, w, ids, ge)
    ye_ref, dwe_ref = O.ref_embedding(w, ids, ge)
    assert np.array_equal(ye, ye_ref)
    assert_close(dwe, dwe_ref, gemm_tol(500), "embedding grad")
    logits = rng.standard_normal((500, 65)).astype(f32)
    tgt = rng.integers(0, 65, 500)
    tgt[::7] = -100
    loss, dl = on_device(O.ref_cross_entropy, logits, tgt, -100, 1.0)
    loss_ref, dl_ref = O.ref_cross_entropy(logits, tgt, -100, 1.0)
    assert abs(loss - loss_ref) <= 1e-5 * max(1.0, abs(loss_ref))
    assert_close(dl, dl_ref, TOL, "cross entropy grad")
    y, dx = on_device(O.ref_dropout, a, 0.1, 77, True)
    y_ref, dx_ref = O.ref_dropout(a, 0.1, 77, True)
    assert np.array_equal(y, y_ref) and np.array_equal(dx, dx_ref)
    s = rng.standard_normal((4, 33, 33)).astype(f32)
    gs = rng.standard_normal(s.shape).astype(f32)
    for got, ref in zip(on_device(O.ref_causal_mask, s, gs), O.ref_causal_mask(s, gs)):
        assert np.array_equal(got, ref)
    for op in ("bmm", "bmm_a_bt", "bmm_at_b"):
        A = rng.standard_normal((5, 40, 24)).astype(f32)
        B = rng.standard_normal((5, 24, 31) if op == "bmm" else (5, 31, 24) if op == "bmm_a_bt" else (5, 40, 31)
                                ).astype(f32)
        assert_close(on_device(O.ref_bmm, op, A, B), O.ref_bmm(op, A, B), gemm_tol(40), op)
    p, m, v = (rng.standard_normal(1000).astype(f32) for _ in range(3))
    v = np.abs(v)
    gp = rng.standard_normal(1000).astype(f32)
    args = (3e-4, 0.9, 0.95, 1e-8, 0.01, 0.1, 0.0975)
    for got, ref in zip(on_device(O.ref_adamw, p, gp, m, v, *args), O.ref_adamw(p, gp, m, v, *args)):
        assert_close(got, ref, 1e-6, "adamw")


def test_glue_gpt_step_at_config5_shape(gpu):
    """The reference's own SGD step of the config-5 GPT (6 layers, d_model 384,
    6 heads, ctx 256, vocab 65), batch 2, on the device through the glue.

    It is bit-identical to aargrad's own step (bench.GPT) on the same kernels:
    binding the reference's C++ to libaar_hip.so changes no result.  Against
    the reference CPU step it agrees to the tolerance at these seeds.  At some
    seeds (8 and 9, for one) a ReLU input of block 0 rounds to opposite sides of
    zero on the CPU and GPU paths, which flips one hidden unit's gradient; that
    discrete difference is outside what a rounding tolerance covers, so the CPU
    comparison uses seeds without such a tie (those of the config-5 SGD test)."""
    ag = gpu
    cfg = dict(bench.GPT5, batch=2)
    params = bench.gpt_init_params(cfg, seed=11)
    ids, tgt = bench.gpt_tokens(cfg, cfg["batch"], seed=12)
    lr = 1.0  # p_new = p - g: the parameter deltas are the gradients
    loss, new = on_device(O.ref_gpt_step, cfg, params, ids, tgt, lr)

    model = bench.GPT(ag, cfg, params)
    B, T = ids.shape
    tids = ag.from_numpy(ids).to(ag.Device.CUDA)
    pos = ag.from_numpy(np.tile(np.arange(T, dtype=np.int64), (B, 1))).to(ag.Device.CUDA)
    ttgt = ag.from_numpy(np.ascontiguousarray(tgt.reshape(-1))).to(ag.Device.CUDA)
    loss_own = float(ag.to_numpy(model.step(tids, pos, ttgt, lr).to(ag.Device.CPU)))
    assert loss == loss_own
    for i, (name, _) in enumerate(bench.gpt_param_shapes(**cfg)):
        assert np.array_equal(new[i], ag.to_numpy(model.p[i].to(ag.Device.CPU))), name

    loss_ref, new_ref = O.ref_gpt_step(cfg, params, ids, tgt, lr)
    assert abs(loss - loss_ref) <= 1e-4 * max(abs(loss_ref), 1.0)
    tol = 1e-4 * np.sqrt(ids.size)
    for i, (name, _) in enumerate(bench.gpt_param_shapes(**cfg)):
        assert_close(params[i] - new[i], params[i] - new_ref[i], tol, f"grad of {name}")


def test_glue_lm_step_with_dropout(gpu):
    """The reference's Shakespeare GPT step (GELU, dropout 0.1, AdamW) through
    the glue: same dropout masks (Philox), so the same loss and gradients."""
    cfg = {"vocab": 65, "ctx": 64, "layers": 2, "d_model": 64, "heads": 4}
    rng = np.random.default_rng(12)
    shapes = [s for _, s in bench.gpt_param_shapes(**cfg)]
    params = [(0.05 * rng.standard_normal(s)).astype(f32) for s in shapes]
    ids = rng.integers(0, 65, (3, 64))
    tgt = rng.integers(0, 65, (3, 64))
    kw = dict(dropout=0.1, seed=2026, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, wd=0.01, t=1, grads=True)
    runs = []
    for device in (True, False):
        p = [x.copy() for x in params]
        m = [np.zeros_like(x) for x in params]
        v = [np.zeros_like(x) for x in params]
        call = (lambda *a, **k: on_device(O.ref_lm_step, *a, **k)) if device else O.ref_lm_step
        loss, grads = call(cfg, p, m, v, ids, tgt, **kw)
        runs.append((loss, grads, p))
    (loss, grads, p), (loss_ref, grads_ref, p_ref) = runs
    assert abs(loss - loss_ref) <= 1e-4 * max(abs(loss_ref), 1.0)
    tol = 1e-4 * np.sqrt(ids.size)
    for i, shape in enumerate(shapes):
        assert_close(grads[i], grads_ref[i], tol, f"grad {i} {shape}")
        assert_close(p[i], p_ref[i], 1e-5, f"param {i} after AdamW")
