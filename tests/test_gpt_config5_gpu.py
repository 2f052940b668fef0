"""BASELINE config 5 at its stated shape: the decoder-only char GPT with 6
layers, d_model 384, 6 heads, context 256, vocab 65 (reference
python/shakespeare/scripts/model.py:8-57, one training step as in
train.py:204-213 with SGD).

* One SGD step at the full model shape, batch 2, against the reference's own
  CPU step (oracle/_ref ref_gpt_step: its autograd, ops and kernels): the loss
  and every parameter delta.
* Batch 64 (the benchmarked step): finite loss, a bit-identical rerun from
  the same weights, and a falling loss over ten steps.
* The step's attention shape, causal B64 H6 T256 d64, on sampled heads against
  the oracle plus the full-size checksum identities, both as contiguous
  [B, H, T, d] tensors and through the packed-qkv op the model uses.
Tolerances: 1e-4 for the loss and attention; a parameter delta is a GEMM
gradient contracted over the B*T tokens, so 1e-4*sqrt(B*T)."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from conftest import TOL, assert_close
from devutil import dev, host

sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
import bench  # noqa: E402  (the config-5 workload definition lives with the benchmark)

pytestmark = pytest.mark.gpu
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference tree)")
f32 = np.float32
CFG = bench.GPT5


def _inputs(ag, ids, tgt):
    B, T = ids.shape
    tids = ag.from_numpy(ids).to(ag.Device.CUDA)
    pos = ag.from_numpy(np.tile(np.arange(T, dtype=np.int64), (B, 1))).to(ag.Device.CUDA)
    ttgt = ag.from_numpy(np.ascontiguousarray(tgt.reshape(-1))).to(ag.Device.CUDA)
    return tids, pos, ttgt


def _loss(ag, t):
    return float(ag.to_numpy(t.to(ag.Device.CPU)))


@needs_ref
def test_config5_sgd_step_matches_reference_cpu(gpu):
    ag = gpu
    assert (CFG["layers"], CFG["d_model"], CFG["heads"], CFG["ctx"], CFG["vocab"]) == (6, 384, 6, 256, 65)
    cfg = dict(CFG, batch=2)
    params = bench.gpt_init_params(cfg, seed=11)
    ids, tgt = bench.gpt_tokens(cfg, 2, seed=12)
    lr = 1.0  # p_new = p - g: the parameter deltas are the gradients
    print("config 5 reference CPU step (batch 2) ...", flush=True)
    loss_ref, new_ref = O.ref_gpt_step(cfg, params, ids, tgt, lr)
    model = bench.GPT(ag, cfg, params)
    loss = model.step(*_inputs(ag, ids, tgt), lr)
    got = _loss(ag, loss)
    assert abs(got - loss_ref) <= TOL * max(abs(loss_ref), 1.0), (got, loss_ref)
    tol = 1e-4 * np.sqrt(ids.size)
    for i, (name, _) in enumerate(bench.gpt_param_shapes(**cfg)):
        d_got = params[i] - host(ag, model.p[i])
        d_ref = params[i] - new_ref[i]
        assert_close(d_got, d_ref, tol, f"delta of {name}")


def test_config5_batch64_rerun_and_loss(gpu):
    ag = gpu
    params = bench.gpt_init_params(CFG, seed=0)
    ids, tgt = bench.gpt_tokens(CFG, CFG["batch"], seed=1)
    inputs = _inputs(ag, ids, tgt)
    runs = []
    for _ in range(2):
        model = bench.GPT(ag, CFG, params)
        losses = [_loss(ag, model.step(*inputs, 1e-3)) for _ in range(10)]
        runs.append((losses, [host(ag, p) for p in model.p]))
    (l1, p1), (l2, p2) = runs
    assert all(np.isfinite(l1)), l1
    # ln(65) = 4.17 for uniform logits; N(0, 0.02) weights start near it
    assert 3.5 < l1[0] < 5.0, l1[0]
    assert l1 == l2, (l1, l2)  # every kernel of the step is deterministic
    for a, b in zip(p1, p2):
        np.testing.assert_array_equal(a, b)
    # SGD at lr 1e-3 on a fixed batch: the loss falls every step
    assert all(b < a for a, b in zip(l1, l1[1:])), l1


def _checksums(o, dk, dv, do):
    """Size-independent identities over every head: sum_j dV[j] = sum_i dO[i]
    (rows of P sum to 1) and sum_j dK[j] = 0 (rows of dS sum to 0)."""
    assert np.isfinite(o).all()
    assert_close(dv.astype(np.float64).sum(2), do.astype(np.float64).sum(2), TOL, "sum dV = sum dO")
    sdk = np.abs(dk.astype(np.float64).sum(2)).max()
    scale = np.abs(dk.astype(np.float64)).sum(2).max()
    assert sdk <= TOL * scale, f"sum dK = {sdk:.3e} (scale {scale:.3e})"


def test_config5_attention_shape(gpu):
    """Causal flash attention at B64 H6 T256 d64 (one GPT layer's attention):
    sampled heads against the oracle, checksums over all 384 heads, and the
    packed-qkv op on the same data bit-identical to the contiguous op."""
    ag = gpu
    B, H, T, d = CFG["batch"], CFG["heads"], CFG["ctx"], CFG["d_model"] // CFG["heads"]
    rng = np.random.default_rng(5)
    q, k, v, do = (rng.standard_normal((B, H, T, d)).astype(f32) for _ in range(4))
    tq, tk, tv = dev(ag, q, True), dev(ag, k, True), dev(ag, v, True)
    o = ag.flash_attention(tq, tk, tv, True)
    o.backward(dev(ag, do))
    oh, dq, dk, dv = host(ag, o), host(ag, tq.grad), host(ag, tk.grad), host(ag, tv.grad)
    _, lse = ag._core._flash_attention_fwd(dev(ag, q), dev(ag, k), dev(ag, v), True)
    lse = host(ag, lse)
    for b, h in ((0, 0), (31, 3), (63, 5)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        assert_close(oh[sl], O.attention(q[sl], k[sl], v[sl], True), TOL, f"O ({b},{h})")
        rq, rk, rv = O.attention_backward(q[sl], k[sl], v[sl], do[sl], True)
        assert_close(dq[sl], rq, TOL, f"dq ({b},{h})")
        assert_close(dk[sl], rk, TOL, f"dk ({b},{h})")
        assert_close(dv[sl], rv, TOL, f"dv ({b},{h})")
        assert_close(lse[sl], O.attention_lse(q[sl], k[sl], True), TOL, f"lse ({b},{h})")
    _checksums(oh, dk, dv, do)
    # the same heads packed as the model's [B, T, 3*D] projection
    D = H * d
    qkv = np.stack([x.transpose(0, 2, 1, 3) for x in (q, k, v)], axis=2).reshape(B, T, 3 * D)
    t = dev(ag, qkv, True)
    op = ag._core._flash_attention_qkv(t, H, True)
    op.backward(dev(ag, np.ascontiguousarray(do.transpose(0, 2, 1, 3)).reshape(B, T, D)))
    np.testing.assert_array_equal(host(ag, op).reshape(B, T, H, d).transpose(0, 2, 1, 3), oh)
    g = host(ag, t.grad).reshape(B, T, 3, H, d)
    for i, ref in enumerate((dq, dk, dv)):
        np.testing.assert_array_equal(g[:, :, i].transpose(0, 2, 1, 3), ref)
