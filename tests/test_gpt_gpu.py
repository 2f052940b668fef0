"""End-to-end GPT training step (BASELINE config 5 composition) on the GPU
against the reference's own CPU path (oracle/_ref ref_gpt_step): the loss
and every parameter gradient of one SGD step, on a small configuration; plus
the nn/optim layer (MultiHeadAttention, Linear, LayerNorm, SGD) reducing the
loss over a few steps."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from conftest import assert_close

sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
import bench  # noqa: E402  (the config-5 workload definition lives with the benchmark)

pytestmark = pytest.mark.gpu
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference tree)")


@needs_ref
@pytest.mark.parametrize("cfg", [dict(vocab=65, ctx=32, layers=2, d_model=64, heads=2, batch=3),
                                 dict(vocab=65, ctx=64, layers=1, d_model=128, heads=2, batch=2)])
def test_gpt_sgd_step_matches_reference_cpu(gpu, cfg):
    ag = gpu
    params = bench.gpt_init_params(cfg, seed=5)
    ids, tgt = bench.gpt_tokens(cfg, cfg["batch"], seed=6)
    lr = 1.0  # p_new = p - g, so the parameter deltas are the gradients
    loss_ref, new_ref = O.ref_gpt_step(cfg, params, ids, tgt, lr)
    model = bench.GPT(ag, cfg, params)
    B, T = ids.shape
    tids = ag.from_numpy(ids).to(ag.Device.CUDA)
    pos = ag.from_numpy(np.tile(np.arange(T, dtype=np.int64), (B, 1))).to(ag.Device.CUDA)
    ttgt = ag.from_numpy(tgt.reshape(-1)).to(ag.Device.CUDA)
    loss = model.step(tids, pos, ttgt, lr)
    assert abs(float(ag.to_numpy(loss.to(ag.Device.CPU))) - loss_ref) <= 1e-4 * max(abs(loss_ref), 1.0)
    for i, (name, _) in enumerate(bench.gpt_param_shapes(**cfg)):
        got = params[i] - ag.to_numpy(model.p[i].to(ag.Device.CPU))
        ref = params[i] - new_ref[i]
        assert_close(got, ref, 1e-4 * np.sqrt(B * T), f"grad of {name}")


def test_transformer_block_loss_decreases(gpu):
    """A pre-LN block (nn.LayerNorm, nn.MultiHeadAttention, nn.Linear, ReLU)
    trained with optim.SGD on a fixed batch: the loss must drop
    (tests/python/test_mha.py:109-137 style)."""
    ag = gpu
    from aargrad import nn, optim

    rng = np.random.default_rng(0)
    d, H, T, B, V = 32, 4, 16, 4, 11

    class Tiny(nn.Module):
        def __init__(self):
            super().__init__()
            self.emb = nn.Embedding(V, d, rng=rng)
            self.ln = nn.LayerNorm(d)
            self.attn = nn.MultiHeadAttention(d, H, causal=True, bias=False, rng=rng)
            self.fc = nn.Linear(d, V, bias=True, rng=rng)

        def forward(self, ids):
            x = self.emb(ids)
            x = ag.add(x, self.attn(self.ln(x)))
            return self.fc(ag.relu(x))

    model = Tiny().to(ag.Device.CUDA)
    opt = optim.SGD(model.parameters(), lr=0.05)
    ce = nn.CrossEntropyLoss()
    ids_np = rng.integers(0, V, (B, T + 1))
    ids = ag.from_numpy(ids_np[:, :-1].copy()).to(ag.Device.CUDA)
    tgt = ag.from_numpy(ids_np[:, 1:].copy()).to(ag.Device.CUDA)
    losses = []
    for _ in range(30):
        loss = ce(model(ids), tgt)
        opt.zero_grad()
        loss.backward()
        opt.step()
        losses.append(float(ag.to_numpy(loss.to(ag.Device.CPU))))
    assert losses[-1] < 0.7 * losses[0], losses


def test_adamw_optimizer_runs(gpu):
    ag = gpu
    from aargrad import nn, optim

    rng = np.random.default_rng(1)
    lin = nn.Linear(8, 3, bias=True, rng=rng).to(ag.Device.CUDA)
    opt = optim.AdamW(lin.parameters(), lr=1e-2)
    x = ag.from_numpy(rng.standard_normal((16, 8)).astype(np.float32)).to(ag.Device.CUDA)
    t = ag.from_numpy(rng.integers(0, 3, 16)).to(ag.Device.CUDA)
    first = None
    for _ in range(20):
        loss = ag.cross_entropy(lin(x), t)
        opt.zero_grad()
        loss.backward()
        opt.step()
        v = float(ag.to_numpy(loss.to(ag.Device.CPU)))
        first = v if first is None else first
    assert v < first
