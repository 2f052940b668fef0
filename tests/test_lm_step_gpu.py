"""Two AdamW training steps of the reference Shakespeare GPT (GELU MLP,
dropout 0.1 on the embeddings and both residual branches, bias-free
attention; python/shakespeare/scripts/model.py, train.py) on the device,
against the same steps on the reference's own CPU path (oracle/_ref, its
autograd, ops and Philox dropout).  The dropout masks are bit-identical, so
losses agree to 1e-4 and the step-1 gradients of every parameter to the 1e-4
bar (both metrics)."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import aargrad as ag
import lmutil
import oracle as O
from aargrad import data as D
from aargrad.optim import AdamW
from conftest import assert_close
from devutil import host

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference tree)")]
FIX = Path(__file__).resolve().parent / "golden" / "shakespeare"


@pytest.mark.parametrize("dropout", [0.1, 0.0])
def test_two_adamw_steps_match_reference(gpu, dropout):
    cfg = {"vocab_size": 65, "max_seq_len": 64, "n_layer": 2, "n_head": 4, "d_model": 64}
    rcfg = {"vocab": 65, "ctx": 64, "layers": 2, "d_model": 64, "heads": 4}
    model = lmutil.GPT(65, 64, 2, 4, 64, dropout=dropout, rng=np.random.default_rng(11))
    params = [np.ascontiguousarray(ag.to_numpy(p.tensor), np.float32).copy() for p in model.parameters()]
    model.to(gpu.Device.CUDA)
    opt = AdamW(list(model.parameters()), lr=3e-4, betas=(0.9, 0.95), weight_decay=0.01)
    ce = ag.nn.CrossEntropyLoss()
    loader = D.DeviceTokenLoader(FIX / "val_head.bin", 64, 4, shuffle=True, seed=0)
    batches = iter(loader)
    m = [np.zeros_like(p) for p in params]
    v = [np.zeros_like(p) for p in params]
    gpu.manual_seed(2026)
    for t in (1, 2):
        x, y = next(batches)
        logits = model(x)
        loss = ce(logits, y)
        opt.zero_grad()
        loss.backward()
        grads = [host(gpu, p.tensor.grad) for p in model.parameters()]
        opt.step()
        ids, tgt = gpu.to_numpy(x.to(gpu.Device.CPU)), gpu.to_numpy(y.to(gpu.Device.CPU))
        ref_loss, ref_grads = O.ref_lm_step(rcfg, params, m, v, ids, tgt, dropout=dropout,
                                            seed=2026 if t == 1 else -1, lr=3e-4, betas=(0.9, 0.95), eps=1e-8,
                                            wd=0.01, t=t, grads=True)
        got = float(host(gpu, loss))
        assert abs(got - ref_loss) <= 1e-4 * max(abs(ref_loss), 1.0), (t, got, ref_loss)
        if t == 1:
            for i, (g, r) in enumerate(zip(grads, ref_grads)):
                assert_close(g, r, 1e-4, f"grad of parameter {i}")
