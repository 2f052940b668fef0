"""Optimizers over aargrad._core, API-compatible with the reference's
aargrad/optim.py (AARONKANG04/aar-vlm, aargrad/optim.py:4-54).  Both update
parameters in place on the device.  The reference calls scaled_add_inplace /
adamw_step once per parameter; here one multi-tensor call covers them all (up
to 48 parameters per kernel launch), with the same per-element arithmetic,
so the updates are bit-identical."""
from __future__ import annotations

from . import _core


class SGD:
    def __init__(self, params, lr=0.01):
        self.params = list(params)
        self.lr = lr

    def zero_grad(self):
        for p in self.params:
            p.tensor.zero_grad()

    def step(self):
        dsts, srcs = [], []
        for p in self.params:
            g = p.tensor.grad
            if g is not None:
                dsts.append(p.tensor)
                srcs.append(g)
        if dsts:
            _core._scaled_add_inplace_multi(dsts, srcs, -self.lr)


class AdamW:
    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01):
        self.params = list(params)
        self.lr = lr
        self.beta1, self.beta2 = betas
        self.eps = eps
        self.weight_decay = weight_decay
        self.t = 0
        self._state = {}

    def zero_grad(self):
        for p in self.params:
            p.tensor.zero_grad()

    def step(self):
        self.t += 1
        bc1 = 1.0 - self.beta1 ** self.t
        bc2 = 1.0 - self.beta2 ** self.t
        ps, gs, ms, vs = [], [], [], []
        for p in self.params:
            g = p.tensor.grad
            if g is None:
                continue
            state = self._state.get(id(p))
            if state is None:
                t = p.tensor
                state = (_core.Tensor.zeros(t.shape, t.dtype, t.device), _core.Tensor.zeros(t.shape, t.dtype, t.device))
                self._state[id(p)] = state
            ps.append(p.tensor)
            gs.append(g)
            ms.append(state[0])
            vs.append(state[1])
        if ps:
            _core._adamw_step_multi(ps, gs, ms, vs, self.lr, self.beta1, self.beta2, self.eps, self.weight_decay,
                                    bc1, bc2)
