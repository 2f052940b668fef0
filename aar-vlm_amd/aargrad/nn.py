"""Neural-network modules over aargrad._core.

Interface kept from the reference's aargrad/nn.py (AARONKANG04/aar-vlm,
aargrad/nn.py:8-192) so models written against it run unchanged on the MI355X
backend once moved to Device.CUDA: class names, constructor arguments,
attribute names (``weight``, ``bias``, ``qkv_proj``, ``out_proj``, the
``_parameters`` / ``_modules`` registries), parameter registration order
(checkpoints key parameters by it) and the random draws of the initialisers.

Structure: every module keeps two ordered registries filled by attribute
assignment; one pre-order walk over the module tree (``_walk``) drives
``parameters()``, ``to()`` and ``train()``.  Linear layers with a bias and
multi-head attention run as fused device ops (bias in the GEMM epilogue; the
attention reads q/k/v in place from the packed projection).
"""
from __future__ import annotations

import functools
import math

import numpy as np

from . import _core


class Parameter:
    """A trainable leaf: wraps a tensor and marks it as requiring grad."""

    def __init__(self, tensor):
        tensor.requires_grad = True
        self.tensor = tensor


class Module:
    """Base class.  Assigning a Parameter or a Module to an attribute records
    it, in first-assignment order, in ``_parameters`` or ``_modules``
    (re-assigning a recorded name replaces the entry in place; other values
    are plain attributes)."""

    def __init__(self):
        state = {"_parameters": {}, "_modules": {}, "training": True}
        for name, value in state.items():
            object.__setattr__(self, name, value)

    def __setattr__(self, name, value):
        registry = _registry_for(self, value)
        if registry is not None:
            registry[name] = value
        object.__setattr__(self, name, value)

    def _walk(self):
        """This module, then its descendants, depth first in registration
        order (pre-order)."""
        pending = [self]
        while pending:
            mod = pending.pop()
            yield mod
            pending.extend(reversed(list(mod._modules.values())))

    def parameters(self):
        """Own parameters first, then each child's, recursively."""
        for mod in self._walk():
            yield from mod._parameters.values()

    def zero_grad(self):
        for p in self.parameters():
            p.tensor.zero_grad()

    def to(self, device):
        """Moves every parameter to `device`.  Tensor.to returns a fresh leaf
        without autograd state, so each moved tensor is marked again."""
        for mod in self._walk():
            for p in mod._parameters.values():
                moved = p.tensor.to(device)
                moved.requires_grad = True
                p.tensor = moved
        return self

    def train(self, mode=True):
        for mod in self._walk():
            object.__setattr__(mod, "training", mode)
        return self

    def eval(self):
        return self.train(False)

    def forward(self, *args, **kwargs):
        raise NotImplementedError

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)


def _registry_for(module: Module, value):
    """The registry of `module` an attribute value belongs in, or None."""
    if isinstance(value, Parameter):
        return module._parameters
    if isinstance(value, Module):
        return module._modules
    return None


def _new_parameter(array) -> Parameter:
    return Parameter(_core.from_numpy(np.ascontiguousarray(array, np.float32)))


def _rng_or_default(rng):
    return rng if rng is not None else np.random.default_rng()


class Embedding(Module):
    """Lookup table, weight [num_embeddings, embedding_dim] ~ N(0, 1)."""

    def __init__(self, num_embeddings, embedding_dim, *, rng=None):
        super().__init__()
        table = _rng_or_default(rng).standard_normal((num_embeddings, embedding_dim))
        self.weight = _new_parameter(table)

    def forward(self, ids):
        return _core.embedding(self.weight.tensor, ids)


class CrossEntropyLoss(Module):
    """Mean cross entropy; logits of rank > 2 are taken as rows of their last
    dim, with the targets flattened to match."""

    def __init__(self, ignore_index=-100):
        super().__init__()
        self.ignore_index = ignore_index

    def forward(self, logits, targets):
        if len(logits.shape) > 2:
            rows = math.prod(logits.shape[:-1])
            logits = _core.reshape(logits, [rows, logits.shape[-1]])
            targets = _core.reshape(targets, [rows])
        return _core.cross_entropy(logits, targets, self.ignore_index)


class Linear(Module):
    """y = x W^T (+ b), W [out, in] ~ U(-sqrt(6/in), sqrt(6/in)), b = 0.

    Without a bias the forward is matmul_a_bt (backward: matmul for dX,
    matmul_at_b for dW).  With a bias, product and bias are one GEMM whose
    epilogue adds b, bit-identical to matmul_a_bt followed by add_bias."""

    def __init__(self, in_features, out_features, *, bias=False, rng=None):
        super().__init__()
        bound = math.sqrt(6.0 / in_features)
        w = _rng_or_default(rng).uniform(-bound, bound, size=(out_features, in_features))
        self.weight = _new_parameter(w)
        self.bias = _new_parameter(np.zeros(out_features)) if bias else None

    def forward(self, x):
        w = self.weight.tensor
        return _core.matmul_a_bt(x, w) if self.bias is None else _core._linear(x, w, self.bias.tensor)


class _Pointwise(Module):
    """A parameter-free module applying one elementwise device op."""

    _op = None

    def forward(self, x):
        return type(self)._op(x)


class ReLU(_Pointwise):
    _op = staticmethod(_core.relu)


class GELU(_Pointwise):
    _op = staticmethod(_core.gelu)


class Dropout(Module):
    """Inverted dropout while training (mask from the device Philox stream);
    the identity in eval mode or with p = 0."""

    def __init__(self, p=0.5):
        super().__init__()
        if not 0.0 <= p < 1.0:
            raise ValueError("Dropout: p must be in [0, 1)")
        self.p = p

    def forward(self, x):
        active = self.training and self.p != 0.0
        return _core.dropout(x, self.p) if active else x


class LayerNorm(Module):
    """Layer normalisation over the last dim, gamma = 1, beta = 0 at init."""

    def __init__(self, normalized_features, eps=1e-5):
        super().__init__()
        self.weight = _new_parameter(np.ones(normalized_features))
        self.bias = _new_parameter(np.zeros(normalized_features))
        self.eps = eps

    def forward(self, x):
        return _core.layernorm(x, self.weight.tensor, self.bias.tensor, self.eps)


class Sequential(Module):
    """Children named layer_0, layer_1, ... applied in order."""

    def __init__(self, *layers):
        super().__init__()
        for i, layer in enumerate(layers):
            setattr(self, f"layer_{i}", layer)

    def forward(self, x):
        return functools.reduce(lambda h, layer: layer(h), self._modules.values(), x)


def scaled_dot_product_attention(q, k, v, *, causal=False):
    """softmax(q k^T / sqrt(d) [+ causal mask]) v over [..., T, d] operands,
    unfused: each of the five steps is its own device op."""
    inv_sqrt_d = 1.0 / math.sqrt(q.shape[-1])
    logits = _core.scale(_core.matmul_a_bt(q, k), inv_sqrt_d)
    if causal:
        logits = _core.apply_causal_mask(logits)
    return _core.matmul(_core.softmax(logits), v)


class MultiHeadAttention(Module):
    """Packed qkv projection, attention per head, output projection.

    ``forward`` runs the per-head split, the flash attention and the head merge
    as one op (_core._flash_attention_qkv): q, k and v are read in place from
    the [B, T, 3*D] projection and the output is written as [B, T, D].
    ``forward_views`` is the same computation through explicit per-head
    [B, H, T, d] views and flash_attention (used to check the fused path)."""

    def __init__(self, d_model, n_heads, *, causal=False, bias=True, rng=None):
        super().__init__()
        if d_model % n_heads != 0:
            raise ValueError("d_model must be divisible by n_heads")
        self.d_model = d_model
        self.n_heads = n_heads
        self.d_head = d_model // n_heads
        self.causal = causal
        rng = _rng_or_default(rng)
        self.qkv_proj = Linear(d_model, 3 * d_model, bias=bias, rng=rng)
        self.out_proj = Linear(d_model, d_model, bias=bias, rng=rng)

    def forward(self, x):
        heads = _core._flash_attention_qkv(self.qkv_proj(x), self.n_heads, self.causal)
        return self.out_proj(heads)

    def _split_heads(self, packed):
        """[B, T, 3*D] -> three [B, H, T, d] views (q, k, v)."""
        B, T, _ = packed.shape
        grid = _core.reshape(packed, [B, T, 3, self.n_heads, self.d_head])
        views = []
        for which in range(3):
            one = _core.squeeze(_core.slice(grid, 2, which, which + 1), 2)  # [B, T, H, d]
            views.append(_core.transpose(one, 1, 2))
        return views

    def forward_views(self, x):
        B, T, _ = x.shape
        q, k, v = self._split_heads(self.qkv_proj(x))
        merged = _core.transpose(_core.flash_attention(q, k, v, self.causal), 1, 2)  # [B, T, H, d]
        return self.out_proj(_core.reshape(merged, [B, T, self.d_model]))
