"""Neural-network modules over aargrad._core, API-compatible with the
reference's aargrad/nn.py (AARONKANG04/aar-vlm, aargrad/nn.py:8-192): the
same classes, constructor arguments, parameter registration order and
forward compositions, so models written against the reference run unchanged
on the MI355X backend once moved to Device.CUDA.
"""
from __future__ import annotations

import math

import numpy as np

from . import _core


class Parameter:
    """A leaf tensor that requires grad (aargrad/nn.py:8-11)."""

    def __init__(self, tensor):
        tensor.requires_grad = True
        self.tensor = tensor


class Module:
    """Registers Parameters and sub-Modules in assignment order; parameters()
    yields own parameters first, then each child's (aargrad/nn.py:14-60).
    Checkpoints key parameters by this order."""

    def __init__(self):
        object.__setattr__(self, "_parameters", {})
        object.__setattr__(self, "_modules", {})
        object.__setattr__(self, "training", True)

    def __setattr__(self, name, value):
        if isinstance(value, Parameter):
            self._parameters[name] = value
        elif isinstance(value, Module):
            self._modules[name] = value
        super().__setattr__(name, value)

    def parameters(self):
        yield from self._parameters.values()
        for child in self._modules.values():
            yield from child.parameters()

    def zero_grad(self):
        for p in self.parameters():
            p.tensor.zero_grad()

    def to(self, device):
        # Tensor.to drops autograd state, so re-mark the moved leaves.
        for p in self._parameters.values():
            moved = p.tensor.to(device)
            moved.requires_grad = True
            p.tensor = moved
        for child in self._modules.values():
            child.to(device)
        return self

    def train(self, mode=True):
        self.training = mode
        for child in self._modules.values():
            child.train(mode)
        return self

    def eval(self):
        return self.train(False)

    def forward(self, *args, **kwargs):
        raise NotImplementedError

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)


class Embedding(Module):
    def __init__(self, num_embeddings, embedding_dim, *, rng=None):
        super().__init__()
        rng = rng if rng is not None else np.random.default_rng()
        w = rng.standard_normal((num_embeddings, embedding_dim)).astype(np.float32)
        self.weight = Parameter(_core.from_numpy(w))

    def forward(self, ids):
        return _core.embedding(self.weight.tensor, ids)


class CrossEntropyLoss(Module):
    def __init__(self, ignore_index=-100):
        super().__init__()
        self.ignore_index = ignore_index

    def forward(self, logits, targets):
        if len(logits.shape) > 2:
            rows = int(np.prod(logits.shape[:-1]))
            logits = _core.reshape(logits, [rows, logits.shape[-1]])
            targets = _core.reshape(targets, [rows])
        return _core.cross_entropy(logits, targets, self.ignore_index)


class Linear(Module):
    """y = x W^T (+ b) with W [out, in]; the forward is matmul_a_bt, so its
    backward runs matmul (dX) and matmul_at_b (dW).  With a bias the product
    and the bias addition are one GEMM (bias in the epilogue), bit-identical
    to matmul_a_bt followed by add_bias (reference aargrad/nn.py:101-105)."""

    def __init__(self, in_features, out_features, *, bias=False, rng=None):
        super().__init__()
        rng = rng if rng is not None else np.random.default_rng()
        bound = math.sqrt(6.0 / in_features)
        w = rng.uniform(-bound, bound, size=(out_features, in_features)).astype(np.float32)
        self.weight = Parameter(_core.from_numpy(w))
        self.bias = Parameter(_core.from_numpy(np.zeros((out_features,), np.float32))) if bias else None

    def forward(self, x):
        if self.bias is not None:
            return _core._linear(x, self.weight.tensor, self.bias.tensor)
        return _core.matmul_a_bt(x, self.weight.tensor)


class ReLU(Module):
    def forward(self, x):
        return _core.relu(x)


class GELU(Module):
    def forward(self, x):
        return _core.gelu(x)


class Dropout(Module):
    def __init__(self, p=0.5):
        super().__init__()
        if not 0.0 <= p < 1.0:
            raise ValueError("Dropout: p must be in [0, 1)")
        self.p = p

    def forward(self, x):
        if not self.training or self.p == 0.0:
            return x
        return _core.dropout(x, self.p)


class LayerNorm(Module):
    def __init__(self, normalized_features, eps=1e-5):
        super().__init__()
        self.weight = Parameter(_core.from_numpy(np.ones((normalized_features,), np.float32)))
        self.bias = Parameter(_core.from_numpy(np.zeros((normalized_features,), np.float32)))
        self.eps = eps

    def forward(self, x):
        return _core.layernorm(x, self.weight.tensor, self.bias.tensor, self.eps)


class Sequential(Module):
    def __init__(self, *layers):
        super().__init__()
        for i, layer in enumerate(layers):
            setattr(self, f"layer_{i}", layer)

    def forward(self, x):
        for layer in self._modules.values():
            x = layer(x)
        return x


def scaled_dot_product_attention(q, k, v, *, causal=False):
    """Unfused attention over [T, d] operands (aargrad/nn.py:154-161): every
    step (product, scale, causal mask, softmax, product) runs on the device."""
    scores = _core.scale(_core.matmul_a_bt(q, k), 1.0 / math.sqrt(q.shape[-1]))
    if causal:
        scores = _core.apply_causal_mask(scores)
    return _core.matmul(_core.softmax(scores), v)


class MultiHeadAttention(Module):
    """qkv projection, per-head views, flash attention, output projection
    (aargrad/nn.py:164-192).  The views, the attention and the head merge run
    as one op (_core._flash_attention_qkv) that reads q/k/v in place from the
    packed projection and writes the merged heads directly; the math is the
    reference composition's."""

    def __init__(self, d_model, n_heads, *, causal=False, bias=True, rng=None):
        super().__init__()
        if d_model % n_heads != 0:
            raise ValueError("d_model must be divisible by n_heads")
        self.d_model = d_model
        self.n_heads = n_heads
        self.d_head = d_model // n_heads
        self.causal = causal
        rng = rng if rng is not None else np.random.default_rng()
        self.qkv_proj = Linear(d_model, 3 * d_model, bias=bias, rng=rng)
        self.out_proj = Linear(d_model, d_model, bias=bias, rng=rng)

    def _head_view(self, qkv, which):
        # [B, T, 3, H, d] -> [B, H, T, d] view of q, k or v
        part = _core.squeeze(_core.slice(qkv, 2, which, which + 1), 2)
        return _core.transpose(part, 1, 2)

    def forward(self, x):
        return self.out_proj(_core._flash_attention_qkv(self.qkv_proj(x), self.n_heads, self.causal))

    def forward_views(self, x):
        """The reference's literal composition through per-head views and
        flash_attention (same result as forward)."""
        B, T, _ = x.shape
        qkv = _core.reshape(self.qkv_proj(x), [B, T, 3, self.n_heads, self.d_head])
        q, k, v = (self._head_view(qkv, i) for i in range(3))
        out = _core.flash_attention(q, k, v, self.causal)
        out = _core.reshape(_core.transpose(out, 1, 2), [B, T, self.d_model])
        return self.out_proj(out)
