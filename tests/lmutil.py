"""Test model: the Shakespeare char-level GPT of the reference app
(python/shakespeare/scripts/model.py:8-57) built from aargrad modules, with
the attention bias switchable so the reference's shipped checkpoint (which
carries attention biases) loads; and the same model's forward on the oracle's
CPU ops (test infrastructure).

The module tree is organised here as pre-norm residual branches
(x + dropout(body(layernorm(x)))): the attention branch, then the
feed-forward branch (linear -> GELU -> linear).  What has to agree with the
reference model does: the parameters in Module.parameters() order (the
checkpoint keys p0..pN follow it), the initialisers' random draws in the same
order, and the computation including the three dropout sites."""
from __future__ import annotations

import numpy as np

import aargrad as ag
import oracle as O
from aargrad import nn
from aargrad.nn import Module


class PreNormResidual(Module):
    """x + dropout(body(layernorm(x)))."""

    def __init__(self, d_model, body, dropout):
        super().__init__()
        self.norm = nn.LayerNorm(d_model)
        self.body = body
        self.drop = nn.Dropout(dropout)

    def forward(self, x):
        return ag.add(x, self.drop(self.body(self.norm(x))))


def transformer_block(d_model, n_heads, dropout, rng, attn_bias=False):
    """Attention branch then feed-forward branch.  Draw order: qkv and output
    projections, then the two feed-forward layers."""
    attention = nn.MultiHeadAttention(d_model, n_heads, causal=True, bias=attn_bias, rng=rng)
    ffn = nn.Sequential(nn.Linear(d_model, 4 * d_model, bias=True, rng=rng), nn.GELU(),
                        nn.Linear(4 * d_model, d_model, bias=True, rng=rng))
    return nn.Sequential(PreNormResidual(d_model, attention, dropout), PreNormResidual(d_model, ffn, dropout))


class GPT(Module):
    """Token + position embeddings (dropout), the blocks, a final layernorm and
    a bias-free vocabulary head."""

    def __init__(self, vocab_size, max_seq_len, n_layer, n_head, d_model, dropout=0.0, rng=None, attn_bias=False):
        super().__init__()
        rng = rng if rng is not None else np.random.default_rng()
        self.vocab_size = vocab_size
        self.max_seq_len = max_seq_len
        self.tok_emb = nn.Embedding(vocab_size, d_model, rng=rng)
        self.pos_emb = nn.Embedding(max_seq_len, d_model, rng=rng)
        self.drop = nn.Dropout(dropout)
        self.blocks = nn.Sequential(*(transformer_block(d_model, n_head, dropout, rng, attn_bias)
                                      for _ in range(n_layer)))
        self.ln_f = nn.LayerNorm(d_model)
        self.head = nn.Linear(d_model, vocab_size, bias=False, rng=rng)
        self._positions = {}

    def _position_ids(self, batch, length, device):
        key = (batch, length, device)
        if key not in self._positions:
            grid = np.broadcast_to(np.arange(length, dtype=np.int64), (batch, length))
            self._positions[key] = ag.from_numpy(np.ascontiguousarray(grid)).to(device)
        return self._positions[key]

    def forward(self, ids):
        B, T = ids.shape
        if T > self.max_seq_len:
            raise ValueError(f"sequence length {T} > max_seq_len {self.max_seq_len}")
        x = ag.add(self.tok_emb(ids), self.pos_emb(self._position_ids(B, T, ids.device)))
        return self.head(self.ln_f(self.blocks(self.drop(x))))


def gpt_from_config(cfg, rng=None):
    return GPT(cfg["vocab_size"], cfg["max_seq_len"], cfg["n_layer"], cfg["n_head"], cfg["d_model"], 0.0,
               rng=rng, attn_bias=bool(cfg.get("attn_bias", False)))


def oracle_forward(arrays, cfg, ids) -> np.ndarray:
    """Logits [B, T, V] of the model above (dropout off) on the oracle's ops."""
    it = iter(arrays)
    nxt = lambda: next(it)  # noqa: E731
    bias = bool(cfg.get("attn_bias", False))
    H, D = cfg["n_head"], cfg["d_model"]
    d = D // H
    B, T = ids.shape
    tok, pos = nxt(), nxt()
    x = O.add(O.embedding(tok, ids.reshape(-1)), O.embedding(pos, np.tile(np.arange(T, dtype=np.int64), B)))
    for _ in range(cfg["n_layer"]):
        w1, b1 = nxt(), nxt()
        wqkv = nxt()
        bqkv = nxt() if bias else None
        wo = nxt()
        bo = nxt() if bias else None
        w2, b2, wf1, bf1, wf2, bf2 = (nxt() for _ in range(6))
        qkv = O.matmul("nt", O.layernorm(x, w1, b1), wqkv)
        if bias:
            qkv = O.add_bias(qkv, bqkv)
        qkv = qkv.reshape(B, T, 3, H, d)
        q, k, v = (np.ascontiguousarray(qkv[:, :, i].transpose(0, 2, 1, 3)) for i in range(3))
        o = np.ascontiguousarray(O.attention(q, k, v, True).transpose(0, 2, 1, 3)).reshape(B * T, D)
        a = O.matmul("nt", o, wo)
        if bias:
            a = O.add_bias(a, bo)
        x = O.add(x, a)
        h = O.gelu(O.add_bias(O.matmul("nt", O.layernorm(x, w2, b2), wf1), bf1))
        x = O.add(x, O.add_bias(O.matmul("nt", h, wf2), bf2))
    lw, lb, head = nxt(), nxt(), nxt()
    return O.matmul("nt", O.layernorm(x, lw, lb), head).reshape(B, T, -1)
