"""The Shakespeare char-level GPT of the reference app
(python/shakespeare/scripts/model.py:8-57), restated over aargrad for the
data-format tests, with the attention bias switchable so the reference's
shipped checkpoint (which carries attention biases) loads; and the same
model's forward on the oracle's CPU ops (test infrastructure)."""
from __future__ import annotations

import numpy as np

import aargrad as ag
import oracle as O
from aargrad import nn
from aargrad.nn import Module


class TransformerBlock(Module):
    def __init__(self, d_model, n_heads, dropout, rng, attn_bias=False):
        super().__init__()
        self.ln1 = nn.LayerNorm(d_model)
        self.attn = nn.MultiHeadAttention(d_model, n_heads, causal=True, bias=attn_bias, rng=rng)
        self.ln2 = nn.LayerNorm(d_model)
        self.fc1 = nn.Linear(d_model, 4 * d_model, bias=True, rng=rng)
        self.gelu = nn.GELU()
        self.fc2 = nn.Linear(4 * d_model, d_model, bias=True, rng=rng)
        self.drop = nn.Dropout(dropout)

    def forward(self, x):
        x = ag.add(x, self.drop(self.attn(self.ln1(x))))
        h = self.gelu(self.fc1(self.ln2(x)))
        return ag.add(x, self.drop(self.fc2(h)))


class GPT(Module):
    def __init__(self, vocab_size, max_seq_len, n_layer, n_head, d_model, dropout=0.0, rng=None, attn_bias=False):
        super().__init__()
        rng = rng if rng is not None else np.random.default_rng()
        self.vocab_size = vocab_size
        self.max_seq_len = max_seq_len
        self.tok_emb = nn.Embedding(vocab_size, d_model, rng=rng)
        self.pos_emb = nn.Embedding(max_seq_len, d_model, rng=rng)
        self.drop = nn.Dropout(dropout)
        self.blocks = nn.Sequential(*[TransformerBlock(d_model, n_head, dropout, rng, attn_bias)
                                      for _ in range(n_layer)])
        self.ln_f = nn.LayerNorm(d_model)
        self.head = nn.Linear(d_model, vocab_size, bias=False, rng=rng)

    def forward(self, ids):
        B, T = ids.shape
        if T > self.max_seq_len:
            raise ValueError(f"sequence length {T} > max_seq_len {self.max_seq_len}")
        positions = ag.from_numpy(np.tile(np.arange(T, dtype=np.int64), (B, 1))).to(ids.device)
        x = ag.add(self.tok_emb(ids), self.pos_emb(positions))
        x = self.blocks(self.drop(x))
        return self.head(self.ln_f(x))


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
