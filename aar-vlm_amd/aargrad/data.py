"""Token data of the language-model training loop: the reference Shakespeare
pipeline's on-disk formats, its dataset/loader classes, and a loader that
keeps the token stream in device memory.

Formats (python/shakespeare/scripts/prepare.py:37-47, data.py:7-33):
  * ``meta.json``: ``{"vocab": [...], "vocab_size": N}``; a token id is the
    character's index in ``vocab``.
  * ``train.bin`` / ``val.bin``: the ids as raw little-endian int64, no
    header (read as ``np.memmap(path, dtype=np.int64)``, train.py:148-149).

``CharTokenizer``, ``TokenWindowDataset`` and ``DataLoader`` keep the
reference classes (data.py:7-71): same arguments, same windows, same shuffle
order for a seed.  ``DeviceTokenLoader`` yields exactly the batches that
``DataLoader(TokenWindowDataset(tokens, T), batch_size, shuffle, seed=seed)``
yields, already on the device: the stream is uploaded once and each batch is
gathered there from its window starts (``_core._token_windows``), so a step
moves 16*B*T bytes device-side instead of a host gather, collate and copy.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

from . import _core


def read_tokens(path) -> np.ndarray:
    """Memory-mapped int64 little-endian token file (train.py:148-149)."""
    return np.memmap(path, dtype="<i8", mode="r")


def write_tokens(ids, path) -> None:
    """Raw little-endian int64 ids, no header (prepare.py:44-47)."""
    np.ascontiguousarray(ids, dtype="<i8").tofile(path)


class CharTokenizer:
    """Character vocabulary in ``meta.json`` (data.py:7-33)."""

    def __init__(self, vocab):
        self.vocab = list(vocab)
        self.stoi = {c: i for i, c in enumerate(self.vocab)}
        self.itos = {i: c for i, c in enumerate(self.vocab)}

    @classmethod
    def from_text(cls, text):
        return cls(sorted(set(text)))

    @classmethod
    def load(cls, path):
        with open(path) as f:
            return cls(json.load(f)["vocab"])

    def save(self, path):
        with open(path, "w") as f:
            json.dump({"vocab": self.vocab, "vocab_size": len(self.vocab)}, f)

    @property
    def vocab_size(self):
        return len(self.vocab)

    def encode(self, s):
        return np.array([self.stoi[c] for c in s], dtype=np.int64)

    def decode(self, ids):
        return "".join(self.itos[int(i)] for i in ids)


class TokenWindowDataset:
    """Window i: input tokens[i:i+T], target tokens[i+1:i+T+1] (data.py:36-48)."""

    def __init__(self, tokens, max_seq_len):
        self.tokens = tokens
        self.max_seq_len = max_seq_len

    def __len__(self):
        return len(self.tokens) - self.max_seq_len

    def __getitem__(self, i):
        x = np.asarray(self.tokens[i: i + self.max_seq_len], dtype=np.int64)
        y = np.asarray(self.tokens[i + 1: i + self.max_seq_len + 1], dtype=np.int64)
        return {"input": x, "target": y}


def default_collate(batch):
    keys = batch[0].keys()
    return {k: np.stack([b[k] for b in batch]) for k in keys}


def _batches(rng, n, batch_size, shuffle, drop_last):
    """Index batches of one epoch: a fresh permutation per epoch from the
    loader's generator (data.py:62-71)."""
    idx = rng.permutation(n) if shuffle else np.arange(n)
    end = (n // batch_size) * batch_size if drop_last else n
    for start in range(0, end, batch_size):
        yield idx[start: start + batch_size]


class DataLoader:
    """Host loader over a dataset (data.py:51-71)."""

    def __init__(self, dataset, batch_size, shuffle=False, drop_last=True, seed=0, collate_fn=None):
        self.dataset = dataset
        self.batch_size = batch_size
        self.shuffle = shuffle
        self.drop_last = drop_last
        self.collate_fn = collate_fn if collate_fn is not None else default_collate
        self.rng = np.random.default_rng(seed)

    def __iter__(self):
        for batch_idx in _batches(self.rng, len(self.dataset), self.batch_size, self.shuffle, self.drop_last):
            yield self.collate_fn([self.dataset[int(i)] for i in batch_idx])


class DeviceTokenLoader:
    """(x, y) Int64 device tensors of shape [batch, max_seq_len], batch for
    batch equal to ``DataLoader(TokenWindowDataset(tokens, max_seq_len),
    batch_size, shuffle, drop_last, seed)`` followed by ``to_device_batch``
    (train.py:99-102).  ``tokens`` is a path to a token file, a numpy array
    or an Int64 device tensor; it is uploaded once."""

    def __init__(self, tokens, max_seq_len, batch_size, shuffle=False, drop_last=True, seed=0,
                 device=None):
        device = device if device is not None else _core.Device.CUDA
        if isinstance(tokens, (str, Path)):
            tokens = read_tokens(tokens)
        if isinstance(tokens, np.ndarray):
            n = int(tokens.shape[0])
            tokens = _core.from_numpy(np.ascontiguousarray(tokens, dtype=np.int64)).to(device)
        else:
            if tokens.dtype != _core.DType.Int64 or len(tokens.shape) != 1:
                raise ValueError("DeviceTokenLoader: tokens must be a 1D Int64 tensor")
            n = int(tokens.shape[0])
        if n <= max_seq_len:
            raise ValueError("DeviceTokenLoader: token stream shorter than one window")
        self.tokens = tokens
        self.n_tokens = n
        self.max_seq_len = max_seq_len
        self.batch_size = batch_size
        self.shuffle = shuffle
        self.drop_last = drop_last
        self.rng = np.random.default_rng(seed)

    def __len__(self):
        n = self.n_tokens - self.max_seq_len
        return n // self.batch_size if self.drop_last else -(-n // self.batch_size)

    def batch(self, starts):
        """(x, y) for explicit window starts (host int64 array)."""
        s = _core.from_numpy(np.ascontiguousarray(starts, dtype=np.int64))
        return _core._token_windows(self.tokens, s, self.max_seq_len)

    def __iter__(self):
        n = self.n_tokens - self.max_seq_len
        for batch_idx in _batches(self.rng, n, self.batch_size, self.shuffle, self.drop_last):
            yield self.batch(batch_idx)
