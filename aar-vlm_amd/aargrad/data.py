"""Token data of the language-model training loop: the reference Shakespeare
pipeline's on-disk formats, its dataset/loader classes, and a loader that
keeps the token stream in device memory.

Formats (python/shakespeare/scripts/prepare.py:37-47, data.py:7-33):
  * ``meta.json``: ``{"vocab": [...], "vocab_size": N}``; a token id is the
    character's index in ``vocab``.
  * ``train.bin`` / ``val.bin``: the ids as raw little-endian int64, no
    header (read as ``np.memmap(path, dtype=np.int64)``, train.py:148-149).

``CharTokenizer``, ``TokenWindowDataset``, ``default_collate`` and
``DataLoader`` keep the interface of the reference pipeline's classes
(data.py:7-71): same arguments, same ids, same windows, same shuffle order for
a seed.  ``DeviceTokenLoader`` yields exactly the batches that
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
    """Character vocabulary (the ``meta.json`` format).  A token id is the
    character's position in ``vocab``; ``from_text`` sorts the distinct
    characters, so ids follow code-point order.  ``stoi`` / ``itos`` map
    characters to ids and back.  Encoding and decoding are vectorised through
    a code-point lookup table; an unknown character or id raises KeyError."""

    def __init__(self, vocab):
        self.vocab = list(vocab)
        self.stoi = dict(zip(self.vocab, range(len(self.vocab))))
        self.itos = dict(enumerate(self.vocab))
        single = all(isinstance(c, str) and len(c) == 1 for c in self.vocab)
        if single and self.vocab:
            cps = np.fromiter((ord(c) for c in self.vocab), dtype=np.int64, count=len(self.vocab))
            self._lut = np.full(int(cps.max()) + 1, -1, dtype=np.int64)
            self._lut[cps] = np.arange(len(self.vocab), dtype=np.int64)
        else:
            self._lut = None
        self._chars = np.array(self.vocab, dtype=object)

    @classmethod
    def from_text(cls, text):
        return cls(sorted(set(text)))

    @classmethod
    def load(cls, path):
        return cls(json.loads(Path(path).read_text())["vocab"])

    def save(self, path):
        Path(path).write_text(json.dumps({"vocab": self.vocab, "vocab_size": len(self.vocab)}))

    @property
    def vocab_size(self):
        return len(self.vocab)

    def encode(self, s):
        try:
            raw = s.encode("utf-32-le") if self._lut is not None else None
        except UnicodeEncodeError:  # lone surrogates: look them up one by one
            raw = None
        if raw is None:
            return np.array([self.stoi[c] for c in s], dtype=np.int64)
        cps = np.frombuffer(raw, dtype="<u4").astype(np.int64)
        ids = np.full(cps.shape, -1, dtype=np.int64)
        known = cps < self._lut.size
        ids[known] = self._lut[cps[known]]
        if (ids < 0).any():
            raise KeyError(chr(int(cps[np.argmax(ids < 0)])))
        return ids

    def decode(self, ids):
        idx = np.asarray(ids, dtype=np.int64).reshape(-1)
        bad = (idx < 0) | (idx >= len(self.vocab))
        if bad.any():
            raise KeyError(int(idx[np.argmax(bad)]))
        return "".join(self._chars[idx])


class TokenWindowDataset:
    """Sample i of a token stream: the window tokens[i : i + T + 1] split into
    ``input`` (its first T tokens) and ``target`` (its last T), int64; there
    are len(tokens) - T samples.  Negative indices count from the end; indices
    outside the dataset raise IndexError."""

    def __init__(self, tokens, max_seq_len):
        self.tokens = tokens
        self.max_seq_len = max_seq_len

    def __len__(self):
        return len(self.tokens) - self.max_seq_len

    def __getitem__(self, i):
        n = len(self)
        i = int(i) + (n if i < 0 else 0)
        if not 0 <= i < n:
            raise IndexError(f"TokenWindowDataset: index out of range for {n} windows")
        window = np.asarray(self.tokens[i: i + self.max_seq_len + 1], dtype=np.int64)
        return {"input": window[:-1], "target": window[1:]}


def default_collate(batch):
    """A list of equal-shaped sample dicts -> one dict of stacked arrays (the
    batch dimension first), keys in the first sample's order."""
    first = batch[0]
    out = {}
    for key, value in first.items():
        value = np.asarray(value)
        stacked = np.empty((len(batch),) + value.shape, dtype=value.dtype)
        for row, sample in enumerate(batch):
            stacked[row] = sample[key]
        out[key] = stacked
    return out


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
