"""Model checkpoints in the reference Shakespeare pipeline's format.

``<prefix>.npz`` holds one array per parameter, keyed ``p0..pN`` in
``Module.parameters()`` order; ``<prefix>.json`` holds the model config
(python/shakespeare/scripts/train.py:108-121, read back by inference.py:31-54).

The checkpoint shipped with the reference (``data/ckpt_final.*``) predates its
current scripts: its config names the context length ``block_size`` (the
scripts read ``max_seq_len``), and it carries the attention projections'
biases (29 arrays at n_layer=2, where the current model builds bias-free
attention and has 25).  ``read_checkpoint`` accepts both: it fills
``max_seq_len`` from ``block_size`` and reports ``attn_bias`` from the array
count, so a caller can build the matching model.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

from . import _core


def save_checkpoint(model, config, prefix) -> None:
    """Write ``<prefix>.npz`` (parameters as p0..pN) and ``<prefix>.json``
    (``config``, indented like the reference) (train.py:108-121)."""
    prefix = Path(prefix)
    arrays = [_core.to_numpy(p.tensor.to(_core.Device.CPU)) for p in model.parameters()]
    np.savez(prefix.with_suffix(".npz"), **{f"p{i}": a for i, a in enumerate(arrays)})
    with open(prefix.with_suffix(".json"), "w") as f:
        json.dump(dict(config), f, indent=2)


def _params_per_layer(attn_bias: bool) -> int:
    # ln1 (2), qkv (1 or 2), out (1 or 2), ln2 (2), fc1 (2), fc2 (2)
    return 12 if attn_bias else 10


def read_checkpoint(prefix):
    """(arrays in p0..pN order, config).  The config gains ``max_seq_len``
    from ``block_size`` when only the latter is present, and ``attn_bias``
    (whether the arrays include attention-projection biases) when the count
    decides it."""
    prefix = Path(prefix)
    with open(prefix.with_suffix(".json")) as f:
        cfg = json.load(f)
    if "max_seq_len" not in cfg and "block_size" in cfg:
        cfg["max_seq_len"] = cfg["block_size"]
    with np.load(prefix.with_suffix(".npz")) as data:
        keys = sorted(data.files, key=lambda k: int(k[1:]))
        arrays = [data[k] for k in keys]
    n_layer = cfg.get("n_layer")
    if isinstance(n_layer, int) and "attn_bias" not in cfg:
        for bias in (False, True):
            if len(arrays) == _params_per_layer(bias) * n_layer + 5:
                cfg["attn_bias"] = bias
    return arrays, cfg


def load_parameters(model, arrays, device) -> None:
    """Replace each parameter's tensor by the matching array on ``device``,
    requiring grad (inference.py:44-53); the counts must agree."""
    params = list(model.parameters())
    if len(params) != len(arrays):
        raise ValueError(f"param count mismatch: model has {len(params)}, ckpt has {len(arrays)}")
    for p, arr in zip(params, arrays):
        if tuple(p.tensor.shape) != tuple(np.shape(arr)):
            raise ValueError(f"param shape mismatch: model {tuple(p.tensor.shape)}, ckpt {tuple(np.shape(arr))}")
        new_t = _core.from_numpy(np.ascontiguousarray(arr, dtype=np.float32)).to(device)
        new_t.requires_grad = True
        p.tensor = new_t
