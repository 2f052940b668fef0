"""aargrad on the MI355X (gfx950) backend.

Same public names as the reference package (aargrad/__init__.py of
AARONKANG04/aar-vlm): the tensor type, enums, numpy I/O and the op functions
all come from the native module ``aargrad._core``, whose device computations
run in hand-written HIP kernels (``libaar_hip.so`` beside this file, C ABI in
``include/aar_hip.h``).  Importing fails loudly when the native module has not
been built; there is no Python or CPU fallback.
"""
from __future__ import annotations

try:
    from . import _core
except ImportError as exc:  # pragma: no cover - exercised only on a broken build
    raise ImportError(
        "aargrad._core is not built; run `python aar-vlm_amd/build.py` "
        "(or __graft_entry__.build()) first"
    ) from exc

from ._core import (  # noqa: E402
    Tensor,
    DType,
    Device,
    from_numpy,
    to_numpy,
    add,
    sub,
    mul,
    relu,
    gelu,
    sum_all,
    add_bias,
    scale,
    matmul,
    matmul_a_bt,
    matmul_at_b,
    softmax,
    layernorm,
    apply_causal_mask,
    reshape,
    transpose,
    slice,
    squeeze,
    unsqueeze,
    contiguous,
    bmm,
    bmm_a_bt,
    bmm_at_b,
    embedding,
    cross_entropy,
    dropout,
    manual_seed,
    scaled_add_inplace,
    adamw_step,
    flash_attention,
    cuda_synchronize,
)

from . import nn  # noqa: E402
from . import optim  # noqa: E402

__all__ = [
    "Tensor",
    "DType",
    "Device",
    "from_numpy",
    "to_numpy",
    "add",
    "sub",
    "mul",
    "relu",
    "gelu",
    "sum_all",
    "add_bias",
    "scale",
    "matmul",
    "matmul_a_bt",
    "matmul_at_b",
    "softmax",
    "layernorm",
    "apply_causal_mask",
    "reshape",
    "transpose",
    "slice",
    "squeeze",
    "unsqueeze",
    "contiguous",
    "bmm",
    "bmm_a_bt",
    "bmm_at_b",
    "embedding",
    "cross_entropy",
    "dropout",
    "manual_seed",
    "scaled_add_inplace",
    "adamw_step",
    "flash_attention",
    "cuda_synchronize",
    "nn",
    "optim",
]


def device_available() -> bool:
    """True when a GPU is visible to the HIP runtime."""
    return _core._device_count() > 0
