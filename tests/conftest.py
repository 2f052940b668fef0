"""Shared test setup.

* Puts the repo root (for ``oracle``) and ``aar-vlm_amd`` (for ``aargrad``) on
  sys.path and builds what is missing (oracle libraries always; the HIP
  library and ``_core`` only when no built copy exists).
* Registers the ``gpu`` marker: those tests need an MI355X and call the HIP
  kernels through the C ABI (directly or via ``aargrad._core``).
* Tolerance helpers implement the parity bar: for each output both
  ``max|g-r| / max(max|r|, 1)`` and the normwise ``||g-r|| / ||r||`` must be
  <= tol, with tol = 1e-4*sqrt(K) for a GEMM of contraction length K and 1e-4
  for softmax, layernorm and attention outputs and gradients.
"""
from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "aar-vlm_amd"
for p in (str(REPO), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def _ensure_built() -> None:
    import oracle

    if not oracle.LIB_PATH.exists() or (not oracle.REF_PATH.exists() and Path("/root/reference/cppsrc").exists()):
        oracle.build()
    lib = PKG / "aargrad" / "libaar_hip.so"
    core = list((PKG / "aargrad").glob("_core*.so"))
    if not lib.exists() or not core:
        sys.path.insert(0, str(PKG))
        import build as pkg_build  # aar-vlm_amd/build.py

        pkg_build.build_all()


_ensure_built()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs the HIP kernels)")


def gpu_available() -> bool:
    import aargrad

    return aargrad.device_available()


@pytest.fixture(scope="session")
def ag():
    import aargrad

    return aargrad


@pytest.fixture(scope="session")
def gpu(ag):
    if not ag.device_available():
        pytest.skip("no GPU visible")
    return ag


def errs(g, r):
    """(max |g-r| / max(max|r|,1), ||g-r||/||r||) in float64."""
    g = np.asarray(g, np.float64)
    r = np.asarray(r, np.float64)
    assert g.shape == r.shape, (g.shape, r.shape)
    if r.size == 0:
        return 0.0, 0.0
    d = np.abs(g - r)
    mixed = float(d.max() / max(np.abs(r).max(), 1.0))
    nr = float(np.linalg.norm(r))
    normwise = float(np.linalg.norm(g - r) / nr) if nr > 0 else float(np.linalg.norm(g - r))
    return mixed, normwise


def assert_close(g, r, tol, what=""):
    mixed, normwise = errs(g, r)
    assert np.all(np.isfinite(np.asarray(g))), f"{what}: non-finite values"
    assert mixed <= tol and normwise <= tol, f"{what}: mixed {mixed:.3e} normwise {normwise:.3e} > tol {tol:.1e}"


def gemm_tol(K: int) -> float:
    return 1e-4 * float(np.sqrt(max(K, 1)))


TOL = 1e-4
