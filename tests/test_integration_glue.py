"""CPU checks of the reference-side glue (oracle/hip_backend.cpp), the file a
reference maintainer adds as cppsrc/ops/hip_backend.cpp to run the reference on
libaar_hip.so.

oracle/Makefile compiles it against the reference's own headers, with the
reference's CPU sources and ref_driver.cpp, into oracle/_ref/libaar_glue.so,
linked with --no-undefined against libaar_hip.so.  These tests check that:
  * the build succeeds (so every device function the reference's C++ calls
    has a definition, and every aar_* call resolves in libaar_hip.so);
  * the glue defines exactly the functions the reference's *_cuda_stub.cpp,
    cuda_allocator_stub.cpp and cuda_copy_stub.cpp define, with the same
    signatures (compared as demangled symbols), so it replaces them one for
    one (reference CMakeLists.txt:70-104);
  * every aar_* symbol it uses is declared in include/aar_hip.h and exported
    by libaar_hip.so;
  * without a GPU its ops fail with an error rather than computing on the CPU.
"""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle as O

REPO = Path(__file__).resolve().parent.parent
OBJ = REPO / "oracle" / "_ref" / "obj"
HIP_LIB = REPO / "aar-vlm_amd" / "aargrad" / "libaar_hip.so"
HEADER = REPO / "include" / "aar_hip.h"

pytestmark = pytest.mark.skipif(
    not Path("/root/reference/cppsrc").exists() or shutil.which("nm") is None,
    reason="needs the reference tree (its headers and CPU sources) and binutils",
)


@pytest.fixture(scope="module")
def glue():
    if not HIP_LIB.exists():
        pytest.skip("libaar_hip.so is not built")
    res = subprocess.run(["make", "-s", "-C", str(REPO / "oracle"), "-j8", "glue"], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout[-3000:] + res.stderr[-3000:]
    assert O.GLUE_PATH.exists()
    return O.GLUE_PATH


def _nm(args, path) -> list[str]:
    return subprocess.run(["nm", *args, str(path)], check=True, capture_output=True, text=True).stdout.splitlines()


def _text_symbols(paths) -> set[str]:
    """Demangled names of the global functions defined in `paths`."""
    out = set()
    for p in paths:
        for line in _nm(["-C", "--defined-only"], p):
            parts = line.split(" ", 2)
            if len(parts) == 3 and parts[1] == "T":
                out.add(parts[2])
    return out


def test_glue_replaces_every_stub(glue):
    stubs = sorted(OBJ.glob("*_stub.o"))
    assert len(stubs) == 14
    want = _text_symbols(stubs)
    got = _text_symbols([OBJ / "hip_backend.o"])
    assert any("matmul_cuda" in s for s in want) and any("cuda_allocator" in s for s in want)
    assert got == want, (sorted(want - got), sorted(got - want))


def test_glue_links_only_declared_exported_abi(glue):
    used = {line.split()[-1] for line in _nm(["-D", "-u"], glue) if line.split()[-1].startswith("aar_")}
    exported = {line.split()[-1] for line in _nm(["-D", "--defined-only"], HIP_LIB)}
    declared = set(re.findall(r"\b(aar_[a-z0-9_]+)\s*\(", HEADER.read_text()))
    assert {"aar_gemm_f32", "aar_flash_bwd_f32", "aar_layernorm_bwd_f32", "aar_malloc", "aar_memcpy"} <= used
    assert used <= exported, sorted(used - exported)
    assert used <= declared, sorted(used - declared)
    dyn = subprocess.run(["readelf", "-d", str(glue)], check=True, capture_output=True, text=True).stdout
    assert "libaar_hip.so" in dyn and "$ORIGIN/../../aar-vlm_amd/aargrad" in dyn


def test_glue_fails_without_a_gpu(glue):
    import aargrad

    if aargrad.device_available():
        pytest.skip("a GPU is visible: the device path runs (checked by the -m gpu glue tests)")
    a = np.ones((4, 4), np.float32)
    with O.reference_on_device():
        with pytest.raises(RuntimeError, match="reference matmul failed"):
            O.ref_matmul("nn", a, a)
    # the CPU build is untouched by the context
    assert np.array_equal(O.ref_matmul("nn", a, a), np.full((4, 4), 4.0, np.float32))
