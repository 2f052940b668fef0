"""In-tree build of the MI355X backend.

Produces, next to the Python package (so a copy of the repository tree carries them):
  aargrad/libaar_hip.so   all HIP kernels + the C ABI (include/aar_hip.h), gfx950
  aargrad/_core<ext>.so   the pybind11 module aargrad._core (host C++), linked to
                          libaar_hip.so through an $ORIGIN rpath

hipcc builds the .hip sources; g++ builds the host C++ (no HIP headers needed,
it only sees the plain-C ABI).  Every call rebuilds what is out of date
(source or header newer than the object) and always relinks.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent          # aar-vlm_amd/
REPO = PKG_ROOT.parent
INCLUDE = REPO / "include"
HIP_DIR = PKG_ROOT / "csrc" / "hip"
HOST_DIR = PKG_ROOT / "csrc" / "host"
OUT_DIR = PKG_ROOT / "aargrad"
OBJ_DIR = PKG_ROOT / "_build"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = os.environ.get("AAR_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", f"-I{INCLUDE}", f"-I{HIP_DIR}",
    # packed fp32 VALU ops are disabled for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]
CXX_FLAGS = ["-O2", "-std=c++20", "-fPIC", "-Wall", "-Wno-sign-compare", f"-I{INCLUDE}", f"-I{HOST_DIR}"]

LIB_NAME = "libaar_hip.so"

# Per-file extra flags.  The flash-attention kernels rescale their MFMA
# accumulators with VALU ops every tile, so their accumulators are kept in
# arch VGPRs (no accvgpr copies in the loop); so do the short-operand GEMMs,
# whose few accumulators the compiler otherwise copied between AGPRs and
# VGPRs every k tile; the tiled GEMM keeps its 256-register accumulator tiles
# in AGPRs.
HIP_FILE_FLAGS = {
    "flash_attn": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "gemm_small": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _headers(d: Path, pattern: str) -> list[Path]:
    return sorted(d.glob(pattern))


def _stale(obj: Path, deps: list[Path]) -> bool:
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    return any(p.stat().st_mtime > t for p in deps)


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{res.stdout}")


def build_hip(force: bool = False, jobs: int = 8) -> Path:
    OBJ_DIR.mkdir(exist_ok=True)
    srcs = sorted(HIP_DIR.glob("*.hip"))
    hdrs = _headers(HIP_DIR, "*.hpp") + [INCLUDE / "aar_hip.h"]
    objs = []
    todo = []
    for s in srcs:
        o = OBJ_DIR / (s.stem + ".hip.o")
        objs.append(o)
        if force or _stale(o, [s] + hdrs):
            todo.append([HIPCC, *HIP_FLAGS, *HIP_FILE_FLAGS.get(s.stem, []), "-c", str(s), "-o", str(o)])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, todo))
    out = OUT_DIR / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_core(force: bool = False, jobs: int = 8) -> Path:
    import pybind11

    OBJ_DIR.mkdir(exist_ok=True)
    srcs = sorted(HOST_DIR.glob("*.cpp"))
    hdrs = _headers(HOST_DIR, "*.hpp") + [INCLUDE / "aar_hip.h"]
    py_inc = sysconfig.get_paths()["include"]
    flags = CXX_FLAGS + [f"-I{pybind11.get_include()}", f"-I{py_inc}", "-fvisibility=hidden"]
    objs = []
    todo = []
    for s in srcs:
        o = OBJ_DIR / (s.stem + ".cpp.o")
        objs.append(o)
        if force or _stale(o, [s] + hdrs):
            todo.append(["g++", *flags, "-c", str(s), "-o", str(o)])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, todo))
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = OUT_DIR / f"_core{suffix}"
    tmp = out.with_suffix(".so.tmp")
    _run(["g++", "-shared", "-fPIC", *map(str, objs), f"-L{OUT_DIR}", "-laar_hip",
          "-Wl,-rpath,$ORIGIN", "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_all(force: bool = False) -> None:
    build_hip(force)
    if any(HOST_DIR.glob("*.cpp")):
        build_core(force)


if __name__ == "__main__":
    build_all(force="--force" in sys.argv)
    print("built", OUT_DIR / LIB_NAME)
