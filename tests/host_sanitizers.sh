#!/bin/bash
# Host-side AddressSanitizer + UndefinedBehaviorSanitizer run of the CPU test
# suite.  The host C++ of aargrad._core (tensors, views, autograd, validation,
# error translation, allocator bookkeeping) is rebuilt with g++
# -fsanitize=address,undefined in a scratch copy of the repository and the
# `-m "not gpu"` tests run against it with the sanitizer runtimes preloaded
# (the Python interpreter itself is not instrumented).  No HIP code is built
# with a sanitizer; the GPU library is used as built.
#
#   bash tests/host_sanitizers.sh [scratch-dir]
set -euo pipefail
REPO="$(cd "$(dirname "$0")/.." && pwd)"
WORK="${1:-/tmp/aar_host_sanitizers}"
rm -rf "$WORK" && mkdir -p "$WORK/repo" "$WORK/obj"
(cd "$REPO" && tar --exclude=./.git --exclude=./_work --exclude=./gpurun_out -cf - .) | tar -xf - -C "$WORK/repo"
cd "$WORK/repo/aar-vlm_amd"
test -f aargrad/libaar_hip.so || { echo "build the package first (__graft_entry__.build())" >&2; exit 1; }
PYINC=$(python -c 'import sysconfig; print(sysconfig.get_paths()["include"])')
PBINC=$(python -c 'import pybind11; print(pybind11.get_include())')
for f in csrc/host/*.cpp; do
  g++ -O1 -g -fno-omit-frame-pointer -fsanitize=address,undefined -std=c++20 -fPIC -Wall -Wno-sign-compare \
      -I../include -Icsrc/host -I"$PBINC" -I"$PYINC" -fvisibility=hidden -c "$f" -o "$WORK/obj/$(basename "$f").o" &
done
wait
CORE=$(ls aargrad/_core*.so)
g++ -shared -fPIC -fsanitize=address,undefined "$WORK"/obj/*.o -Laargrad -laar_hip -Wl,-rpath,'$ORIGIN' -o "$CORE"
nm -D "$CORE" | grep -q __asan_report || { echo "sanitizer instrumentation missing" >&2; exit 1; }
cd "$WORK/repo"
ASAN_OPTIONS=detect_leaks=0:halt_on_error=1 UBSAN_OPTIONS=print_stacktrace=1:halt_on_error=1 \
LD_PRELOAD="$(gcc -print-file-name=libasan.so):$(gcc -print-file-name=libubsan.so)" \
  python -m pytest tests -q -m "not gpu" -p no:cacheprovider
