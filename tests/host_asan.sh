#!/bin/bash
# Host AddressSanitizer/UBSan run of the C ABI (CPU only, no GPU needed).
# Builds libbtl.so's host code and the oracle with the sanitizers
# (bitnet_tt/_build.py --asan, oracle/Makefile asan), then runs the CPU tests
# that drive the library's host paths -- argument checks, size and planning
# queries, layouts, the co-residency rule -- and the oracle pins, with the
# clang sanitizer runtime preloaded into the (uninstrumented) interpreter.
set -euo pipefail
REPO="$(cd "$(dirname "$0")/.." && pwd)"
cd "$REPO"
python3 bitnet-tt_amd/bitnet_tt/_build.py --asan > /dev/null
make -s -C oracle asan
RT="$(/opt/rocm/llvm/bin/clang -print-file-name=libclang_rt.asan-x86_64.so)"
export BTL_LIBRARY="$REPO/bitnet-tt_amd/bitnet_tt/_lib/libbtl_hostasan.so"
export BTL_ORACLE_LIBRARY="$REPO/oracle/_asan/liboracle.so"
# the interpreter itself is not instrumented: leaks at exit are its own
export ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1"
export UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1"
# the instrumented builds are the ones the interpreter loads
LD_PRELOAD="$RT" PYTHONPATH="$REPO/bitnet-tt_amd:$REPO" python3 - <<'PY'
import ctypes
from bitnet_tt import _native as N
from oracle import oracle as O
N.lib(), O.lib()
maps = open("/proc/self/maps").read()
assert "libbtl_hostasan.so" in maps and "_asan/liboracle.so" in maps, "sanitized builds not loaded"
ctypes.CDLL(None).__asan_init  # the sanitizer runtime is in the process
print("host ASan/UBSan builds of libbtl.so and the oracle loaded")
PY
LD_PRELOAD="$RT" python3 -m pytest -q -p no:cacheprovider tests/test_capi.py tests/test_oracle_pins.py "$@"
