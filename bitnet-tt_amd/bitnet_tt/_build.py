"""Build recipe of libbtl.so (the gfx950 BitLinear library).

``build_native()`` compiles every HIP source under ``csrc/`` with hipcc for
gfx950 into ``bitnet_tt/_lib/libbtl.so`` (in-tree, so it travels with the
package).  It runs on a machine without a GPU: hipcc cross-compiles.
"""

from __future__ import annotations

import glob
import os
import subprocess

_PKG = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_PKG)  # bitnet-tt_amd/
_REPO = os.path.dirname(_ROOT)
CSRC = os.path.join(_ROOT, "csrc")
INCLUDE = os.path.join(_REPO, "include")
OUT = os.path.join(_PKG, "_lib", "libbtl.so")
# Measurement build: the same sources with -DBTL_TRACE (phase timestamps of the
# persistent decode step, read by bench.py --step-trace).  Not loaded otherwise.
OUT_TRACE = os.path.join(_PKG, "_lib", "libbtl_trace.so")
# Host-sanitizer build: the host code (argument checks, planning, layouts)
# instrumented with AddressSanitizer and UBSan; device code as in the product
# build.  Loaded only by tests/host_asan.sh (BTL_LIBRARY) on the CPU.
OUT_ASAN = os.path.join(_PKG, "_lib", "libbtl_hostasan.so")
ASAN_FLAGS = ["-Xarch_host", "-fsanitize=address,undefined", "-Xarch_host", "-fno-sanitize-recover=undefined",
              "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-g"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Every float multiply and add is rounded on its own: the kernels' numeric
    # contract (RMS statistic order, epilogue rounding) depends on it.
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # No packed fp32 instructions in device code.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    return "hipcc"


def build_native(verbose: bool = False, trace: bool = False, asan: bool = False) -> str:
    """Compile libbtl.so (trace=True: the -DBTL_TRACE measurement build,
    libbtl_trace.so; asan=True: the host-sanitizer build, libbtl_hostasan.so)."""
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    out = OUT_TRACE if trace else OUT_ASAN if asan else OUT
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    extra = (["-DBTL_TRACE"] if trace else []) + (ASAN_FLAGS if asan else [])
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, f"-I{INCLUDE}", "-o", tmp, *sources]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    errs = "\n".join(ln for ln in proc.stderr.splitlines() if noise not in ln)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{' '.join(cmd)}\n{errs}")
    if verbose and errs.strip():
        print(errs)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    import sys

    print(build_native(verbose=True, trace="--trace" in sys.argv[1:], asan="--asan" in sys.argv[1:]))
