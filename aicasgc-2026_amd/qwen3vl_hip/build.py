"""Build recipe for the C-ABI decode library (``libqwen3vl_decode.so``).

hipcc cross-compiles the HIP sources under ``csrc/`` for gfx950 into one
shared object placed next to the package (in-tree, so it travels with the
source tree to the GPU host).  No GPU is needed to build.

    python -m qwen3vl_hip.build          # from the aicasgc-2026_amd directory
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent.parent          # aicasgc-2026_amd/
CSRC = PKG_ROOT / "csrc"
LIB_NAME = "libqwen3vl_decode.so"
LIB_PATH = PKG_ROOT / LIB_NAME
TRACE_LIB_PATH = PKG_ROOT / "libqwen3vl_decode_trace.so"   # same sources with -DQD_TRACE
SOURCES = ["qd_gemv.hip", "qd_attention.hip", "qd_small_ops.hip", "qd_persistent.hip", "qd_batch.hip", "qd_capi.hip"]
ARCH = os.environ.get("QD_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
    # packed fp32 ops stay disabled for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def build(verbose: bool = False, trace: bool = False) -> Path:
    """Compile every HIP source into LIB_PATH (always recompiles).  With
    ``trace`` the persistent step records its phase timestamps
    (-DQD_TRACE) and the library goes to TRACE_LIB_PATH instead."""
    out = TRACE_LIB_PATH if trace else LIB_PATH
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, *(["-DQD_TRACE"] if trace else []), "-I", str(PKG_ROOT.parent / "include"),
           *[str(CSRC / s) for s in SOURCES], "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    if verbose and res.stderr.strip():
        print(res.stderr, file=sys.stderr)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True, trace="--trace" in sys.argv))
