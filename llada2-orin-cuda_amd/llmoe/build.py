"""Build libllmoe.so for gfx950 in-tree (hipcc), and optionally the CPU checker under oracle/.

    python -m llmoe.build            (from llada2-orin-cuda_amd/)
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent.parent
CSRC = PKG.parent / "csrc"
SOURCES = ["api.hip", "expert_gemm.hip", "tiled_gemm.hip", "act.hip", "route.hip", "relayout.hip", "dense.hip", "loader.cpp"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # the fp32 operation order is part of the numerical contract with the CPU checker
    "-ffp-contract=off",
    # no packed-fp32 instructions (v_pk_*_f32) anywhere in this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    # MFMA accumulators in VGPRs (no accvgpr copies around every MFMA)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def build_library(verbose: bool = False) -> Path:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    out = PKG / "libllmoe.so"
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc, *HIPCC_FLAGS, f"-I{ROOT / 'include'}", f"-I{CSRC}", *[str(CSRC / s) for s in SOURCES], "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed building libllmoe.so")
    if verbose:
        sys.stderr.write(r.stderr)
    os.replace(tmp, out)
    return out


def build_oracle() -> Path:
    r = subprocess.run(["make", "-B", "-s", "-C", str(ROOT / "oracle")], capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("building the CPU checker failed")
    return ROOT / "oracle" / "libmoe_oracle.so"


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))
    print(build_oracle())
