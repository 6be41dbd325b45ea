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
    """Each source compiled to an object in parallel (separate code objects, no device-side linking), then linked."""
    from concurrent.futures import ThreadPoolExecutor

    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    out = PKG / "libllmoe.so"
    tmp = out.with_suffix(".so.tmp")
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    inc = [f"-I{ROOT / 'include'}", f"-I{CSRC}"]
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]

    def compile_one(src: str):
        obj = objdir / (src + ".o")
        cmd = [hipcc, *compile_flags, *inc, "-c", str(CSRC / src), "-o", str(obj)]
        return src, obj, subprocess.run(cmd, capture_output=True, text=True, timeout=900)

    jobs = max(1, min(len(SOURCES), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(compile_one, SOURCES))
    for src, _, r in results:
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError(f"hipcc failed on {src}")
        if verbose:
            sys.stderr.write(r.stderr)
    r = subprocess.run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *[str(o) for _, o, _ in results], "-o",
                        str(tmp)], capture_output=True, text=True, timeout=900)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("linking libllmoe.so failed")
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
