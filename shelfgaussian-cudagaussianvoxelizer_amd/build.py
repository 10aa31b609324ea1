"""Builds libg2v_hip.so (the gfx950 HIP kernels + C ABI) in-tree, next to the Python package.

    python shelfgaussian-cudagaussianvoxelizer_amd/build.py

hipcc cross-compiles for gfx950 without a GPU.  Packed FP32 instructions are disabled
(-packed-fp32-ops): hipcc would otherwise form v_pk_* FP32 operations from scalar code.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "CudaGaussianVoxelizer", "libg2v_hip.so")
SOURCES = ["g2v_csr.hip", "g2v_forward.hip", "g2v_backward.hip", "g2v_cosine.hip", "g2v_covariance.hip", "g2v_capi.hip", "g2v_profile.hip"]
ARCH = os.environ.get("G2V_OFFLOAD_ARCH", "gfx950")


def hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def build(verbose: bool = False) -> str:
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-Wno-unused-command-line-argument", "-o", tmp] + [os.path.join(CSRC, s) for s in SOURCES]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with exit code {res.returncode}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
