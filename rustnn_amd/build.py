"""Builds librnn.so (the HIP product library) in-tree for gfx950.

Usage: python -m rustnn_amd.build   (or rustnn_amd.build.build())

Every .hip file under csrc/ is compiled with hipcc for gfx950 only, then linked
into rustnn_amd/librnn.so, which travels with the source tree.  Packed FP32
VALU ops are disabled (-packed-fp32-ops): the kernels compute on MFMA and plain
scalar VALU only.  Floating-point contraction is off (-ffp-contract=off):
a * b + c in the elementwise and reduction code rounds the product, then the
sum, as the reference's Rust does (it never fuses a multiply-add unless
written with mul_add), so results that feed a comparison -- the ReLU masks
after BatchNorm, the max of a softmax row -- round as the reference's do.
The matrix products run on MFMA builtins, which contraction does not touch.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "librnn.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

CFLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-ffp-contract=off",
    "-Wno-unused-function", "-Wno-unused-variable",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(HERE, "..", "include"),
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    errs = [ln for ln in r.stderr.splitlines() if "warning" in ln and "packed-fp32" not in ln
            and "target-feature" not in ln]
    if errs:
        sys.stderr.write("\n".join(errs[:20]) + "\n")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
