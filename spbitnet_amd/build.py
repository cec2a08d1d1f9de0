"""Builds the gfx950 HIP library in-tree: spbitnet_amd/libspbitnet_amd.so.

hipcc compiles every spbitnet_amd/csrc/*.hip source for gfx950 only, with
packed-FP32 instruction selection disabled, and links one shared library
whose exported symbols are the C ABI declared in include/spbitnet_amd.h.
"""
from __future__ import annotations

import concurrent.futures
import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB = os.path.join(PKG, "libspbitnet_amd.so")
ARCH = os.environ.get("SPB_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Every float32 step rounds on its own, as in the reference: no mul+add
    # contraction and no fused multiply-and-narrow (v_fma_mix*) conversions.
    "-ffp-contract=off",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]


def sources():
    return sorted(glob.glob(os.path.join(PKG, "csrc", "*.hip")))


def build(verbose: bool = False) -> str:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    objdir = os.path.join(PKG, "_build")
    os.makedirs(objdir, exist_ok=True)
    def compile_one(src):
        obj = os.path.join(objdir, os.path.basename(src) + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, "-c", src, "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        msgs = [l for l in (r.stderr or "").splitlines() if "packed-fp32-ops" not in l]
        return src, obj, cmd, r.returncode, msgs

    # one hipcc per source, in parallel (engine.hip alone takes ~20 s)
    jobs = min(len(sources()), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        results = list(pool.map(compile_one, sources()))
    objs = []
    for src, obj, cmd, rc, msgs in results:
        if verbose:
            print(" ".join(cmd), flush=True)
        if rc != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n" + "\n".join(msgs))
        if verbose and msgs:
            print("\n".join(msgs))
        objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
