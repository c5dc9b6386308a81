"""Build libmoe_gpu.so (HIP kernels + C ABI) for gfx950 with hipcc, in-tree.

Usage: python npu-offload_amd/build.py   (also called by __graft_entry__.build()).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libmoe_gpu.so")
CK_LIB = os.path.join(LIBDIR, "libck_gpu.so")  # the reference's cpu_kern.c boundary (ck_*) served by libmoe_gpu
ARCH = os.environ.get("MOE_GPU_ARCH", "gfx950")

# -packed-fp32-ops: keep hipcc from emitting packed fp32 VALU ops (v_pk_fma_f32 & co).
HIPCC_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


# The kernel source is compiled as parts in parallel (its token-bucket kernels dominate the compile time): part 0
# holds everything else, part N only the kernels of token bucket N (MOE_PART in moe_kernels.hip).
KERNEL_PARTS = [0, 1, 2, 4, 8, 16]


def _jobs():
    """(source, defines, object) for every object of the library."""
    obj = os.path.join(PKG, "build")
    jobs = [(os.path.join(CSRC, "moe_gpu_api.hip"), [], os.path.join(obj, "moe_gpu_api.o")),
            (os.path.join(CSRC, "lm_head.hip"), [], os.path.join(obj, "lm_head.o")),
            (os.path.join(CSRC, "attn_decode.hip"), [], os.path.join(obj, "attn_decode.o")),
            (os.path.join(CSRC, "dense_ops.hip"), [], os.path.join(obj, "dense_ops.o")),
            (os.path.join(CSRC, "decode_model.hip"), [], os.path.join(obj, "decode_model.o")),
            (os.path.join(CSRC, "st_loader.cpp"), [], os.path.join(obj, "st_loader.o"))]
    for part in KERNEL_PARTS:
        jobs.append((os.path.join(CSRC, "moe_kernels.hip"), [f"-DMOE_PART={part}"],
                     os.path.join(obj, f"moe_kernels_part{part}.o")))
    return jobs


def build(verbose: bool = False) -> str:
    os.makedirs(LIBDIR, exist_ok=True)
    os.makedirs(os.path.join(PKG, "build"), exist_ok=True)
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    procs = []
    for src, defs, obj in _jobs():
        cmd = [hipcc(), f"--offload-arch={ARCH}", *HIPCC_FLAGS, *defs, *inc, "-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = False
    for cmd, pr in procs:
        out, _ = pr.communicate()
        if pr.returncode != 0:
            failed = True
            sys.stderr.write(" ".join(cmd) + "\n" + out)
        elif verbose and out.strip():
            sys.stderr.write(out)
    if failed:
        raise RuntimeError("hipcc failed")
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *[o for _, _, o in _jobs()], "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc link failed ({r.returncode})")
    os.replace(tmp, LIB)
    build_ck_shim(verbose)
    return LIB


def build_ck_shim(verbose: bool = False) -> str:
    """libck_gpu.so: host code only, linked against libmoe_gpu.so next to it (rpath $ORIGIN)."""
    tmp = CK_LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-fPIC", "-shared", "-I", os.path.join(ROOT, "include"),
           os.path.join(CSRC, "ck_shim.cpp"), "-L", LIBDIR, "-lmoe_gpu", "-Wl,-rpath,$ORIGIN", "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed on ck_shim.cpp ({r.returncode})")
    os.replace(tmp, CK_LIB)
    return CK_LIB


if __name__ == "__main__":
    print(build(verbose=True))
