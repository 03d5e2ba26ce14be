"""Builds the gfx950 HIP library libastro_moe.so in-tree (hipcc, no JIT cache).

Every HIP source is compiled with packed-FP32 instructions disabled
(-Xclang -target-feature -Xclang -packed-fp32-ops).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libastro_moe.so")
SOURCES = ["abi.hip", "gemm.hip", "route.hip", "decode.hip", "elementwise.hip", "synth.hip", "verify.hip",
           # MFMA results in VGPRs: its per-group affine terms are VALU work on the accumulators
           ("gemm_xq.hip", "gemm_xq", ["-Xarch_device", "-mllvm=-amdgpu-mfma-vgpr-form"])]
# decode_gate_up.hip holds most of the decode path's kernel instantiations: one object per
# (code width, token count), compiled in parallel with the rest
VARIANTS = [("decode_gate_up.hip", f"decode_gate_up_b{b}_mt{m}", [f"-DASTRO_GU_BITS={b}", f"-DASTRO_GU_MT={m}"])
            for b in (4, 8) for m in (1, 2, 4, 8)]
# host-only sources (no kernels): the host compiler, against the HIP runtime's C API
HOST_SOURCES = ["pages.cc", "status.cc"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HOSTCXX = os.environ.get("HOSTCXX", "g++")
HOST_FLAGS = ["-O2", "-fPIC", "-std=c++17", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__", "-I", "/opt/rocm/include"]
FLAGS = ["-O3", "--offload-arch=gfx950", "-fPIC", "-std=c++17", "-Wall",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I", os.path.join(os.path.dirname(HERE), "include")]


def _compile(job) -> str:
    src, name, defs = job if isinstance(job, tuple) else (job, os.path.splitext(job)[0], [])
    obj = os.path.join(BUILD, name + ".o")
    if src.endswith(".cc"):
        cmd = [HOSTCXX, *HOST_FLAGS, *defs, "-c", os.path.join(CSRC, src), "-o", obj]
    else:
        cmd = [HIPCC, *FLAGS, *defs, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"{cmd[0]} failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    jobs = VARIANTS + SOURCES + HOST_SOURCES  # the longest compiles first
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(_compile, jobs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
