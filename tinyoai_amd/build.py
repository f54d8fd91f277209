"""Builds libtinyoai_hip.so in-tree with hipcc for gfx950.

Every source is compiled as HIP with contraction off (explicit fmaf in the
hot loops, exact rounding elsewhere) and packed-fp32 instruction selection
disabled. Objects go to tinyoai_amd/_build/, the library next to this file.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libtinyoai_hip.so")
ARCH = os.environ.get("TINYOAI_OFFLOAD_ARCH", "gfx950")

# The streaming matrix-vector kernels come one weight format per file
# (matvec_<format>.hip), so they compile in parallel.
MATVEC_FORMATS = ["q8_0", "bf16", "f32", "f16", "q5_1", "q4_k", "q5_k", "q6_k"]
SOURCES = ["decode.hip", "api.cpp", "llama.cpp", "prefill.hip", "weights.hip", "gemm.hip", "gemm_q8.hip",
           "flash.hip", "logprobs.hip", "kq_rows.hip", "llama_tiny.hip"] + [f"matvec_{f}.hip" for f in MATVEC_FORMATS]
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-x", "hip", f"--offload-arch={ARCH}", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-value", "-Wno-unused-result",
         "-I", os.path.join(ROOT, "include"), "-I", CSRC]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


# Per-source additions: the Q8_0 wide-tile kernel keeps its matrix-core
# results in ordinary vector registers (each quant block's products are
# rescaled on the vector unit, which cannot read the accumulation
# registers); the BF16 kernels keep theirs in the accumulation registers.
EXTRA = {"gemm_q8.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *FLAGS, *EXTRA.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(os.cpu_count() or 8, 16, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    # -z defs: a symbol left undefined (a source missing from SOURCES) fails
    # the link here instead of the load on the device host.
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
