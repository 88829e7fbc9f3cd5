"""Builds librsllm_hip.so (gfx950) in-tree with hipcc.

Each .hip source is compiled to an object in rsllm_amd/_build/ and linked
into rsllm_amd/librsllm_hip.so. Flags:
  --offload-arch=gfx950          CDNA4 only
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                 no v_pk_*_f32 generation
  -O3 -fPIC -std=c++17
prefill.hip additionally gets -mllvm -amdgpu-mfma-vgpr-form: MFMA
accumulators are allocated in VGPRs (the kernel fits in 256), which keeps
the accumulate-in-place form and avoids accumulator copies between MFMAs.
Run: python -m rsllm_amd.build  (or __graft_entry__.build()).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "librsllm_hip.so")

SOURCES = ["abi.hip", "dequant.hip", "gemv.hip", "gemv_mfma.hip", "prefill.hip", "moe.hip",
           "q8_int8.hip", "residency.hip", "probe.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


EXTRA_FLAGS = {
    "prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "gemv_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o",
           obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
