"""Builds libfish_hip.so in-tree: hipcc for gfx950, one object per source."""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libfish_hip.so")
BUILD = os.path.join(HERE, "_build")
SOURCES = ["quantize.hip", "repack.hip", "gemv.hip", "batch.hip", "gemm.hip", "moe.hip", "dqmm.hip", "span.hip",
           "noalloc.hip", "capi.cpp", "pack.cpp"]
# code whose float rounding must follow FISH's baseline x86-64 build step by
# step (no fused multiply-add): the host weight packer, the expert routing
# softmax / combine, the f32-path dequantisers and the layer-span steps
NO_CONTRACT = {"pack.cpp", "moe.hip", "dqmm.hip", "span.hip"}
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    "-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}",
    # correctly rounded f32 division and reciprocal, denormals kept: the
    # activation scales must be bit-identical to FISH's CPU quantizer
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero", "-ffp-contract=fast",
    # no packed-FP32 instructions anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


# Per-file additions. batch.hip: MFMA results in VGPRs, read directly by the
# integer scaling that follows each MFMA (no accumulator-register copies).
EXTRA = {"batch.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    flags = [f for f in FLAGS if not (src in NO_CONTRACT and f.startswith("-ffp-contract"))]
    if src in NO_CONTRACT:
        flags.append("-ffp-contract=off")
    flags += EXTRA.get(src, [])
    cmd = [HIPCC, *flags, *lang, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT + ".tmp"
    r = subprocess.run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp, *objs],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, OUT)
    if verbose:
        print("built", OUT)
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
