"""Builds the in-tree libraries of the MI355X path.

    python -m cllm_inference_amd.build        (or __graft_entry__.build())

Outputs, next to the sources so they travel with the repository snapshot:
    cllm_inference_amd/libcllm_hip.so    HIP kernels + the C ABI (include/cllm_hip.h)
    cllm_inference_amd/libcllm_quant.so  the C++20 Quant API (include/cllm/core/quant.hpp)
                                         over that C ABI
Every .hip file is compiled for gfx950 only. Packed-fp32 instructions are disabled in all
device code.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
HIP_SOURCES = ["k_quantize.hip", "k_gemv.hip", "k_gemm.hip", "k_gemm16.hip", "k_gemmw.hip", "k_gemm_sm.hip", "k_gemv_f.hip", "k_producers.hip", "k_attention.hip", "k_read.hip", "gguf_file.cpp", "capi.hip"]
HIP_FLAGS = [
    "-O3", "-std=c++20", "--offload-arch=gfx950", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: the kernels consume them with VALU instructions, which cannot
    # read the accumulation registers (each use would cost a v_accvgpr_read)
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-I" + CSRC, "-I" + os.path.join(ROOT, "include"),
]
LIB_HIP = os.path.join(PKG, "libcllm_hip.so")
LIB_QUANT = os.path.join(PKG, "libcllm_quant.so")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + proc.stdout + proc.stderr)
        raise RuntimeError(f"build step failed: {cmd[0]} {cmd[-1]}")


def _compile(src: str) -> str:
    out = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", out])
    return out


def build(verbose: bool = False) -> None:
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(4, len(HIP_SOURCES))) as ex:
        objs = list(ex.map(_compile, HIP_SOURCES))
    tmp = LIB_HIP + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB_HIP)
    cxx = shutil.which("clang++") or shutil.which("g++")
    tmp = LIB_QUANT + ".tmp"
    _run([cxx, "-std=c++20", "-O2", "-fPIC", "-shared", "-Wall",
          "-I" + os.path.join(ROOT, "include"), os.path.join(CSRC, "quant_api.cpp"),
          "-o", tmp, "-L" + PKG, "-lcllm_hip", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, LIB_QUANT)
    if verbose:
        print("built", LIB_HIP, LIB_QUANT)


if __name__ == "__main__":
    build(verbose=True)
