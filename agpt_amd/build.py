"""Builds the native libraries in-tree.

  agpt_amd/lib/libagpt_attn.so  HIP kernels + C ABI (include/agpt_attn.h), gfx950
  agpt_amd/lib/libagpt_trie.so  host-only corpus / trie builder (include/agpt_trie.h)

Run `python -m agpt_amd.build` (or __graft_entry__.build()). hipcc cross-compiles
for gfx950 without a GPU.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
ARCH = os.environ.get("AGPT_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed-FP32 instructions are disabled for every HIP object: some of their
# forms have given silently wrong results on the MI355X pool this targets.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Matrix-instruction accumulators in ordinary VGPRs: the kernels rescale
    # and read them between steps, which the AGPR form turns into copies.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # One lane takes each scheduling ticket; combining the lanes' atomics
    # would make the wave wait for the ticket right where it is issued.
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    # No kernel result depends on NaN handling; without IEEE mode the float
    # max/min of the softmax need no NaN-quieting instructions.
    "-fno-honor-nans", "-Xarch_device", "-mno-amdgpu-ieee",
    "-Wall",
    "-Wno-unused-result",
]

HIP_SOURCES = ["trie_attn.hip", "varlen_attn.hip", "agpt_loss.hip", "agpt_block.hip"]


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_trie_lib() -> Path:
    LIB.mkdir(exist_ok=True)
    out = LIB / "libagpt_trie.so"
    _run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall",
          str(CSRC / "trie_build.cpp"), "-o", str(out)])
    return out


def build_attn_lib() -> Path:
    LIB.mkdir(exist_ok=True)
    objs = []
    for src in HIP_SOURCES:
        obj = LIB / (Path(src).stem + ".o")
        _run([HIPCC, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(str(obj))
    out = LIB / "libagpt_attn.so"
    tmp = LIB / "libagpt_attn.so.tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_trie_lib()
    build_attn_lib()


if __name__ == "__main__":
    build_all()
    sys.exit(0)
