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

# Per-source flags. The trie kernels are scheduled for instruction-level
# parallelism: the block pair's S/dP products, softmax and dV/dK/dQ products
# interleave more deeply (C2 trie_bwd 33.95 -> 33.45 ms; the deep kernels
# within noise; the memory-clause strategy was 0.15 ms slower on C2 and
# 1 ms on C4). The loss kernel is 4 % slower that way and keeps the default.
SOURCE_FLAGS = {"trie_attn.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]}


# hipcc applies -Xclang options to the host pass too, whose x86 target does
# not know the AMDGPU feature and says so once per host compile; clang's
# -Xarch_device cannot forward an -Xclang pair, so the line is dropped here.
_HOST_NOISE = "'-packed-fp32-ops' is not a recognized feature for this target (ignoring feature)"


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(ln for ln in r.stdout.splitlines() if ln.strip() != _HOST_NOISE)
    if out.strip():
        print(out, flush=True)
    if r.returncode:
        raise subprocess.CalledProcessError(r.returncode, cmd)


def build_trie_lib() -> Path:
    LIB.mkdir(exist_ok=True)
    out = LIB / "libagpt_trie.so"
    _run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall",
          str(CSRC / "trie_build.cpp"), "-o", str(out)])
    return out


def build_attn_lib() -> Path:
    LIB.mkdir(exist_ok=True)
    from concurrent.futures import ThreadPoolExecutor

    objs = [str(LIB / (Path(src).stem + ".o")) for src in HIP_SOURCES]
    jobs = int(os.environ.get("MAX_JOBS", "4"))
    with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(HIP_SOURCES)))) as ex:
        list(ex.map(lambda so: _run([HIPCC, *HIP_FLAGS, *SOURCE_FLAGS.get(so[0], []), "-c", str(CSRC / so[0]),
                                     "-o", so[1]]),
                    zip(HIP_SOURCES, objs)))
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
