"""Builds the C restatement (TEST INFRASTRUCTURE, the checker) into
oracle/liboracle.so.

The reference's own implementation of the path cannot be built here: it is
Crystal (no `crystal` toolchain in the image) on top of the unvendored µGPT
shard (shard.lock:15-17), and agpt_train.cu needs nvcc, cuBLAS and the absent
µGPT kernels.cu. So there is no oracle/_ref build.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent


def build() -> Path:
    out = HERE / "liboracle.so"
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-std=c99", "-shared", "-fPIC",
           "-Wall", str(HERE / "trie_attn_oracle.c"), str(HERE / "loss_oracle.c"),
           str(HERE / "block_oracle.c"), "-o", str(out), "-lm"]
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    return out


if __name__ == "__main__":
    build()
