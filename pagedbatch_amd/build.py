"""Build libpbsample.so in-tree with hipcc for gfx950.

``python -m pagedbatch_amd.build`` compiles ``csrc/pbsample.hip`` (the sampler) and
``csrc/pbattn.hip`` (the paged-attention decode kernel) into
``pagedbatch_amd/libpbsample.so`` (the file ``_lib.py`` loads). Packed-FP32 instruction
selection is disabled (``-packed-fp32-ops``); the kernels are written for wave64 gfx950
and nothing else.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "csrc", "pbsample.hip")
SRCS = [SRC, os.path.join(HERE, "csrc", "pbattn.hip")]
OUT = os.path.join(HERE, "libpbsample.so")
ARCH = os.environ.get("PBS_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def command(out: str = OUT) -> list[str]:
    return [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", os.path.join(ROOT, "include"),
        "-o", out,
        *SRCS,
    ]


def build(out: str = OUT, verbose: bool = True) -> str:
    tmp = out + ".tmp"
    cmd = command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    build(sys.argv[1] if len(sys.argv) > 1 else OUT)
