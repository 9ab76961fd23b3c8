"""Build libpbsample.so in-tree with hipcc for gfx950.

``python -m pagedbatch_amd.build`` compiles ``csrc/pbsample.hip`` (the sampler),
``csrc/pbattn.hip`` (the paged-attention decode kernel) and ``csrc/pblmhead.hip`` (the
fused lm_head + greedy kernel) into ``pagedbatch_amd/libpbsample.so`` (the file
``_lib.py`` loads). The sampler is compiled
as several translation units in parallel (one per logits type, ``-DPBS_TU_DTYPE=n``, and
one for the C ABI, ``-DPBS_TU_ABI``), then everything is linked into one shared library.
Packed-FP32 instruction selection is disabled (``-packed-fp32-ops``); the kernels are
written for wave64 gfx950 and nothing else.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "csrc", "pbsample.hip")
ATTN = os.path.join(HERE, "csrc", "pbattn.hip")
LMHEAD = os.path.join(HERE, "csrc", "pblmhead.hip")
SRCS = [SRC, ATTN, LMHEAD]
OUT = os.path.join(HERE, "libpbsample.so")
ARCH = os.environ.get("PBS_OFFLOAD_ARCH", "gfx950")

# (source, extra defines, object name)
UNITS = [
    (SRC, ["-DPBS_TU_DTYPE=2"], "pbsample_bf16.o"),
    (SRC, ["-DPBS_TU_DTYPE=1"], "pbsample_f16.o"),
    (SRC, ["-DPBS_TU_DTYPE=0"], "pbsample_f32.o"),
    (SRC, ["-DPBS_TU_ABI"], "pbsample_abi.o"),
    (ATTN, [], "pbattn.o"),
    (LMHEAD, [], "pblmhead.o"),
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def _flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", os.path.join(ROOT, "include"),
    ]


def compile_command(src: str, defines: list[str], obj: str) -> list[str]:
    return [hipcc(), *_flags(), *defines, "-c", "-o", obj, src]


def link_command(objs: list[str], out: str) -> list[str]:
    return [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out, *objs]


def command(out: str = OUT) -> list[str]:
    """One hipcc line building the whole library from both sources (no unit split)."""
    return [hipcc(), *_flags(), "-shared", "-o", out, *SRCS]


def build(out: str = OUT, verbose: bool = True) -> str:
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    jobs = [(compile_command(s, d, os.path.join(objdir, o)), os.path.join(objdir, o)) for s, d, o in UNITS]

    def run(job):
        cmd, _ = job
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)

    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        list(ex.map(run, jobs))
    tmp = out + ".tmp"
    cmd = link_command([o for _, o in jobs], tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    build(sys.argv[1] if len(sys.argv) > 1 else OUT)
