"""Seeded synthetic sampler workloads (CPU tensors), shared by tests, smoke and bench.

Each is one engine step's worth of logits plus per-row parameters and uniforms:

* ``steps8_smollm_mixed``   fp32 [8, 49152]: N(0, 2^2) from seed 0; rows 0-1 greedy,
  2-3 temperature 0.8, 4-5 top-k 50, 6-7 top-p 0.9 (SmolLM2-135M vocabulary).
* ``greedy512_quantized``   fp32 [512, 49152]: N(0, 1) rounded to multiples of 1/4, so
  every row has ties at its maximum; all greedy.
* ``mixed256_llama3_bf16``  bf16 [256, 128256]: N(0, 1) plus a Zipf boost 8*rank^-1.1 on
  64 random token ids per row; temperature U[0.5, 1.5], top-k cycled over
  {1, 20, 50, 1000, off}, top-p cycled over {0.8, 0.95, 1.0} (Llama-3 vocabulary).
* ``nucleus1024_qwen_fp32`` fp32 [1024, 151936]: flat N(0, 0.5^2), temperature 1,
  top-p 0.95, no top-k.

The engine generator choice (pagedbatch/engine.py:58, 84) is mirrored by giving each row
its own seeded generator for its uniform.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class Workload:
    name: str
    logits: torch.Tensor  # CPU, [rows, vocab]
    temperature: list[float]
    top_k: list[int]
    top_p: list[float]
    uniform: list[float]

    @property
    def rows(self) -> int:
        return self.logits.shape[0]

    @property
    def vocab(self) -> int:
        return self.logits.shape[1]


def _uniforms(n: int, seed: int) -> list[float]:
    g = torch.Generator().manual_seed(seed)
    return [float(x) for x in torch.rand(n, generator=g)]


def steps8_smollm_mixed() -> Workload:
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(8, 49152, generator=g) * 2.0
    temperature = [0.0, 0.0, 0.8, 0.8, 1.0, 1.0, 1.0, 1.0]
    top_k = [0, 0, 0, 0, 50, 50, 0, 0]
    top_p = [1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 0.9, 0.9]
    # one seeded generator per row, one draw each (greedy rows draw nothing)
    uniform = [0.0 if temperature[r] == 0 else float(torch.rand((), generator=torch.Generator().manual_seed(1000 + r)))
               for r in range(8)]
    return Workload("steps8_smollm_mixed", logits, temperature, top_k, top_p, uniform)


def greedy512_quantized(rows: int = 512, vocab: int = 49152) -> Workload:
    g = torch.Generator().manual_seed(0)
    logits = torch.round(torch.randn(rows, vocab, generator=g) * 4.0) / 4.0
    return Workload("greedy512_quantized", logits, [0.0] * rows, [0] * rows, [1.0] * rows, [0.0] * rows)


def mixed256_llama3_bf16(rows: int = 256, vocab: int = 128256) -> Workload:
    g = torch.Generator().manual_seed(0)
    x = torch.randn(rows, vocab, generator=g)
    gi = torch.Generator().manual_seed(1)
    boost = 8.0 * torch.arange(1, 65, dtype=torch.float32).pow(-1.1)
    for r in range(rows):
        ids = torch.randperm(vocab, generator=gi)[:64]
        x[r, ids] += boost
    logits = x.to(torch.bfloat16)
    gp = torch.Generator().manual_seed(2)
    temperature = [float(t) for t in (0.5 + torch.rand(rows, generator=gp))]
    top_k = [[1, 20, 50, 1000, 0][r % 5] for r in range(rows)]
    top_p = [[0.8, 0.95, 1.0][r % 3] for r in range(rows)]
    return Workload("mixed256_llama3_bf16", logits, temperature, top_k, top_p, _uniforms(rows, 3))


def nucleus1024_qwen_fp32(rows: int = 1024, vocab: int = 151936) -> Workload:
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(rows, vocab, generator=g) * 0.5
    return Workload("nucleus1024_qwen_fp32", logits, [1.0] * rows, [0] * rows, [0.95] * rows, _uniforms(rows, 3))


WORKLOADS = {
    "steps8_smollm_mixed": steps8_smollm_mixed,
    "greedy512_quantized": greedy512_quantized,
    "mixed256_llama3_bf16": mixed256_llama3_bf16,
    "nucleus1024_qwen_fp32": nucleus1024_qwen_fp32,
}
