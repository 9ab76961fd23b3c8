"""Op-for-op CPU restatement of pagedbatch's sampler -- TEST INFRASTRUCTURE ONLY.

Used by tests (as the distributional reference for chi-square checks and as the
source of the reference's exact kept sets / probabilities) and by
``bench.py``'s ``cpu_baseline`` leg (``kind: "port"``). Nothing in the product
imports it.

``sample_token_ops`` makes the same torch calls as
``pagedbatch/sampling.py:10-27``, in the same order and with the same
generator use, because the reference's tie order at the top-p cutoff (unstable
``torch.sort``) and its exact ``torch.multinomial`` token are torch library
behaviour: the only way to reproduce them without importing the reference is
to issue the identical op sequence on the same torch build. ``engine_step_ops``
loops over the rows the way ``pagedbatch/engine.py:133-139`` does.
"""

from __future__ import annotations

import torch

NEG_INF = float("-inf")


def filtered_logits_ops(row: torch.Tensor, temperature: float, top_k: int, top_p: float) -> torch.Tensor:
    """The masked, temperature-scaled row that sampling.py:14-25 hands to softmax."""
    x = row.float() / temperature                                        # sampling.py:14
    n = x.shape[-1]
    if 0 < top_k < n:                                                    # sampling.py:15
        kth = torch.topk(x, top_k).values[-1]                            # sampling.py:16
        x = x.masked_fill(x < kth, NEG_INF)                              # sampling.py:17
    if top_p < 1.0:                                                      # sampling.py:18
        desc, perm = torch.sort(x, descending=True)                      # sampling.py:19
        p_sorted = torch.softmax(desc, dim=-1)                           # sampling.py:20
        running = torch.cumsum(p_sorted, dim=-1)                         # sampling.py:21
        desc = desc.masked_fill(running - p_sorted > top_p, NEG_INF)     # sampling.py:23-24
        x = torch.full_like(x, NEG_INF).scatter(0, perm, desc)           # sampling.py:25
    return x


def probs_ops(row: torch.Tensor, temperature: float, top_k: int, top_p: float) -> torch.Tensor:
    """Final distribution of sampling.py:26 (fp32)."""
    return torch.softmax(filtered_logits_ops(row, temperature, top_k, top_p), dim=-1)


def sample_token_ops(row: torch.Tensor, temperature: float, top_k: int, top_p: float,
                     generator: torch.Generator) -> int:
    """One call of sampling.py:10-27 on a [vocab] CPU row."""
    if temperature == 0:                                                 # sampling.py:12, config.py:156-158
        return int(torch.argmax(row))                                    # sampling.py:13
    probs = probs_ops(row, temperature, top_k, top_p)                    # sampling.py:14-26
    return int(torch.multinomial(probs, 1, generator=generator))         # sampling.py:27


def engine_step_ops(logits: torch.Tensor, params: list[tuple[float, int, float]],
                    generators: list[torch.Generator]) -> list[int]:
    """All rows of one engine step, one sample_token call per row as in engine.py:133-139.

    ``params[i]`` is ``(temperature, top_k, top_p)`` for row ``i``.
    """
    return [sample_token_ops(logits[i], t, k, p, generators[i]) for i, (t, k, p) in enumerate(params)]
