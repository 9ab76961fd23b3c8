"""Per-request sampling parameters.

Same fields, defaults and validation as ``SamplingParams`` in pagedbatch/config.py:134-158,
so requests built for the reference engine can be passed straight through. ``sample`` also
accepts the reference's own ``SamplingParams`` objects (it reads ``temperature``,
``top_k`` and ``top_p`` only).
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass
class SamplingParams:
    """Per-request decoding parameters (pagedbatch/config.py:134-158)."""

    max_tokens: int = 64
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = 0
    ignore_eos: bool = False
    seed: int | None = None
    stop_token_ids: tuple[int, ...] = ()

    def __post_init__(self) -> None:
        if self.max_tokens < 1:
            raise ValueError("max_tokens must be >= 1")
        if self.temperature < 0:
            raise ValueError("temperature must be >= 0")
        if not 0 < self.top_p <= 1:
            raise ValueError("top_p must be in (0, 1]")
        if self.top_k < 0:
            raise ValueError("top_k must be >= 0")

    @property
    def greedy(self) -> bool:
        return self.temperature == 0
