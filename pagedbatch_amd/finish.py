"""Finish reasons on the device: pagedbatch's per-token stop check for a whole step.

pagedbatch/engine.py:173-182 (``Engine._finish_reason``, called for every sampled row at
engine.py:149 once the token is appended) returns "stop" when the token is the model's
EOS id or one of the request's stop ids (unless ``ignore_eos``), else "length" when the
request has ``max_tokens`` outputs or the sequence holds ``max_model_len`` tokens, else
None. ``finish_codes`` evaluates that for every row of a step in one kernel, from the
sampler's device tokens, so the engine can read tokens and reasons back in one copy.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .sampling import SamplerError

# PBS_FINISH_* code -> the reference's reason string
REASONS = (None, "stop", "length")


@dataclass(frozen=True)
class FinishRule:
    """What the stop check needs of one sampled sequence (engine.py:173-182)."""

    ignore_eos: bool
    stop_token_ids: tuple[int, ...]
    num_output: int  # output tokens, the new one included (engine.py:140)
    max_tokens: int
    num_tokens: int  # prompt + output tokens, the new one included


def finish_codes(tokens: torch.Tensor, rules: Sequence[FinishRule], eos_token_id: int | None,
                 max_model_len: int) -> torch.Tensor:
    """PBS_FINISH_* codes, an int32 device tensor [rows], for the step's device tokens
    (int32 [rows], e.g. what the sampler wrote). Asynchronous on the current stream."""
    if tokens.dim() != 1 or tokens.dtype != torch.int32 or not tokens.is_cuda:
        raise ValueError("tokens must be a 1-D int32 device tensor")
    n = len(rules)
    if tokens.shape[0] != n:
        raise ValueError(f"{tokens.shape[0]} tokens for {n} rules")
    out = torch.empty(n, dtype=torch.int32, device=tokens.device)
    if n == 0:
        return out
    # one pinned host block, one copy: ignore_eos bytes (padded to 4), then int32
    # stop_offsets [n + 1] | num_output | max_tokens | num_tokens | stop_ids
    nstop = sum(len(r.stop_token_ids) for r in rules)
    pad = (n + 3) // 4 * 4
    ints = (n + 1) + 3 * n + nstop
    h = torch.empty(pad + 4 * ints, dtype=torch.uint8, pin_memory=True)
    hb = h.numpy()
    hb[:n] = np.fromiter((1 if r.ignore_eos else 0 for r in rules), np.uint8, n)
    hi = hb[pad:].view(np.int32)
    offs = np.zeros(n + 1, np.int64)
    offs[1:] = np.cumsum([len(r.stop_token_ids) for r in rules])
    hi[: n + 1] = offs
    hi[n + 1 : 2 * n + 1] = [r.num_output for r in rules]
    hi[2 * n + 1 : 3 * n + 1] = [r.max_tokens for r in rules]
    hi[3 * n + 1 : 4 * n + 1] = [r.num_tokens for r in rules]
    if nstop:
        hi[4 * n + 1 :] = [t for r in rules for t in r.stop_token_ids]
    d = h.to(tokens.device, non_blocking=True)
    base = d.data_ptr()
    i32 = base + pad
    lib = _lib.load()
    stream = torch.cuda.current_stream(tokens.device).cuda_stream
    rc = lib.pbs_finish_reasons(
        tokens.data_ptr(), n, -1 if eos_token_id is None else int(eos_token_id), base,
        i32, i32 + 4 * (4 * n + 1) if nstop else None, i32 + 4 * (n + 1), i32 + 4 * (2 * n + 1),
        i32 + 4 * (3 * n + 1), int(max_model_len), out.data_ptr(), stream)
    if rc != _lib.OK:
        raise SamplerError(f"pbs_finish_reasons failed ({rc}): {_lib.last_error(lib)}")
    # h and d may go now: torch's host allocator holds pinned blocks until their copies
    # complete, and its device allocator reuses d only for later work on this stream
    return out


def finish_reasons(tokens: torch.Tensor, rules: Sequence[FinishRule], eos_token_id: int | None,
                   max_model_len: int) -> list[str | None]:
    """The reference's reason strings ("stop", "length" or None) per row."""
    return [REASONS[c] for c in finish_codes(tokens, rules, eos_token_id, max_model_len).cpu().tolist()]
