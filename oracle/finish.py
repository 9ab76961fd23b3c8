"""CPU oracle for the finish-reason check -- TEST INFRASTRUCTURE ONLY.

Nothing in the product imports this module: only ``tests/`` use it, to hold the expected results of
``pbs_finish_reasons`` (``pagedbatch_amd/finish.py``), which runs on the GPU and fails
loudly when the library is missing.

It restates ``pagedbatch/engine.py:173-182`` (``Engine._finish_reason``) for one sampled
sequence, with the token already appended to its outputs (engine.py:140, 149):

* "stop" when ``ignore_eos`` is off and the token is the model's EOS id (if it has one)
  or one of the request's ``stop_token_ids`` (engine.py:176-177);
* otherwise "length" when the request has ``max_tokens`` outputs (engine.py:178-179) or
  the sequence holds ``max_model_len`` tokens (engine.py:180-181);
* otherwise None.

Pinned by ``tests/test_finish.py``: the reference's own engine tests
(tests/test_engine.py:46 "length" after max_tokens outputs, :54 "stop" on a stop id with
the stop token kept as the last output), the precedence of "stop" over "length", and
``ignore_eos`` suppressing both stop kinds (engine.py:176) but not the length limits.
"""

from __future__ import annotations

from collections.abc import Sequence


def finish_reason(token: int, eos_token_id: int | None, ignore_eos: bool, stop_token_ids: Sequence[int],
                  num_output: int, max_tokens: int, num_tokens: int, max_model_len: int) -> str | None:
    """engine.py:173-182 for one sequence; ``num_output`` and ``num_tokens`` count the new token."""
    if not ignore_eos and ((eos_token_id is not None and token == eos_token_id) or token in stop_token_ids):
        return "stop"
    if num_output >= max_tokens:
        return "length"
    if num_tokens >= max_model_len:
        return "length"
    return None
