"""The op-for-op CPU restatement (oracle/reference_ops.py) against pagedbatch's own tokens.

tests/golden/reference_tokens.npz holds tokens that pagedbatch.sampling.sample_token
(pagedbatch/sampling.py:10-27) returned for seeded rows, parameters and generators
(written by tests/golden/make_reference_tokens.py). The restatement must return the same
token on every call: that makes it a faithful stand-in for the reference wherever the tests
need the reference's exact distribution (chi-square) or its exact kept sets.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import reference_ops

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_tokens.npz")


def _row(raw: np.ndarray, dtype: str) -> torch.Tensor:
    if dtype == "bfloat16":
        return torch.from_numpy(raw.view(np.int16).copy()).view(torch.bfloat16)
    return torch.from_numpy(raw.view(np.float32).copy())


def test_reference_ops_reproduce_reference_tokens():
    z = np.load(GOLDEN, allow_pickle=False)
    n = z["token"].size
    assert n >= 64
    if str(z["torch_version"]) != torch.__version__:
        pytest.skip(f"fixture written with torch {z['torch_version']}, running {torch.__version__}")
    mismatches = []
    for i in range(n):
        row = _row(z[f"raw_{i}"], str(z["dtypes"][i]))
        gen = torch.Generator().manual_seed(int(z["seed"][i]))
        tok = reference_ops.sample_token_ops(row, float(z["temperature"][i]), int(z["top_k"][i]),
                                             float(z["top_p"][i]), gen)
        if tok != int(z["token"][i]):
            mismatches.append((i, tok, int(z["token"][i])))
    assert not mismatches, mismatches[:10]


def test_engine_step_ops_row_loop():
    """engine_step_ops is one sample_token_ops call per row, each on its own generator."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(6, 300, generator=g)
    params = [(0.0, 0, 1.0), (1.0, 0, 1.0), (0.8, 20, 1.0), (1.0, 0, 0.9), (1.2, 5, 0.5), (0.0, 3, 0.2)]
    a = reference_ops.engine_step_ops(x, params, [torch.Generator().manual_seed(s) for s in range(6)])
    b = [reference_ops.sample_token_ops(x[i], *params[i], torch.Generator().manual_seed(i)) for i in range(6)]
    assert a == b
    assert a[0] == int(torch.argmax(x[0])) and a[5] == int(torch.argmax(x[5]))
