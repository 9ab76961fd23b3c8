"""Write tests/golden/reference_tokens.npz: tokens drawn by pagedbatch's own sample_token.

The exact token ``torch.multinomial`` returns (pagedbatch/sampling.py:27) and the members
of a tie group that survive the unstable sort at the top-p cutoff (sampling.py:19) are
torch library behaviour that no closed form pins. This script imports the reference's
``pagedbatch.sampling`` in the build container (from /root/reference, which the GPU test
machines do not have) and records, for seeded rows, parameters and generators, the token
each call returns. ``tests/test_reference_ops.py`` then checks that the op-for-op
restatement ``oracle/reference_ops.py`` returns the identical token for every call, which
makes it a faithful stand-in for the reference in the chi-square tests.

Run from the repository root:  python tests/golden/make_reference_tokens.py
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

REF = "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_tokens.npz")


def cases():
    """(logits row, temperature, top_k, top_p) with one seeded generator per call."""
    g = torch.Generator().manual_seed(7)
    for V in (4, 50, 1000):
        for dt in (torch.float32, torch.bfloat16):
            x = (torch.randn(V, generator=g) * 1.5).to(dt)
            q = (torch.round(torch.randn(V, generator=g) * 2.0) / 2.0).to(dt)
            for row in (x, q):
                for t, k, p in ((0.0, 0, 1.0), (1.0, 0, 1.0), (0.7, 0, 1.0), (1.0, max(1, V // 4), 1.0),
                                (1.2, 0, 0.9), (1.0, 0, 0.5), (0.9, max(2, V // 2), 0.8), (1.0, 1, 1.0)):
                    yield row, t, k, p


def main():
    sys.path.insert(0, REF)
    from pagedbatch.config import SamplingParams  # the reference's own modules
    from pagedbatch.sampling import sample_token

    raws, dtypes, T, K, P, seeds, tokens = [], [], [], [], [], [], []
    for i, (row, t, k, p) in enumerate(cases()):
        seed = 1000 + i
        gen = torch.Generator().manual_seed(seed)
        tok = sample_token(row, SamplingParams(temperature=t, top_k=k, top_p=p), gen)
        raws.append(row.view(torch.int16).numpy().view(np.uint16).copy() if row.dtype == torch.bfloat16
                    else row.numpy().view(np.uint32).copy())
        dtypes.append("bfloat16" if row.dtype == torch.bfloat16 else "float32")
        T.append(t)
        K.append(k)
        P.append(p)
        seeds.append(seed)
        tokens.append(tok)
    arrays = {f"raw_{i}": r for i, r in enumerate(raws)}
    arrays.update(dtypes=np.array(dtypes), temperature=np.array(T, dtype=np.float32), top_k=np.array(K, np.int32),
                  top_p=np.array(P, dtype=np.float32), seed=np.array(seeds, np.int64), token=np.array(tokens, np.int64),
                  torch_version=np.array(torch.__version__))
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {len(tokens)} reference calls to {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
