"""Write tests/golden/torch_ops_vectors.npz: small sampler cases with the outputs of the
torch ops pagedbatch/sampling.py:10-27 calls.

For every case the file holds the raw logits row (bf16 as uint16 bits), the parameters and
what the reference's own ops produce for it on this torch build:

* ``argmax``  int(torch.argmax(row))                     sampling.py:13 (greedy rows)
* ``kth``     torch.topk(row.float() / T, k).values[-1]  sampling.py:16 (top-k rows)
* ``probs``   the fp32 distribution softmax hands to multinomial, sampling.py:14-26

The last one is produced by ``oracle.reference_ops.probs_ops``, which issues the same torch
calls in the same order as sampling.py:14-26. Rows cover fp32/fp16/bf16, odd vocab sizes,
ties at the maximum, at the k-th value and at the top-p cutoff, and NaN/inf/-0 values.

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle.reference_ops import probs_ops  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "torch_ops_vectors.npz")
DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}


def raw_of(x: torch.Tensor) -> np.ndarray:
    if x.dtype == torch.bfloat16:
        return x.view(torch.int16).numpy().view(np.uint16).copy()
    if x.dtype == torch.float16:
        return x.view(torch.int16).numpy().view(np.uint16).copy()
    return x.numpy().copy()


def rows():
    """(name, logits row tensor, temperature, top_k, top_p) cases."""
    g = torch.Generator().manual_seed(20240611)
    # the reference's own known-answer row (tests/test_engine.py:88)
    kat = torch.tensor([0.1, 3.0, 0.2, 2.9])
    yield "kat_greedy", kat, 0.0, 0, 1.0
    yield "kat_top_k1", kat, 1.0, 1, 1.0
    yield "kat_top_p1e-6", kat, 1.0, 0, 1e-6
    yield "kat_top_k2", kat, 1.0, 2, 1.0
    # the top-k tie example: k=2 on [3, 1, 3, 2, 3, .5] keeps three tokens
    yield "topk_tie_multiplicity", torch.tensor([3.0, 1.0, 3.0, 2.0, 3.0, 0.5]), 1.0, 2, 1.0
    for dt in ("float32", "float16", "bfloat16"):
        for V in (7, 257, 1000):
            base = torch.randn(V, generator=g) * 2.0
            x = base.to(DTYPES[dt])
            yield f"{dt}_V{V}_greedy", x, 0.0, 0, 1.0
            yield f"{dt}_V{V}_temp", x, 0.7, 0, 1.0
            yield f"{dt}_V{V}_topk", x, 1.3, max(1, V // 5), 1.0
            yield f"{dt}_V{V}_topp", x, 1.0, 0, 0.9
            yield f"{dt}_V{V}_topk_topp", x, 0.8, max(2, V // 3), 0.6
            # quantized values: ties everywhere, incl. at the max, the k-th and the cutoff
            q = (torch.round(torch.randn(V, generator=g) * 2.0) / 2.0).to(DTYPES[dt])
            yield f"{dt}_V{V}_ties_greedy", q, 0.0, 0, 1.0
            yield f"{dt}_V{V}_ties_topk", q, 1.0, max(1, V // 4), 1.0
            yield f"{dt}_V{V}_ties_topp", q, 1.0, 0, 0.5
    # special values
    s = torch.tensor([1.0, float("nan"), 3.0, float("nan"), 3.0])
    yield "nan_greedy", s, 0.0, 0, 1.0
    z = torch.tensor([-0.0, 0.0, -1.0, -0.0])
    yield "signed_zero_greedy", z, 0.0, 0, 1.0
    z16 = torch.tensor([-0.0, -2.0, 0.0, -0.0]).to(torch.bfloat16)
    yield "signed_zero_greedy_bf16", z16, 0.0, 0, 1.0
    yield "signed_zero_topk_bf16", z16, 1.0, 1, 1.0
    ninf = torch.tensor([float("-inf")] * 5)
    yield "all_neg_inf_greedy", ninf, 0.0, 0, 1.0
    mix = torch.tensor([float("-inf"), 2.0, float("-inf"), 1.0, 2.0, -5.0])
    yield "neg_inf_mixed_temp", mix, 1.0, 0, 1.0
    yield "neg_inf_mixed_topk", mix, 0.5, 3, 1.0
    yield "neg_inf_mixed_topp", mix, 2.0, 0, 0.7
    big = torch.tensor([60000.0, 59000.0, -60000.0, 0.0]).to(torch.float16)
    yield "f16_wide_temp", big, 100.0, 0, 1.0


def main():
    arrays = {}
    names, dtypes, T, K, P = [], [], [], [], []
    for i, (name, x, t, k, p) in enumerate(rows()):
        dt = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}[x.dtype]
        names.append(name)
        dtypes.append(dt)
        T.append(t)
        K.append(k)
        P.append(p)
        arrays[f"raw_{i}"] = raw_of(x)
        arrays[f"argmax_{i}"] = np.int64(int(torch.argmax(x)))
        V = x.shape[0]
        if t > 0:
            xs = x.float() / t
            arrays[f"kth_{i}"] = np.float32(torch.topk(xs, k).values[-1].item() if 0 < k < V else float("-inf"))
            arrays[f"probs_{i}"] = probs_ops(x, t, k, p).numpy().astype(np.float32)
    arrays["names"] = np.array(names)
    arrays["dtypes"] = np.array(dtypes)
    arrays["temperature"] = np.array(T, dtype=np.float32)
    arrays["top_k"] = np.array(K, dtype=np.int32)
    arrays["top_p"] = np.array(P, dtype=np.float32)
    arrays["torch_version"] = np.array(torch.__version__)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {len(names)} cases to {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
