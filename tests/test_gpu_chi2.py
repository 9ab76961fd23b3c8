"""Distribution of the kernel's draws: chi-square over 10^6 draws against the reference.

One logits row is sampled 10^6 times in a single call (``row_map`` points every output row
at it), each draw with its own uniform from a seeded ``torch.rand``. The expected
distribution is the one pagedbatch's ``torch.multinomial`` samples from: the fp32 output of
the reference's ops (oracle/reference_ops.probs_ops, the op sequence of
pagedbatch/sampling.py:14-26). Bins with expected count below 5 are pooled; so are the
members of a tie group the top-p cutoff splits, because which of them the reference keeps
depends on its unstable sort.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from scipy import stats

from oracle import reference_ops
from pagedbatch_amd.sampling import sample_arrays

pytestmark = pytest.mark.gpu

N_DRAWS = 1_000_000


def _chi2(tokens: np.ndarray, probs: np.ndarray, x_scaled: np.ndarray):
    V = probs.size
    obs = np.bincount(tokens, minlength=V).astype(np.float64)
    # pool the tie group at the smallest kept value (where a top-p cutoff splits ties)
    kept = probs > 0
    cut = x_scaled[kept].min()
    tie = x_scaled == cut
    groups = [np.flatnonzero(kept & ~tie)[i:i + 1] for i in range(int((kept & ~tie).sum()))]
    groups.append(np.flatnonzero(tie))
    o = np.array([obs[g].sum() for g in groups])
    e = np.array([probs[g].sum() for g in groups]) * tokens.size
    outside = obs[~kept & ~tie].sum()
    small = e < 5
    o = np.append(o[~small], o[small].sum())
    e = np.append(e[~small], e[small].sum())
    keep = e > 0
    return stats.chisquare(o[keep], e[keep] * o[keep].sum() / e[keep].sum()).pvalue, outside


@pytest.mark.parametrize("name,dtype,V,T,k,p,quant", [
    ("bf16_topk_topp", torch.bfloat16, 4096, 0.9, 64, 0.9, False),
    ("fp32_nucleus", torch.float32, 1000, 1.0, 0, 0.95, False),
    ("fp32_ties_split_cutoff", torch.float32, 64, 1.0, 0, 0.6, True),
    ("fp16_temperature", torch.float16, 300, 1.3, 0, 1.0, False),
])
def test_chi_square_million_draws(dev, name, dtype, V, T, k, p, quant):
    print(f"[case] chi2 {name} V={V} draws={N_DRAWS}", flush=True)
    g = torch.Generator().manual_seed(V)
    x = torch.randn(V, generator=g) * 1.5
    if quant:
        x = torch.round(x * 2) / 2
    x = x.to(dtype)
    u = torch.rand(N_DRAWS, generator=torch.Generator().manual_seed(99)).numpy()
    out = sample_arrays(x.view(1, V).to(dev), np.full(N_DRAWS, T, np.float32), np.full(N_DRAWS, k, np.int32),
                        np.full(N_DRAWS, p, np.float32), u, row_map=np.zeros(N_DRAWS, np.int32))
    tokens, status = out
    assert (status == 0).all()
    probs = reference_ops.probs_ops(x, T, k, p).numpy().astype(np.float64)
    xs = (x.float() / T).numpy()
    pval, outside = _chi2(tokens, probs, xs)
    print(f"[case] chi2 {name}: p-value {pval:.4f}", flush=True)
    assert outside == 0, f"{outside} draws outside the reference's support"
    assert pval > 1e-4, pval
