"""The CPU oracle against everything that pins it (CPU only, no GPU).

See tests/oracle_checks.py for what each check compares against; the chi-square tests here
pin the one thing no closed form does: that the oracle's inverse-CDF draw samples the same
distribution as the reference's ``torch.multinomial`` (pagedbatch/sampling.py:27).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from scipy import stats

import oracle_checks as oc
from oracle import oracle, reference_ops


@pytest.mark.parametrize("check", oc.ALL_CHECKS, ids=lambda c: c.__name__)
def test_oracle_check(check):
    failures = check(oracle)
    assert not failures, "\n".join(failures[:20])


def test_bf16_conversions_match_torch():
    g = torch.Generator().manual_seed(0)
    x = torch.cat([torch.randn(50000, generator=g) * 10, torch.tensor([0.0, -0.0, 1e-40, -1e-40, 3.4e38, -3.4e38,
                                                                       float("inf"), float("-inf")])])
    want = x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.f32_to_bf16_bits(x.numpy()), want)
    back = x.to(torch.bfloat16).float().numpy()
    assert np.array_equal(oracle.bf16_bits_to_f32(want).view(np.uint32), back.view(np.uint32))
    h = x.to(torch.float16)
    assert np.array_equal(oracle.logits_to_f32(h.numpy(), "float16").view(np.uint32), h.float().numpy().view(np.uint32))


def test_error_statuses():
    row = np.array([1.0, np.nan, 2.0], dtype=np.float32)
    assert oracle.sample_row(row, "float32", 1.0, 0, 1.0, 0.5).status == oracle.ROW_NAN
    assert oracle.sample_row(row, "float32", 0.0, 0, 1.0, 0.5).token == 1  # greedy returns the NaN index
    inf = np.array([1.0, np.inf], dtype=np.float32)
    assert oracle.sample_row(inf, "float32", 1.0, 0, 1.0, 0.5).status == oracle.ROW_NONFINITE
    ninf = np.full(3, -np.inf, dtype=np.float32)
    assert oracle.sample_row(ninf, "float32", 1.0, 0, 1.0, 0.5).status == oracle.ROW_NONFINITE
    for t, k, p, u in ((-1.0, 0, 1.0, 0.5), (1.0, -1, 1.0, 0.5), (1.0, 0, 0.0, 0.5), (1.0, 0, 1.5, 0.5),
                       (1.0, 0, 1.0, 1.0), (float("nan"), 0, 1.0, 0.5)):
        assert oracle.sample_row(np.zeros(3, np.float32), "float32", t, k, p, u).status == oracle.ROW_BAD_PARAM
    # the reference raises on exactly these distributions (torch.multinomial, sampling.py:27)
    for bad in (row, inf, ninf):
        with pytest.raises(RuntimeError):
            reference_ops.sample_token_ops(torch.from_numpy(bad), 1.0, 0, 1.0, torch.Generator().manual_seed(0))


def _chi2_case(V, T, k, p, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(V, generator=g) * 1.5
    probs = reference_ops.probs_ops(x, T, k, p).numpy().astype(np.float64)
    return x, probs


@pytest.mark.parametrize("V,T,k,p", [(16, 1.0, 0, 1.0), (24, 0.8, 10, 1.0), (24, 1.2, 0, 0.8), (32, 1.0, 20, 0.9)])
def test_chi_square_oracle_vs_multinomial(V, T, k, p):
    """Oracle draws (one torch.rand uniform each) and torch.multinomial draws against the
    reference ops' distribution, and against each other."""
    n = 20000
    x, probs = _chi2_case(V, T, k, p, seed=V + k)
    g = torch.Generator().manual_seed(123)
    us = torch.rand(n, generator=g).numpy()
    toks = np.array([oracle.sample_row(x.numpy(), "float32", T, k, p, float(u)).token for u in us])
    obs = np.bincount(toks, minlength=V)
    gm = torch.Generator().manual_seed(456)
    mt = torch.multinomial(torch.from_numpy(probs).float(), n, replacement=True, generator=gm).numpy()
    obs_m = np.bincount(mt, minlength=V)
    support = probs > 0
    assert obs[~support].sum() == 0 and obs_m[~support].sum() == 0
    exp = probs[support] * n
    # pool bins with expected count below 5
    small = exp < 5
    o1 = np.append(obs[support][~small], obs[support][small].sum())
    o2 = np.append(obs_m[support][~small], obs_m[support][small].sum())
    e = np.append(exp[~small], exp[small].sum())
    keep = e > 0
    p_oracle = stats.chisquare(o1[keep], e[keep] * o1[keep].sum() / e[keep].sum()).pvalue
    p_multi = stats.chisquare(o2[keep], e[keep] * o2[keep].sum() / e[keep].sum()).pvalue
    p_two = stats.chi2_contingency(np.stack([o1[keep], o2[keep]]))[1]
    assert p_oracle > 1e-3, p_oracle
    assert p_multi > 1e-3, p_multi
    assert p_two > 1e-3, p_two
