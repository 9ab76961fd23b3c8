"""Checks that pin the CPU oracle (oracle/oracle.py) to pagedbatch's sampler.

Each ``check_*`` function takes an oracle module and returns a list of failure strings
(empty = pass), so the same checks run on the real oracle (tests/test_oracle.py) and on
copies of it with a planted mistake (tests/test_oracle_mutations.py), which they must
reject. What pins what:

* ``check_reference_kat``   the reference's known answers, tests/test_engine.py:86-93;
* ``check_greedy``          torch.argmax (sampling.py:13) incl. NaN, -0/+0, -inf, ties;
* ``check_scale``           torch's fp32 true division (sampling.py:14), bit for bit;
* ``check_kth``             torch.topk(x, k).values[-1] (sampling.py:16) on tie-heavy rows;
* ``check_golden``          tests/golden/torch_ops_vectors.npz: argmax, k-th value and the
                            final fp32 distribution produced by the reference's own torch ops;
* ``check_exact_boundaries`` rows whose weights are exact in binary (equal logits), where the
                            top-p rule of sampling.py:23 ("drop if cum - p > top_p") and the
                            inverse-CDF interval rule have one right answer each;
* ``check_brute_force``     a rational-arithmetic (fractions.Fraction) restatement with
                            explicit loops on tiny rows: order, ties, cutoff, draw.
"""

from __future__ import annotations

import math
import os
from fractions import Fraction

import numpy as np
import torch

from oracle import reference_ops

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "torch_ops_vectors.npz")
BAND = 1e-6
PROB_TOL = 1e-5
TORCH_DT = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}


def torch_row(raw: np.ndarray, dtype: str) -> torch.Tensor:
    if dtype == "bfloat16":
        return torch.from_numpy(raw.astype(np.uint16).view(np.int16).copy()).view(torch.bfloat16)
    if dtype == "float16":
        return torch.from_numpy(raw.astype(np.uint16).view(np.float16).copy())
    return torch.from_numpy(np.asarray(raw, dtype=np.float32).copy())


def oracle_raw(x: torch.Tensor) -> np.ndarray:
    """Row in the form the oracle takes (bf16 as uint16 bits, fp16 as float16)."""
    if x.dtype == torch.bfloat16:
        return x.view(torch.int16).numpy().view(np.uint16)
    return x.numpy()


def dtype_name(x: torch.Tensor) -> str:
    return {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}[x.dtype]


# ------------------------------------------------------------------------------------------
def check_reference_kat(orc) -> list[str]:
    """tests/test_engine.py:86-93 on the row [0.1, 3.0, 0.2, 2.9]."""
    f = []
    row = np.array([0.1, 3.0, 0.2, 2.9], dtype=np.float32)
    us = [i / 64 for i in range(64)]
    if orc.sample_row(row, "float32", 0.0, 0, 1.0, 0.0).token != 1:
        f.append("kat: greedy != 1")
    for u in us:
        if orc.sample_row(row, "float32", 1.0, 1, 1.0, u).token != 1:
            f.append(f"kat: top_k=1 u={u} != 1")
            break
    for u in us:
        if orc.sample_row(row, "float32", 1.0, 0, 1e-6, u).token != 1:
            f.append(f"kat: top_p=1e-6 u={u} != 1")
            break
    picks = {orc.sample_row(row, "float32", 1.0, 2, 1.0, u).token for u in us}
    if not picks <= {1, 3} or len(picks) != 2:
        f.append(f"kat: top_k=2 picks {sorted(picks)} (expected both of 1 and 3 and nothing else)")
    return f


def _special_rows():
    g = torch.Generator().manual_seed(11)
    yield torch.tensor([1.0, float("nan"), 3.0, float("nan")])
    yield torch.tensor([float("-inf")] * 6)
    yield torch.tensor([-0.0, 0.0, -0.0, -1.0])
    yield torch.tensor([0.0, -0.0, -3.0])
    yield torch.tensor([float("-inf"), -2.0, float("inf"), float("inf")])
    yield torch.tensor([float("-inf"), -2.0, float("-inf")])
    for _ in range(40):
        yield torch.round(torch.randn(int(torch.randint(1, 300, (1,), generator=g)), generator=g) * 2) / 2


def check_greedy(orc) -> list[str]:
    f = []
    for x in _special_rows():
        for dt in TORCH_DT.values():
            xd = x.to(dt)
            want = int(torch.argmax(xd))
            got = orc.sample_row(oracle_raw(xd), dtype_name(xd), 0.0, 0, 1.0, 0.0).token
            if got != want:
                f.append(f"greedy {dt} {x.tolist()[:6]}: {got} != torch.argmax {want}")
    return f


def check_scale(orc) -> list[str]:
    g = torch.Generator().manual_seed(5)
    x = torch.randn(20000, generator=g) * 7
    f = []
    for t in (0.1, 0.3, 0.7, 0.8, 1.3, 1.7, 3.0, 1e-3):
        want = (x.float() / t).numpy()
        got = orc.scale(x.numpy(), t)
        if not np.array_equal(want.view(np.uint32), np.asarray(got, dtype=np.float32).view(np.uint32)):
            f.append(f"scale T={t}: differs from torch's x / T")
    return f


def check_kth(orc) -> list[str]:
    g = torch.Generator().manual_seed(3)
    f = []
    for V in (1, 2, 7, 100, 1000):
        x = torch.round(torch.randn(V, generator=g) * 3) / 3  # many ties
        for k in sorted({1, 2, 3, V // 2, V - 1, V} - {0}):
            if not 0 < k <= V:
                continue
            want = float(torch.topk(x, k).values[-1])
            got = float(orc.kth_largest(x.numpy(), k))
            if got != want:
                f.append(f"kth V={V} k={k}: {got} != torch.topk {want}")
    return f


def _compare_distribution(res, probs_ref: np.ndarray, x_scaled: np.ndarray, name: str) -> list[str]:
    """Oracle RowResult (with probs) vs the reference ops' fp32 final distribution.

    The reference's unstable sort may keep other members of a tie group split by the
    top-p cutoff, so inside that group only the count of kept members and the multiset of
    their probabilities are compared; everything else is compared element by element.
    """
    f = []
    if res.cut_margin < BAND:
        return f
    p = res.probs
    tie = x_scaled == np.float32(res.x_cut)
    err = float(np.max(np.abs(p[~tie] - probs_ref[~tie].astype(np.float64)), initial=0.0))
    err_tie = float(np.max(np.abs(np.sort(p[tie]) - np.sort(probs_ref[tie].astype(np.float64))), initial=0.0))
    if max(err, err_tie) > PROB_TOL:
        f.append(f"{name}: max |p - p_ref| = {max(err, err_tie):.2e}")
    on_ref = probs_ref > 0
    on_orc = p > 1e-30  # fp32 softmax underflows to 0 below exp(-103); fp64 does not
    if not np.array_equal(on_ref[~tie], on_orc[~tie]):
        f.append(f"{name}: kept set outside the cutoff tie group differs")
    if int(on_ref[tie].sum()) != int(on_orc[tie].sum()):
        f.append(f"{name}: kept count in the cutoff tie group {int(on_orc[tie].sum())} != {int(on_ref[tie].sum())}")
    return f


def check_golden(orc, path: str = GOLDEN) -> list[str]:
    f = []
    z = np.load(path, allow_pickle=False)
    names = z["names"]
    for i, name in enumerate(names):
        dt = str(z["dtypes"][i])
        raw = z[f"raw_{i}"]
        if dt == "float16":
            raw = raw.view(np.float16)
        t, k, p = float(z["temperature"][i]), int(z["top_k"][i]), float(z["top_p"][i])
        if t == 0:
            tok = orc.sample_row(raw, dt, 0.0, k, p, 0.0).token
            if tok != int(z[f"argmax_{i}"]):
                f.append(f"golden {name}: greedy {tok} != {int(z[f'argmax_{i}'])}")
            continue
        res = orc.sample_row(raw, dt, t, k, p, 0.5, want_probs=True)
        if res.status != orc.ROW_OK:
            f.append(f"golden {name}: status {res.status}")
            continue
        kth = float(z[f"kth_{i}"])
        if not (res.x_kth == kth or (math.isinf(kth) and math.isinf(res.x_kth))):
            f.append(f"golden {name}: x_kth {res.x_kth} != torch.topk {kth}")
        xs = orc.scale(orc.logits_to_f32(raw, dt), t)
        f += _compare_distribution(res, z[f"probs_{i}"], xs, f"golden {name}")
    return f


def check_live_reference_ops(orc, seed: int = 0, n: int = 24) -> list[str]:
    """Random rows (fresh draws, not the fixture) against reference_ops.probs_ops."""
    g = torch.Generator().manual_seed(seed)
    f = []
    for i in range(n):
        V = int(torch.randint(2, 3000, (1,), generator=g))
        dt = list(TORCH_DT.values())[i % 3]
        x = (torch.randn(V, generator=g) * float(torch.rand((), generator=g) * 3 + 0.2)).to(dt)
        t = float(torch.rand((), generator=g)) * 1.5 + 0.25
        k = [0, 1, 5, V // 3, V - 1][i % 5]
        p = [1.0, 0.9, 0.5, 0.99, 0.3][(i // 5) % 5]
        res = orc.sample_row(oracle_raw(x), dtype_name(x), t, k, p, 0.5, want_probs=True)
        probs_ref = reference_ops.probs_ops(x, t, k, p).numpy()
        xs = orc.scale(x.float().numpy(), t)
        f += _compare_distribution(res, probs_ref, xs, f"live row {i} V={V} {dt} T={t:.3f} k={k} p={p}")
    return f


def check_exact_boundaries(orc) -> list[str]:
    """Equal logits: every weight is exactly 1, so masses are small integers."""
    f = []
    row = np.zeros(4, dtype=np.float32)
    # top-p 0.5 of mass 4: exclusive masses 0, 1, 2, 3; sampling.py:23 drops only 3 > 2
    r = orc.sample_row(row, "float32", 1.0, 0, 0.5, 0.0, want_probs=True)
    if r.n_kept != 3 or list(np.flatnonzero(r.kept)) != [0, 1, 2]:
        f.append(f"boundary: top_p=0.5 on 4 equal logits keeps {list(np.flatnonzero(r.kept))} (want [0, 1, 2])")
    # top-p 0.25: exclusive 0 and 1 <= 1 -> 2 kept
    r = orc.sample_row(row, "float32", 1.0, 0, 0.25, 0.0, want_probs=True)
    if r.n_kept != 2:
        f.append(f"boundary: top_p=0.25 keeps {r.n_kept} (want 2)")
    # the reference's own ops agree on the counts
    for p, want in ((0.5, 3), (0.25, 2)):
        got = int((reference_ops.probs_ops(torch.zeros(4), 1.0, 0, p) > 0).sum())
        if got != want:
            f.append(f"boundary: reference ops keep {got} at top_p={p}")
    # inverse CDF on masses 1,2,3,4: u*4 = 1.0 is the start of token 1's interval [1, 2)
    for u, want in ((0.0, 0), (0.25, 1), (0.5, 2), (0.75, 3), (0.2499999, 0), (0.9999999, 3)):
        tok = orc.sample_row(row, "float32", 1.0, 0, 1.0, u).token
        if tok != want:
            f.append(f"boundary: u={u} draws {tok} (want {want})")
    # a zero-weight tail is never drawn, even at u -> 1
    row2 = np.array([0.0, -1e4, 0.0], dtype=np.float32)
    tok = orc.sample_row(row2, "float32", 1.0, 0, 1.0, 0.9999999).token
    if tok != 2:
        f.append(f"boundary: u->1 with a zero-weight token draws {tok} (want 2)")
    return f


def brute_force_row(x32: np.ndarray, T: float, k: int, p: float, u: float):
    """Rational restatement of sampling.py:14-27 with explicit loops; returns (kept set, token)."""
    V = x32.size
    x = [float(v) for v in (x32 / np.float32(T)).astype(np.float32)]
    m = max(x)
    order = sorted(range(V), key=lambda i: (-x[i], i))  # value descending, index ascending
    cand = order
    if 0 < k < V:
        kth = order[k - 1]
        cand = [i for i in order if x[i] >= x[kth]]
    w = {i: Fraction(math.exp(x[i] - m)) for i in cand}
    Z = sum(w.values(), Fraction(0))
    kept = []
    run = Fraction(0)
    for j, i in enumerate(cand):
        # sampling.py:23: drop if (cumulative incl. self) - self > top_p  ->  exclusive > p
        if p < 1.0 and run > Fraction(float(np.float32(p))) * Z and j > 0:
            break
        kept.append(i)
        run += w[i]
    Zp = sum((w[i] for i in kept), Fraction(0))
    t = Fraction(float(np.float32(u))) * Zp
    acc = Fraction(0)
    tok = None
    for i in kept:
        lo = acc
        acc += w[i]
        if lo <= t < acc:
            tok = i
            break
    return set(kept), tok


def check_brute_force(orc, seed: int = 1, n: int = 300) -> list[str]:
    rng = np.random.default_rng(seed)
    f = []
    for c in range(n):
        V = int(rng.integers(1, 12))
        if c % 3 == 0:
            x = (rng.integers(-3, 4, V) * 0.5).astype(np.float32)  # ties
        else:
            x = rng.normal(0, 1.5, V).astype(np.float32)
        T = float(rng.choice([0.5, 1.0, 1.7]))
        k = int(rng.integers(0, V + 1))
        p = float(rng.choice([1.0, 0.9, 0.6, 0.3, 0.05]))
        u = float(np.float32(rng.random()))
        kept, tok = brute_force_row(x, T, k, p, u)
        r = orc.sample_row(x, "float32", T, k, p, u, want_probs=True)
        got_kept = set(np.flatnonzero(r.kept).tolist()) if r.kept is not None else set()
        exempt = r.cut_margin < BAND
        if got_kept != kept and not exempt:
            f.append(f"brute case {c}: kept {sorted(got_kept)} != {sorted(kept)} (x={x.tolist()} T={T} k={k} p={p})")
            continue
        if got_kept == kept and r.draw_margin >= BAND and r.token != tok:
            f.append(f"brute case {c}: token {r.token} != {tok} (x={x.tolist()} T={T} k={k} p={p} u={u})")
    return f


ALL_CHECKS = (check_reference_kat, check_greedy, check_scale, check_kth, check_golden, check_live_reference_ops,
              check_exact_boundaries, check_brute_force)
