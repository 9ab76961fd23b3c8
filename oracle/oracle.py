"""CPU oracle for the token sampler -- TEST INFRASTRUCTURE ONLY.

Nothing in the product imports this module: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg use it, and
only for expected results and the CPU timing. The product path (``pagedbatch_amd``) runs the HIP
kernels and fails loudly when they are missing.

It restates ``pagedbatch/sampling.py:10-27`` row by row in numpy, in float64
wherever the reference accumulates, with two choices the reference leaves
open written down explicitly:

* **Tie order at the top-p cutoff.** The reference sorts with the unstable
  CPU ``torch.sort`` (sampling.py:19), so which members of a tie group at the
  cutoff survive is an accident of that sort. Here the order is fixed as
  value descending, index ascending (a stable sort).
* **Draw.** The reference draws with ``torch.multinomial`` (sampling.py:27),
  an exponential race that consumes ``vocab`` random numbers. Here one uniform
  ``u`` in [0, 1) is consumed and the token is the first kept element, in the
  same value-descending/index-ascending order, whose cumulative mass exceeds
  ``u * Z_P`` (inverse CDF). Both draw from the same categorical
  distribution, which the chi-square tests check against the reference ops.

Parity checks that pin this module (``tests/test_oracle.py``):
  * reference known answers, tests/test_engine.py:86-93;
  * greedy == ``torch.argmax`` (the reference's own op) incl. NaN, -0/+0, -inf;
  * top-k threshold == ``torch.topk(x, k).values[-1]`` (sampling.py:16);
  * kept set and probabilities == the op-for-op torch restatement
    (``oracle/reference_ops.py``) on rows without a tie at the cutoff;
  * exact rational brute force on tiny rows (``fractions.Fraction``);
  * chi-square of oracle draws against ``torch.multinomial`` draws.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

ROW_OK = 0
ROW_NAN = 1
ROW_NONFINITE = 2
ROW_BAD_PARAM = 3

DTYPES = ("float32", "float16", "bfloat16")

# sampling-order positions kept on each side of the cutoff in RowResult.cut_window
WINDOW = 256


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns (uint16) -> float32, exact."""
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits, round to nearest even (what ``Tensor.to(torch.bfloat16)`` does)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def logits_to_f32(raw: np.ndarray, dtype: str) -> np.ndarray:
    """Row(s) stored in ``dtype`` -> float32 values (``Tensor.float()`` at sampling.py:14)."""
    if dtype == "float32":
        return np.asarray(raw, dtype=np.float32)
    if dtype == "float16":
        return np.asarray(raw, dtype=np.float16).astype(np.float32)
    if dtype == "bfloat16":
        return bf16_bits_to_f32(np.asarray(raw, dtype=np.uint16))
    raise ValueError(dtype)


@dataclass
class RowResult:
    token: int
    status: int = ROW_OK
    x_max: float = float("nan")
    x_kth: float = float("-inf")
    x_cut: float = float("nan")
    n_cut_tie: int = 0
    n_cut_keep: int = 0
    n_kept: int = 0
    z_k: float = float("nan")
    z_p: float = float("nan")
    target: float = float("nan")
    # distance (in units of the normalised CDF) from u to the nearest CDF
    # boundary of the draw, and from top_p to the nearest cumulative boundary
    # at the cutoff: rows closer than 1e-6 are exempt from token / kept-set parity
    draw_margin: float = float("inf")
    cut_margin: float = float("inf")
    kept: np.ndarray | None = field(default=None, repr=False)
    probs: np.ndarray | None = field(default=None, repr=False)
    # the sampling order (value descending, index ascending over the top-k set) near the
    # cutoff and near the draw, for checking rows inside the 1e-6 bands:
    #   cut_window  (first position, indices, exclusive mass / Z_K) around the kept count
    #   draw_window (first position, indices, exclusive and inclusive mass / Z_P) around
    #               the drawn position
    cut_window: tuple | None = field(default=None, repr=False)
    draw_window: tuple | None = field(default=None, repr=False)


def greedy_token(x: np.ndarray) -> int:
    """``int(torch.argmax(row))`` (sampling.py:13): first NaN if any, else first maximum."""
    nan = np.isnan(x)
    if nan.any():
        return int(np.argmax(nan))
    return int(np.argmax(x))  # numpy returns the first maximum; -0.0 == +0.0


def scale(row32: np.ndarray, temperature: float) -> np.ndarray:
    """``logits.float() / temperature`` (sampling.py:14): IEEE float32 division."""
    return (row32 / np.float32(temperature)).astype(np.float32)


def kth_largest(x: np.ndarray, k: int) -> np.float32:
    """k-th largest value counting multiplicity (``torch.topk(x, k).values[-1]``, sampling.py:16)."""
    return np.partition(x, x.size - k)[x.size - k]


def sample_row(row, dtype: str, temperature: float, top_k: int, top_p: float, u: float,
               want_probs: bool = False) -> RowResult:
    """One row of pagedbatch/sampling.py:10-27 in inverse-CDF form (see module docstring)."""
    x32 = logits_to_f32(row, dtype)
    V = x32.size
    temperature = float(np.float32(temperature))
    top_p = float(np.float32(top_p))
    u = float(np.float32(u))
    # the C ABI's parameter contract (include/pbsample.h): a finite temperature >= 0,
    # top_p in (0, 1], top_k >= 0 (an infinite temperature, which SamplingParams lets
    # through, is rejected there too)
    if (not temperature >= 0.0) or not np.isfinite(temperature) or not (0.0 < top_p <= 1.0) or top_k < 0:
        return RowResult(token=0, status=ROW_BAD_PARAM)
    if temperature == 0.0:  # SamplingParams.greedy, config.py:156-158
        return RowResult(token=greedy_token(x32))
    if not (0.0 <= u < 1.0):
        return RowResult(token=0, status=ROW_BAD_PARAM)
    x = scale(x32, temperature)
    if np.isnan(x).any():
        return RowResult(token=0, status=ROW_NAN)
    m = x.max()
    if not np.isfinite(m):
        return RowResult(token=0, status=ROW_NONFINITE, x_max=float(m))
    res = RowResult(token=-1, x_max=float(m))

    # top-k (sampling.py:15-17): keep x >= k-th largest; ties at kth all kept
    if 0 < top_k < V:
        kth = kth_largest(x, top_k)
        in_k = x >= kth
        res.x_kth = float(kth)
    else:
        in_k = np.ones(V, dtype=bool)

    w = np.zeros(V, dtype=np.float64)
    w[in_k] = np.exp(x[in_k].astype(np.float64) - np.float64(m))
    idx_k = np.flatnonzero(in_k)
    # value descending, index ascending (a stable sort of -x keeps index order inside ties)
    order = idx_k[np.argsort(-x[idx_k], kind="stable")]
    ws = w[order]
    csum = np.cumsum(ws)
    z_k = float(csum[-1])
    res.z_k = z_k
    excl = np.concatenate(([0.0], csum[:-1]))

    # top-p (sampling.py:18-25): keep j iff exclusive mass <= top_p * Z
    if top_p < 1.0:
        thr = top_p * z_k
        n_keep_sorted = int(np.searchsorted(excl, thr, side="right"))  # excl is non-decreasing
        n_keep_sorted = max(n_keep_sorted, 1)
        # boundary margins around the cutoff, normalised by Z
        cands = []
        if n_keep_sorted - 1 < excl.size:
            cands.append(abs(excl[n_keep_sorted - 1] - thr))
        if n_keep_sorted < excl.size:
            cands.append(abs(excl[n_keep_sorted] - thr))
        res.cut_margin = float(min(cands) / z_k) if cands else float("inf")
    else:
        n_keep_sorted = order.size
    kept_sorted = order[:n_keep_sorted]
    x_cut = x[kept_sorted[-1]]
    res.x_cut = float(x_cut)
    tie = x[idx_k] == x_cut
    res.n_cut_tie = int(tie.sum())
    res.n_cut_keep = int((x[kept_sorted] == x_cut).sum())
    res.n_kept = int(n_keep_sorted)

    ck = csum[:n_keep_sorted]
    z_p = float(ck[-1])
    res.z_p = z_p
    t = u * z_p
    res.target = t
    j = int(np.searchsorted(ck, t, side="right"))  # first j with C_j > t
    if j >= n_keep_sorted:
        pos = np.flatnonzero(ws[:n_keep_sorted] > 0)
        j = int(pos[-1])
    res.token = int(kept_sorted[j])
    # distance of u from the nearest CDF boundary (normalised)
    lo = ck[j - 1] if j > 0 else 0.0
    hi = ck[j]
    res.draw_margin = float(min(abs(t - lo), abs(hi - t)) / z_p)
    if top_p < 1.0:
        a, b = max(0, n_keep_sorted - WINDOW), min(order.size, n_keep_sorted + WINDOW)
        res.cut_window = (a, order[a:b].copy(), excl[a:b] / z_k)
    a, b = max(0, j - 4), min(order.size, j + 5)
    res.draw_window = (a, order[a:b].copy(), excl[a:b] / z_p, csum[a:b] / z_p)

    if want_probs:
        kept = np.zeros(V, dtype=bool)
        kept[kept_sorted] = True
        probs = np.zeros(V, dtype=np.float64)
        probs[kept_sorted] = w[kept_sorted] / z_p
        res.kept = kept
        res.probs = probs
    return res


def sample_batch(logits, dtype: str, temperature, top_k, top_p, uniform, row_map=None,
                 want_probs: bool = False) -> list[RowResult]:
    """All output rows of one call; ``logits`` is [n_rows, vocab] in ``dtype`` (bf16 as uint16 bits)."""
    n_out = len(temperature)
    out = []
    for b in range(n_out):
        r = int(row_map[b]) if row_map is not None else b
        if not (0 <= r < logits.shape[0]):
            out.append(RowResult(token=0, status=ROW_BAD_PARAM))
            continue
        out.append(sample_row(logits[r], dtype, float(temperature[b]), int(top_k[b]), float(top_p[b]),
                              float(uniform[b]), want_probs=want_probs))
    return out
