"""Parity comparison of sampler outputs against the oracle -- TEST INFRASTRUCTURE ONLY.

Used by tests/, ``__graft_entry__.smoke()`` and bench.py to check kernel results. The
bar for the sampler, applied row by row:

* greedy rows: token bit-exact (lowest-index ties, first NaN);
* error statuses identical;
* top-k threshold (``x_kth``) identical: it is a count, no tolerance applies;
* kept set identical; a difference is tolerated only on rows where top_p lies within
  ``band`` (1e-6) of a cumulative boundary at the cutoff;
* token identical whenever the kept sets agree, unless the uniform lies within ``band``
  of a CDF boundary of the draw;
* probabilities within ``prob_tol`` (1e-5) absolute wherever the kept sets agree.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .oracle import ROW_OK, RowResult

BAND = 1e-6
PROB_TOL = 1e-5


@dataclass
class Report:
    rows: int = 0
    checked_tokens: int = 0
    exempt_tokens: int = 0
    checked_kept: int = 0
    exempt_kept: int = 0
    max_prob_err: float = 0.0
    failures: list[str] = field(default_factory=list)

    def ok(self) -> bool:
        return not self.failures

    def summary(self) -> str:
        s = (f"rows={self.rows} tokens checked={self.checked_tokens} exempt={self.exempt_tokens} "
             f"kept checked={self.checked_kept} exempt={self.exempt_kept} max|dp|={self.max_prob_err:.2e}")
        if self.failures:
            s += f" FAILURES={len(self.failures)}: " + "; ".join(self.failures[:8])
        return s


def compare_rows(tokens, status, refs: list[RowResult], greedy_mask, probs=None, kept=None, info=None,
                 band: float = BAND, prob_tol: float = PROB_TOL, report: Report | None = None) -> Report:
    """Compare one call's outputs row by row. ``probs``/``kept`` are host numpy [rows, vocab]."""
    rep = report or Report()
    for b, ref in enumerate(refs):
        rep.rows += 1
        tok, st = int(tokens[b]), int(status[b])
        if st != ref.status:
            rep.failures.append(f"row {b}: status {st} != oracle {ref.status}")
            continue
        if st != ROW_OK:
            continue
        if greedy_mask[b]:
            rep.checked_tokens += 1
            if tok != ref.token:
                rep.failures.append(f"row {b}: greedy token {tok} != oracle {ref.token}")
            continue
        if info is not None:
            kx = float(info["x_kth"][b])
            if not (kx == np.float32(ref.x_kth) or (np.isneginf(kx) and np.isneginf(ref.x_kth))):
                rep.failures.append(f"row {b}: x_kth {kx} != oracle {ref.x_kth}")
        cut_close = ref.cut_margin < band
        # kept set: exact unless the cutoff sits within the band
        if kept is not None and ref.kept is not None:
            same = bool(np.array_equal(kept[b].astype(bool), ref.kept))
        elif info is not None:
            same = int(info["n_kept"][b]) == ref.n_kept
        else:
            same = not cut_close
        if same:
            rep.checked_kept += 1
        elif cut_close:
            rep.exempt_kept += 1
        else:
            what = "kept set" if kept is not None else "n_kept"
            rep.failures.append(f"row {b}: {what} differs from the oracle (cutoff margin {ref.cut_margin:.2e})")
        if same and probs is not None and ref.probs is not None:
            err = float(np.max(np.abs(probs[b].astype(np.float64) - ref.probs)))
            rep.max_prob_err = max(rep.max_prob_err, err)
            if err > prob_tol:
                rep.failures.append(f"row {b}: max |p - p_oracle| = {err:.3e} > {prob_tol}")
        # token: exact whenever the kept sets agree and u is clear of every CDF boundary
        if not same or ref.draw_margin < band:
            rep.exempt_tokens += 1
            continue
        rep.checked_tokens += 1
        if tok != ref.token:
            rep.failures.append(f"row {b}: token {tok} != oracle {ref.token} (u margin {ref.draw_margin:.2e})")
    return rep
