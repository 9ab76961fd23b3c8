"""Parity comparison of sampler outputs against the oracle -- TEST INFRASTRUCTURE ONLY.

Used by tests/, ``__graft_entry__.smoke()`` and bench.py to check kernel results. The
bar for the sampler, applied row by row:

* greedy rows: token bit-exact (lowest-index ties, first NaN);
* error statuses identical;
* top-k threshold (``x_kth``) identical: it is a count, no tolerance applies;
* kept set identical. Only on rows where top_p lies within ``band`` (1e-6) of a
  cumulative boundary at the cutoff may it differ, and then only as the mathematics
  allows: the kernel's kept set must still be a prefix of the oracle's sampling order
  (value descending, index ascending), and every position between the two kept counts
  must have its exclusive mass within 2 * band of top_p;
* token identical whenever the kept sets agree and the uniform lies clear of every CDF
  boundary by ``band``. On the other rows the token must still be one whose CDF interval
  holds the draw point up to 2 * band (the token next to the boundary the draw sits on);
* probabilities within ``prob_tol`` (1e-5) absolute wherever the kept sets agree.

``Report.checked_*`` count rows held to the exact bar, ``Report.exempt_*`` rows held to
the band bar; tests assert a minimum of exactly checked rows per case.
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


def _kept_within_band(b: int, ref: RowResult, top_p: float, gpu_kept: np.ndarray | None, n_gpu: int,
                      band: float) -> str | None:
    """None if the kernel's kept set differs from the oracle's only at positions whose
    exclusive mass lies within 2 * band of top_p (and is a prefix of the oracle's order);
    otherwise what is wrong."""
    if ref.cut_window is None:
        return f"row {b}: kept set differs without a top-p cutoff"
    a, order, excl = ref.cut_window
    n_ref = ref.n_kept
    lo, hi = min(n_ref, n_gpu), max(n_ref, n_gpu)
    if lo < a or hi > a + order.size:
        return f"row {b}: kept count {n_gpu} vs oracle {n_ref}: outside the compared window"
    dev = np.abs(excl[lo - a:hi - a] - top_p)
    if dev.size and float(dev.max()) > 2 * band:
        return (f"row {b}: kept count {n_gpu} vs oracle {n_ref}, a position between them has exclusive mass "
                f"{float(dev.max()):.2e} from top_p")
    if gpu_kept is not None:
        # the kernel's set must be the first n_gpu of the oracle's order: the oracle's set
        # plus or minus exactly the positions between the two counts
        ref_kept = ref.kept.copy()
        between = order[lo - a:hi - a]
        ref_kept[between] = n_gpu > n_ref
        if not np.array_equal(ref_kept, gpu_kept):
            return f"row {b}: kept set is not a prefix of the oracle's sampling order"
    return None


def _token_within_band(b: int, ref: RowResult, tok: int, u: float, z_ratio: float, band: float) -> str | None:
    """None if the kernel's token is one whose CDF interval (oracle masses / Z_P) holds the
    draw point u * (kernel's Z_P / oracle's Z_P) up to 2 * band."""
    if ref.draw_window is None:
        return f"row {b}: no draw window"
    a, order, excl, incl = ref.draw_window
    pos = np.flatnonzero(order == tok)
    if pos.size == 0:
        return f"row {b}: token {tok} is not next to the oracle's draw position {ref.token}"
    i = int(pos[0])
    t = u * z_ratio
    if not (excl[i] - 2 * band <= t <= incl[i] + 2 * band):
        return (f"row {b}: token {tok}'s CDF interval [{excl[i]:.9f}, {incl[i]:.9f}] does not hold the draw "
                f"point {t:.9f}")
    return None


def compare_rows(tokens, status, refs: list[RowResult], greedy_mask, probs=None, kept=None, info=None,
                 band: float = BAND, prob_tol: float = PROB_TOL, report: Report | None = None,
                 top_p=None, uniform=None) -> Report:
    """Compare one call's outputs row by row. ``probs``/``kept`` are host numpy [rows, vocab];
    ``top_p`` and ``uniform`` (per row) let the rows inside the bands be checked against
    the oracle's order and masses instead of being skipped."""
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
        gpu_kept = kept[b].astype(bool) if kept is not None else None
        # kept set: exact unless the cutoff sits within the band
        if gpu_kept is not None and ref.kept is not None:
            same = bool(np.array_equal(gpu_kept, ref.kept))
            n_gpu = int(gpu_kept.sum())
        elif info is not None:
            n_gpu = int(info["n_kept"][b])
            same = n_gpu == ref.n_kept
            gpu_kept = None
        else:
            same = not cut_close
            n_gpu = ref.n_kept
        if same:
            rep.checked_kept += 1
        elif cut_close:
            rep.exempt_kept += 1
            if top_p is not None:
                why = _kept_within_band(b, ref, float(np.float32(top_p[b])), gpu_kept, n_gpu, band)
                if why:
                    rep.failures.append(why)
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
            if uniform is not None:
                z_ratio = 1.0
                if info is not None and ref.z_p > 0:
                    z_ratio = float(info["z_p"][b]) / ref.z_p
                why = _token_within_band(b, ref, tok, float(np.float32(uniform[b])), z_ratio, band)
                if why:
                    rep.failures.append(why)
            continue
        rep.checked_tokens += 1
        if tok != ref.token:
            rep.failures.append(f"row {b}: token {tok} != oracle {ref.token} (u margin {ref.draw_margin:.2e})")
    return rep
