"""The parity bar itself (oracle/compare.py), on the CPU: rows inside the 1e-6 bands are
still held to what the mathematics fixes, and planted mistakes just outside it fail.

Rows of equal logits make every weight 1, so the exclusive mass of sampling position q is
exactly q / Z: the cutoff and the CDF boundaries sit where the test puts them.
"""

from __future__ import annotations

import numpy as np

from oracle import oracle
from oracle.compare import compare_rows


def _flat_row(V=1000):
    return np.zeros(V, dtype=np.float32)


def _info(ref, n_kept=None, z_p=None):
    info = np.zeros(1, dtype=[("x_kth", "<f4"), ("n_kept", "<i4"), ("z_p", "<f8")])
    info["x_kth"][0] = ref.x_kth
    info["n_kept"][0] = ref.n_kept if n_kept is None else n_kept
    info["z_p"][0] = ref.z_p if z_p is None else z_p
    return info


def _kept_prefix(ref, n):
    """The first n positions of the oracle's sampling order, as a kept mask."""
    a, order, _ = ref.cut_window
    kept = ref.kept.copy()
    if n > ref.n_kept:
        kept[order[ref.n_kept - a:n - a]] = True
    else:
        kept[order[n - a:ref.n_kept - a]] = False
    return kept.astype(np.uint8)


def test_cutoff_on_a_boundary_allows_the_one_element_at_it():
    # V equal weights, top_p = 0.5: position 500 has exclusive mass exactly 0.5 * Z
    row = _flat_row()
    ref = oracle.sample_row(row, "float32", 1.0, 0, 0.5, 0.3, want_probs=True)
    assert ref.n_kept == 501 and ref.cut_margin == 0.0
    for n in (500, 501):  # either side of the boundary is within the band
        kept = _kept_prefix(ref, n)[None]
        rep = compare_rows([ref.token], [0], [ref], [False], kept=kept, info=_info(ref, n_kept=n),
                           top_p=[0.5], uniform=[0.3])
        assert rep.ok(), rep.summary()
    # one element further is 1e-3 of the mass away from top_p: a failure
    kept = _kept_prefix(ref, 502)[None]
    rep = compare_rows([ref.token], [0], [ref], [False], kept=kept, info=_info(ref, n_kept=502), top_p=[0.5],
                       uniform=[0.3])
    assert not rep.ok() and "exclusive mass" in rep.failures[0]
    # the right count but not a prefix of the sampling order (a kept element swapped for a
    # later one)
    kept = _kept_prefix(ref, 501)
    a, order, _ = ref.cut_window
    kept[order[0]] = 0
    kept[order[501 - a]] = 1
    rep = compare_rows([ref.token], [0], [ref], [False], kept=kept[None], info=_info(ref, n_kept=501),
                       top_p=[0.5], uniform=[0.3])
    assert not rep.ok() and "not a prefix" in rep.failures[0]


def test_draw_on_a_boundary_allows_the_neighbouring_token_only():
    # no top-p: Z_P = V = 1000, and u = 0.125 puts the draw point exactly on the boundary
    # between sampling positions 124 and 125
    row = _flat_row()
    u = 0.125
    ref = oracle.sample_row(row, "float32", 1.0, 0, 1.0, u)
    assert ref.draw_margin < 1e-6 and ref.token == 125
    for tok in (124, 125):
        rep = compare_rows([tok], [0], [ref], [False], info=_info(ref), top_p=[1.0], uniform=[u])
        assert rep.ok(), (tok, rep.summary())
        assert rep.exempt_tokens == 1 and rep.checked_tokens == 0
    for tok in (123, 126, 900):
        rep = compare_rows([tok], [0], [ref], [False], info=_info(ref), top_p=[1.0], uniform=[u])
        assert not rep.ok(), tok
    # clear of every boundary the token is held to exact equality
    ref = oracle.sample_row(row, "float32", 1.0, 0, 1.0, 0.1255)
    assert ref.draw_margin > 1e-6
    assert compare_rows([ref.token], [0], [ref], [False], top_p=[1.0], uniform=[0.1255]).checked_tokens == 1
    assert not compare_rows([ref.token + 1], [0], [ref], [False], top_p=[1.0], uniform=[0.1255]).ok()


def test_draw_point_follows_the_kernels_kept_mass():
    # the kernel kept one element fewer at the cutoff (Z_P 500 instead of 501): its draw
    # point u * 500 lies in the interval of the token it picks, not the oracle's
    row = _flat_row()
    u = 0.999
    ref = oracle.sample_row(row, "float32", 1.0, 0, 0.5, u, want_probs=True)
    assert ref.n_kept == 501
    kept = _kept_prefix(ref, 500)[None]
    tok_kernel = int(ref.cut_window[1][499 - ref.cut_window[0]])  # position floor(0.999 * 500) = 499
    rep = compare_rows([tok_kernel], [0], [ref], [False], kept=kept, info=_info(ref, n_kept=500, z_p=500.0),
                       top_p=[0.5], uniform=[u])
    assert rep.ok(), rep.summary()
    rep = compare_rows([ref.token], [0], [ref], [False], kept=kept, info=_info(ref, n_kept=500, z_p=500.0),
                       top_p=[0.5], uniform=[u])
    assert not rep.ok()


def test_infinite_temperature_is_a_bad_parameter():
    row = _flat_row(8)
    assert oracle.sample_row(row, "float32", float("inf"), 0, 1.0, 0.5).status == oracle.ROW_BAD_PARAM
    assert oracle.sample_row(row, "float32", float("nan"), 0, 1.0, 0.5).status == oracle.ROW_BAD_PARAM
