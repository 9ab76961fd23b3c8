"""Planted mistakes in the oracle must be caught by the checks that pin it (CPU only).

Each case copies oracle/oracle.py, changes one line into a plausible mistake (a wrong
comparison side, inclusive instead of exclusive mass, a reversed tie order, an off-by-one
k-th value, a reciprocal instead of a division, ...) and runs the pinning checks of
tests/oracle_checks.py on the copy. A mistake no check notices would mean the oracle is not
pinned where that line matters.
"""

from __future__ import annotations

import os
import sys
import types

import pytest

import oracle_checks as oc

SRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "oracle.py")

MUTATIONS = {
    "draw_side_left": ('j = int(np.searchsorted(ck, t, side="right"))', 'j = int(np.searchsorted(ck, t, side="left"))'),
    "top_p_side_left": ('np.searchsorted(excl, thr, side="right")', 'np.searchsorted(excl, thr, side="left")'),
    "top_p_inclusive_mass": ('np.searchsorted(excl, thr, side="right")', 'np.searchsorted(csum, thr, side="right")'),
    "tie_order_index_descending": (
        'order = idx_k[np.argsort(-x[idx_k], kind="stable")]',
        'order = idx_k[::-1][np.argsort(-x[idx_k][::-1], kind="stable")]'),
    "kth_off_by_one": ("return np.partition(x, x.size - k)[x.size - k]",
                       "return np.partition(x, max(x.size - k - 1, 0))[max(x.size - k - 1, 0)]"),
    "top_k_strict": ("in_k = x >= kth", "in_k = x > kth"),
    "greedy_last_max": ("return int(np.argmax(x))  #", "return int(x.size - 1 - np.argmax(x[::-1]))  #"),
    "greedy_skips_nan": ("return int(np.argmax(nan))", "return int(np.nanargmax(x)) if not nan.all() else 0"),
    "scale_by_reciprocal": ("return (row32 / np.float32(temperature)).astype(np.float32)",
                            "return (row32 * (np.float32(1.0) / np.float32(temperature))).astype(np.float32)"),
    "probs_over_top_k_mass": ("probs[kept_sorted] = w[kept_sorted] / z_p", "probs[kept_sorted] = w[kept_sorted] / z_k"),
    "top_p_on_unfiltered_row": ("    if 0 < top_k < V:\n        kth", "    if False:\n        kth"),
}


def mutated_oracle(name: str):
    old, new = MUTATIONS[name]
    src = open(SRC).read()
    assert src.count(old) == 1, f"mutation {name}: pattern must occur exactly once in oracle.py"
    mod = types.ModuleType(f"oracle_mutant_{name}")
    sys.modules[mod.__name__] = mod  # dataclasses resolve annotations through sys.modules
    try:
        exec(compile(src.replace(old, new), f"<oracle mutant {name}>", "exec"), mod.__dict__)
    finally:
        del sys.modules[mod.__name__]
    return mod


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_planted_mistake_is_caught(name):
    mod = mutated_oracle(name)
    caught = {}
    for check in oc.ALL_CHECKS:
        try:
            fails = check(mod)
        except Exception as e:  # a mutant that crashes on a pinned case is caught too
            fails = [f"{type(e).__name__}: {e}"]
        if fails:
            caught[check.__name__] = fails[0]
    assert caught, f"planted mistake {name!r} passes every pinning check"
