"""Finish reasons (pagedbatch/engine.py:173-182): the oracle pinned on the reference's own
engine tests and the rule's cases; the C ABI's argument checks; the GPU kernel against
the oracle, exactly."""

from __future__ import annotations

import ctypes
import random

import numpy as np
import pytest
import torch

from oracle.finish import finish_reason
from pagedbatch_amd import _lib


# ------------------------------------------------------------------ the oracle, pinned
def test_reference_engine_tests_length_and_stop():
    # tests/test_engine.py:46: a greedy request with max_tokens=10 ends with "length" after
    # exactly 10 outputs (none of them EOS), and not before
    for n in range(1, 10):
        assert finish_reason(5, 2, False, (), n, 10, 3 + n, 2048) is None
    assert finish_reason(5, 2, False, (), 10, 10, 13, 2048) == "length"
    # tests/test_engine.py:54: stop_token_ids=(first,) ends the request with "stop" right
    # after the first output, which is kept
    assert finish_reason(17, 2, False, (17,), 1, 10, 4, 2048) == "stop"


def test_rule_cases():
    # EOS and stop ids, unless ignore_eos (engine.py:176-177)
    assert finish_reason(2, 2, False, (), 1, 64, 10, 2048) == "stop"
    assert finish_reason(2, None, False, (), 1, 64, 10, 2048) is None  # no EOS id
    assert finish_reason(9, 2, False, (4, 9, 11), 1, 64, 10, 2048) == "stop"
    assert finish_reason(2, 2, True, (2,), 1, 64, 10, 2048) is None
    # stop before length when both hold (engine.py:176 before 178)
    assert finish_reason(2, 2, False, (), 64, 64, 2048, 2048) == "stop"
    # ignore_eos leaves the length limits (engine.py:178-181)
    assert finish_reason(2, 2, True, (), 64, 64, 70, 2048) == "length"
    assert finish_reason(7, 2, True, (), 3, 64, 2048, 2048) == "length"
    assert finish_reason(7, 2, False, (), 3, 64, 2047, 2048) is None
    assert finish_reason(7, 2, False, (), 63, 64, 100, 2048) is None


# ------------------------------------------------------------------ the C ABI (no GPU)
def test_header_finish_constants_match_binding():
    import re
    from test_host import HEADER

    consts = dict((k, int(v)) for k, v in re.findall(r"(PBS_\w+)\s*=\s*(-?\d+)", open(HEADER).read()))
    assert consts["PBS_FINISH_NONE"] == _lib.FINISH_NONE
    assert consts["PBS_FINISH_STOP"] == _lib.FINISH_STOP
    assert consts["PBS_FINISH_LENGTH"] == _lib.FINISH_LENGTH


def _finish(lib, **kw):
    a = dict(tok=1 << 20, rows=4, eos=2, ign=1 << 20, offs=1 << 20, ids=None, nout=1 << 20, maxt=1 << 20,
             ntok=1 << 20, mml=2048, out=1 << 20)
    a.update(kw)
    return lib.pbs_finish_reasons(a["tok"], a["rows"], a["eos"], a["ign"], a["offs"], a["ids"], a["nout"],
                                  a["maxt"], a["ntok"], a["mml"], a["out"], None)


@pytest.mark.parametrize("kw,msg", [
    ({"rows": -1}, "negative"),
    ({"tok": None}, "null"),
    ({"offs": None}, "null"),
    ({"out": None}, "null"),
    ({"eos": -2}, "eos_token_id"),
])
def test_finish_abi_rejects_bad_arguments(kw, msg):
    lib = _lib.load()
    assert _finish(lib, **kw) == _lib.ERR_INVALID_ARGUMENT
    assert msg in _lib.last_error(lib)


def test_finish_abi_zero_rows_is_a_no_op():
    assert _finish(_lib.load(), rows=0) == _lib.OK


# ------------------------------------------------------------------ the kernel
def _random_rules(n, seed, eos):
    from pagedbatch_amd.finish import FinishRule

    rng = random.Random(seed)
    rules, toks = [], []
    for _ in range(n):
        stops = tuple(rng.sample(range(50), rng.choice([0, 0, 1, 2, 5, 17])))
        max_tokens = rng.randint(1, 40)
        num_output = rng.randint(1, 45)
        num_tokens = num_output + rng.randint(0, 120)
        tok = rng.choice([eos if eos is not None else 3, rng.randint(0, 60), rng.choice(stops) if stops else 49])
        rules.append(FinishRule(ignore_eos=rng.random() < 0.25, stop_token_ids=stops, num_output=num_output,
                                max_tokens=max_tokens, num_tokens=num_tokens))
        toks.append(tok)
    return rules, toks


@pytest.mark.gpu
@pytest.mark.parametrize("n,eos,mml", [(1, 2, 2048), (7, None, 64), (1000, 2, 100), (4099, 0, 150)])
def test_finish_kernel_matches_oracle(n, eos, mml):
    from pagedbatch_amd.finish import REASONS, finish_codes

    print(f"[case] finish n={n} eos={eos} max_model_len={mml}", flush=True)
    rules, toks = _random_rules(n, n * 31 + 7, eos)
    dev = torch.device("cuda", 0)
    codes = finish_codes(torch.tensor(toks, dtype=torch.int32, device=dev), rules, eos, mml).cpu().numpy()
    want = [finish_reason(t, eos, r.ignore_eos, r.stop_token_ids, r.num_output, r.max_tokens, r.num_tokens, mml)
            for t, r in zip(toks, rules)]
    got = [REASONS[c] for c in codes.tolist()]
    assert got == want
    # every reason occurs in the larger cases
    if n >= 1000:
        assert {None, "stop", "length"} <= set(got)


@pytest.mark.gpu
def test_finish_after_sampling_on_device():
    """The engine's use: sample a step's tokens, then the finish reasons, one copy back."""
    from pagedbatch_amd.finish import FinishRule, finish_reasons
    from pagedbatch_amd.sampling import sample_arrays

    dev = torch.device("cuda", 0)
    x = torch.zeros(3, 100, device=dev)
    x[0, 2] = 5.0   # greedy picks 2 = EOS
    x[1, 17] = 5.0  # greedy picks 17, a stop id of row 1
    x[2, 40] = 5.0  # greedy picks 40: no stop, at max_tokens
    tok, st = sample_arrays(x, [0.0] * 3, [0] * 3, [1.0] * 3, [0.0] * 3)
    rules = [FinishRule(False, (), 1, 10, 5), FinishRule(False, (17,), 1, 10, 5), FinishRule(False, (17,), 10, 10, 14)]
    got = finish_reasons(torch.from_numpy(np.asarray(tok, np.int32)).to(dev), rules, 2, 2048)
    assert got == ["stop", "stop", "length"]


@pytest.mark.gpu
@pytest.mark.parametrize("n", [3, 300])
def test_sample_and_finish_matches_the_oracle(n):
    """sample_and_finish: the sampler's tokens and, in the same copy back, the stop check
    of every row (engine.py:173-182) against the oracle on the tokens it produced; the
    tokens equal a plain sample() on the same inputs."""
    from pagedbatch_amd import SamplingParams, sample
    from pagedbatch_amd.sampling import sample_and_finish

    print(f"[case] sample_and_finish n={n}", flush=True)
    dev = torch.device("cuda", 0)
    rules, want_tok = _random_rules(n, 5 + n, 2)
    # greedy rows whose argmax is the planted token, so that EOS, stop ids and plain
    # tokens all occur; every fifth row stochastic
    x = torch.zeros(n, 64)
    x[torch.arange(n), torch.tensor(want_tok)] = 8.0
    params = [SamplingParams(temperature=0.0) if i % 5 else SamplingParams(temperature=1.0, top_k=3)
              for i in range(n)]
    g1, g2 = torch.Generator().manual_seed(4), torch.Generator().manual_seed(4)
    logits = x.to(dev)
    toks, reasons = sample_and_finish(logits, params, [g1] * n, rules, 2, 150)
    assert toks == sample(logits, params, [g2] * n)
    assert all(t == w for i, (t, w) in enumerate(zip(toks, want_tok)) if i % 5)
    want = [finish_reason(t, 2, r.ignore_eos, r.stop_token_ids, r.num_output, r.max_tokens, r.num_tokens, 150)
            for t, r in zip(toks, rules)]
    assert reasons == want
    if n >= 300:
        assert {None, "stop", "length"} <= set(reasons)
