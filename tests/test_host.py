"""Host side of the sampler without a GPU: parameter mirror, packing, uniforms, the C ABI's
exported symbols and argument validation (calls that return before any HIP work).
"""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest
import torch

from pagedbatch_amd import SamplingParams, _lib, sample, sample_token
from pagedbatch_amd import sampling as smp

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pbsample.h")
ATTN_HEADER = os.path.join(ROOT, "include", "pbattn.h")
LMHEAD_HEADER = os.path.join(ROOT, "include", "pblmhead.h")


# ---------------------------------------------------------------- SamplingParams mirror
@pytest.mark.parametrize("kw,msg", [
    ({"max_tokens": 0}, "max_tokens must be >= 1"),
    ({"temperature": -0.1}, "temperature must be >= 0"),
    ({"top_p": 0.0}, r"top_p must be in \(0, 1\]"),
    ({"top_p": 1.01}, r"top_p must be in \(0, 1\]"),
    ({"top_k": -1}, "top_k must be >= 0"),
])
def test_sampling_params_validation(kw, msg):
    """Same errors as pagedbatch/config.py:146-154."""
    with pytest.raises(ValueError, match=msg):
        SamplingParams(**kw)


def test_sampling_params_defaults():
    sp = SamplingParams()
    assert (sp.max_tokens, sp.temperature, sp.top_p, sp.top_k, sp.ignore_eos, sp.seed, sp.stop_token_ids) == \
        (64, 1.0, 1.0, 0, False, None, ())
    assert SamplingParams(temperature=0.0).greedy and not sp.greedy


# ---------------------------------------------------------------- packing and uniforms
def test_pack_layout():
    h = smp._pack(3, [0.0, 0.7, 1.0], [0, 5, 1000], [1.0, 0.9, 0.5], [0.0, 0.25, 0.75], [2, 0, 1], vocab=1000)
    assert h.dtype == np.int32 and h.shape == (5, 3)
    assert np.array_equal(h[0].view(np.float32), np.float32([0.0, 0.7, 1.0]))
    assert list(h[1]) == [0, 5, 0]  # top_k >= vocab is off (sampling.py:15)
    assert np.array_equal(h[2].view(np.float32), np.float32([1.0, 0.9, 0.5]))
    assert np.array_equal(h[3].view(np.float32), np.float32([0.0, 0.25, 0.75]))
    assert list(h[4]) == [2, 0, 1]


def test_draw_uniforms_consumes_generators_like_the_reference():
    """One torch.rand per stochastic row, in row order; greedy rows draw nothing
    (pagedbatch/sampling.py:12-13 returns before touching the generator)."""
    shared = torch.Generator().manual_seed(42)
    params = [SamplingParams(temperature=1.0), SamplingParams(temperature=0.0), SamplingParams(temperature=0.5)]
    us = smp.draw_uniforms(params, [shared, shared, shared])
    ref = torch.Generator().manual_seed(42)
    a, b = float(torch.rand((), generator=ref)), float(torch.rand((), generator=ref))
    assert us == [a, 0.0, b]
    # the generator has advanced by exactly two draws
    assert float(torch.rand((), generator=shared)) == float(torch.rand((), generator=ref))


def test_draw_uniforms_mixed_generators_match_scalar_draws():
    """Runs of rows sharing a generator are drawn in one call; the numbers and the final
    generator states equal one scalar torch.rand per stochastic row in row order."""
    def make():
        shared = torch.Generator().manual_seed(7)
        seeded = [torch.Generator().manual_seed(100 + i) for i in range(3)]
        gens = [shared, shared, seeded[0], shared, shared, shared, seeded[1], seeded[1], shared, seeded[2]] * 3
        return shared, seeded, gens
    temps = [1.0, 0.0, 0.7, 1.0, 0.0, 1.3, 1.0, 1.0, 0.0, 0.9] * 3
    params = [SamplingParams(temperature=t) for t in temps]
    shared, seeded, gens = make()
    us = smp.draw_uniforms(params, gens)
    rshared, rseeded, rgens = make()
    want = [float(torch.rand((), generator=g)) if t != 0 else 0.0 for t, g in zip(temps, rgens)]
    assert us == want
    for a, b in zip([shared] + seeded, [rshared] + rseeded):
        assert float(torch.rand((), generator=a)) == float(torch.rand((), generator=b))


def test_top_k_codes():
    """top_k as the kernel gets it: 0 < k < V kept, k >= V off (sampling.py:15), a negative
    k passed on as -1 so that the kernel flags the row instead of silently sampling it."""
    assert list(smp._top_k_codes([0, 1, 999, 1000, 10**12, -1, -7], 1000)) == [0, 1, 999, 0, 0, -1, -1]
    h = smp._pack(2, [1.0, 1.0], [-2, 5], [1.0, 1.0], [0.5, 0.5], None, vocab=10)
    assert list(h[1]) == [-1, 5]


@pytest.mark.parametrize("n", [16, 17, 64, 255, 1000, 20000])
def test_batched_rand_equals_scalar_draws(n):
    """torch.rand(n) gives the numbers of n scalar torch.rand draws, in order, and leaves
    the generator where they leave it: what lets a run of rows that share a generator (the
    engine's, engine.py:58) take its uniforms from one call."""
    a, b = torch.Generator().manual_seed(n), torch.Generator().manual_seed(n)
    batch = torch.rand(n, generator=a)
    scalars = torch.tensor([float(torch.rand((), generator=b)) for _ in range(n)])
    assert torch.equal(batch, scalars)
    assert torch.equal(a.get_state(), b.get_state())


def test_shared_generator_uniforms_match_scalar_draws():
    """256 rows, every stochastic one on the shared generator (the fast path: one call)."""
    temps = np.array([0.0 if i % 3 == 0 else 1.0 for i in range(256)])
    g, r = torch.Generator().manual_seed(9), torch.Generator().manual_seed(9)
    u = smp._uniforms(temps, [g] * 256)
    want = [0.0 if t == 0 else float(torch.rand((), generator=r)) for t in temps]
    assert u.dtype == np.float32 and list(u.astype(np.float64)) == want
    assert torch.equal(g.get_state(), r.get_state())


def test_finish_staging_layout():
    """The finish block matches what _launch hands pbs_finish_reasons (engine.py:173-182
    inputs): stop offsets, num_output, max_tokens, num_tokens, ignore_eos bytes, stop ids."""
    from pagedbatch_amd.finish import FinishRule

    rules = [FinishRule(False, (), 3, 10, 20), FinishRule(True, (5, 9), 10, 10, 30), FinishRule(False, (7,), 1, 4, 5)]
    cap, base = 64, 7
    stop_base = base + (cap + 1) + 3 * cap + cap // 4
    hin = np.zeros(stop_base + 64, dtype=np.int32)
    assert smp._write_finish(hin, base, cap, stop_base, rules, 3) == 3
    assert list(hin[base:base + 4]) == [0, 0, 2, 3]
    o = base + cap + 1
    assert list(hin[o:o + 3]) == [3, 10, 1]
    assert list(hin[o + cap:o + cap + 3]) == [10, 10, 4]
    assert list(hin[o + 2 * cap:o + 2 * cap + 3]) == [20, 30, 5]
    assert list(hin[o + 3 * cap:o + 3 * cap + 1].view(np.uint8)[:3]) == [0, 1, 0]
    assert list(hin[stop_base:stop_base + 3]) == [5, 9, 7]


def test_no_cpu_path():
    x = torch.randn(2, 100)
    with pytest.raises(ValueError, match="no CPU path"):
        sample(x, [SamplingParams()] * 2, [torch.Generator()] * 2)
    with pytest.raises(ValueError):
        sample_token(torch.randn(3, 4), SamplingParams(), torch.Generator())


def test_status_mapping():
    smp._raise_for_status(np.zeros(4, np.int32))
    with pytest.raises(RuntimeError, match="probability tensor contains"):
        smp._raise_for_status(np.array([0, _lib.ROW_NAN], np.int32))
    with pytest.raises(RuntimeError, match="probability tensor contains"):
        smp._raise_for_status(np.array([_lib.ROW_NONFINITE], np.int32))
    with pytest.raises(ValueError):
        smp._raise_for_status(np.array([0, 0, _lib.ROW_BAD_PARAM], np.int32))


# ---------------------------------------------------------------- the C ABI library
def _header_functions(path: str = HEADER) -> list[str]:
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"\b(pb[sa]_\w+)\s*\(", text)


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    names = _header_functions()
    assert set(names) == set(_lib.SYMBOLS), (names, _lib.SYMBOLS)
    attn = _header_functions(ATTN_HEADER)
    assert set(attn) == set(_lib.ATTN_SYMBOLS), (attn, _lib.ATTN_SYMBOLS)
    lmh = _header_functions(LMHEAD_HEADER)
    assert set(lmh) == set(_lib.LMHEAD_SYMBOLS), (lmh, _lib.LMHEAD_SYMBOLS)
    raw = ctypes.CDLL(_lib.LIB_PATH)
    for n in names + attn + lmh:
        assert hasattr(raw, n), n
    assert lib.pbs_abi_version() == _lib.ABI_VERSION
    m = re.search(r"#define PBS_ABI_VERSION (\d+)", open(HEADER).read())
    assert int(m.group(1)) == _lib.ABI_VERSION
    assert lib.pbs_workspace_bytes(256, 128256, _lib.DTYPE_BF16) == 0


def test_header_constants_match_binding():
    text = open(HEADER).read()
    consts = dict((k, int(v)) for k, v in re.findall(r"(PBS_\w+)\s*=\s*(-?\d+)", text))
    assert consts["PBS_DTYPE_F32"] == _lib.DTYPE_F32
    assert consts["PBS_DTYPE_F16"] == _lib.DTYPE_F16
    assert consts["PBS_DTYPE_BF16"] == _lib.DTYPE_BF16
    assert consts["PBS_OK"] == _lib.OK
    assert consts["PBS_ERR_INVALID_ARGUMENT"] == _lib.ERR_INVALID_ARGUMENT
    assert consts["PBS_ERR_UNSUPPORTED_DTYPE"] == _lib.ERR_UNSUPPORTED_DTYPE
    assert consts["PBS_ERR_HIP"] == _lib.ERR_HIP
    assert consts["PBS_ROW_NAN"] == _lib.ROW_NAN
    assert consts["PBS_ROW_NONFINITE"] == _lib.ROW_NONFINITE
    assert consts["PBS_ROW_BAD_PARAM"] == _lib.ROW_BAD_PARAM


def test_row_info_layout_matches_c(tmp_path):
    """offsetof() of every pbs_row_info field, from gcc, against the numpy record type."""
    fields = _lib.ROW_INFO_DTYPE.names
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "pbsample.h"\nint main(void){\n'
                   + "".join(f'printf("%zu\\n", offsetof(pbs_row_info, {f}));\n' for f in fields)
                   + 'printf("%zu\\n", sizeof(pbs_row_info));\nreturn 0;}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)], check=True)
    out = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    assert out[:-1] == [_lib.ROW_INFO_DTYPE.fields[f][1] for f in fields]
    assert out[-1] == _lib.ROW_INFO_DTYPE.itemsize


def _call(lib, **kw):
    a = dict(logits=1 << 20, dtype=_lib.DTYPE_BF16, n_rows=4, rows=4, vocab=1000, stride=1000, row_map=None,
             t=1 << 20, k=1 << 20, p=1 << 20, u=1 << 20, tok=1 << 20, st=1 << 20)
    a.update(kw)
    return lib.pbs_sample(a["logits"], a["dtype"], a["n_rows"], a["rows"], a["vocab"], a["stride"], a["row_map"],
                          a["t"], a["k"], a["p"], a["u"], a["tok"], a["st"], None, 0, None)


@pytest.mark.parametrize("kw,code,msg", [
    ({"dtype": 7}, _lib.ERR_UNSUPPORTED_DTYPE, "unsupported dtype"),
    ({"rows": -1}, _lib.ERR_INVALID_ARGUMENT, "negative"),
    ({"vocab": 0}, _lib.ERR_INVALID_ARGUMENT, "vocab"),
    ({"vocab": (1 << 27) + 1, "stride": (1 << 27) + 1}, _lib.ERR_INVALID_ARGUMENT, "vocab"),
    ({"stride": 999}, _lib.ERR_INVALID_ARGUMENT, "row_stride"),
    ({"logits": None}, _lib.ERR_INVALID_ARGUMENT, "null"),
    ({"u": None}, _lib.ERR_INVALID_ARGUMENT, "null"),
    ({"n_rows": 2}, _lib.ERR_INVALID_ARGUMENT, "n_logit_rows"),
])
def test_abi_rejects_bad_arguments_before_any_device_work(kw, code, msg):
    """Validation happens on the host before anything is launched (no GPU needed here)."""
    lib = _lib.load()
    assert _call(lib, **kw) == code
    assert msg in _lib.last_error(lib)


@pytest.mark.parametrize("kw,code,msg", [
    ({"hdim": 100}, _lib.ERR_INVALID_ARGUMENT, "multiple of 64"),
    ({"stride": 60}, _lib.ERR_INVALID_ARGUMENT, "hidden_stride"),
    ({"vocab": 0}, _lib.ERR_INVALID_ARGUMENT, "vocab"),
    ({"weight": None}, _lib.ERR_INVALID_ARGUMENT, "null"),
    ({"vocab": 1 << 24, "hdim": 128, "stride": 128}, _lib.ERR_INVALID_ARGUMENT, "2^31"),
    ({"hidden": (1 << 20) + 8}, _lib.ERR_INVALID_ARGUMENT, "16-byte"),
    ({"ws_bytes": 8}, _lib.ERR_WORKSPACE, "workspace"),
])
def test_lm_head_abi_rejects_bad_arguments(kw, code, msg):
    lib = _lib.load()
    a = dict(hidden=1 << 20, stride=64, weight=1 << 20, rows=4, hdim=64, vocab=1000, ws_bytes=1 << 20)
    a.update(kw)
    rc = lib.pbs_lm_head_argmax(a["hidden"], a["stride"], a["weight"], a["rows"], a["hdim"], a["vocab"], None,
                                1 << 20, 1 << 20, a["ws_bytes"], None)
    assert rc == code
    assert msg in _lib.last_error(lib)
    assert lib.pbs_lm_head_workspace_bytes(4, 1000) == 4 * 16 * 8


def test_abi_zero_rows_is_a_no_op():
    lib = _lib.load()
    assert _call(lib, rows=0) == _lib.OK


def _argmax_call(lib, **kw):
    a = dict(logits=1 << 20, dtype=_lib.DTYPE_BF16, n_rows=4, rows=4, vocab=1000, stride=1000, row_map=None,
             tok=1 << 20, st=1 << 20)
    a.update(kw)
    return lib.pbs_argmax(a["logits"], a["dtype"], a["n_rows"], a["rows"], a["vocab"], a["stride"], a["row_map"],
                          a["tok"], a["st"], None)


@pytest.mark.parametrize("kw,code,msg", [
    ({"dtype": 3}, _lib.ERR_UNSUPPORTED_DTYPE, "unsupported dtype"),
    ({"n_rows": -1}, _lib.ERR_INVALID_ARGUMENT, "negative"),
    ({"vocab": 0}, _lib.ERR_INVALID_ARGUMENT, "vocab"),
    ({"stride": 10}, _lib.ERR_INVALID_ARGUMENT, "row_stride"),
    ({"tok": None}, _lib.ERR_INVALID_ARGUMENT, "null"),
    ({"st": None}, _lib.ERR_INVALID_ARGUMENT, "null"),
    ({"rows": 5}, _lib.ERR_INVALID_ARGUMENT, "n_logit_rows"),
])
def test_argmax_abi_rejects_bad_arguments(kw, code, msg):
    lib = _lib.load()
    assert _argmax_call(lib, **kw) == code
    assert msg in _lib.last_error(lib)
    assert _argmax_call(lib, rows=0) == _lib.OK


def test_all_greedy_routing():
    """The Python surface sends a block to pbs_argmax only when every row is greedy with
    parameters pbs_sample would accept, so both entry points give the same result."""
    def block(t, k, p):
        return smp._pack(len(t), t, k, p, [0.5] * len(t), None, 1000)

    assert smp._all_greedy(block([0.0, -0.0], [0, 5], [1.0, 0.3]))
    assert not smp._all_greedy(block([0.0, 1.0], [0, 0], [1.0, 1.0]))
    assert not smp._all_greedy(block([0.0, 0.0], [0, -1], [1.0, 1.0]))
    assert not smp._all_greedy(block([0.0], [0], [0.0]))
    assert not smp._all_greedy(block([0.0], [0], [1e-50]))  # zero in float32
    assert not smp._all_greedy(block([0.0], [0], [float("nan")]))


def test_debug_outputs_need_info():
    lib = _lib.load()
    rc = lib.pbs_sample_debug(1 << 20, _lib.DTYPE_F32, 1, 1, 10, 10, None, 1 << 20, 1 << 20, 1 << 20, 1 << 20,
                              1 << 20, 1 << 20, 1 << 20, None, None, None, 0, None)
    assert rc == _lib.ERR_INVALID_ARGUMENT and "out_info" in _lib.last_error(lib)


def test_paged_kv_slots_are_distinct_and_blocked():
    """Block tables give every (sequence, position) its own slot, block_size consecutive
    positions per block (block_manager.py:88-91)."""
    from pagedbatch_amd.engine_step import ModelShape, PagedKV

    kv = PagedKV(ModelShape.tiny(), num_seqs=5, max_len=37, block_size=8, device="cpu", dtype=torch.float32)
    seq = torch.arange(5).view(-1, 1)
    pos = torch.arange(37).view(1, -1).expand(5, -1)
    s = kv.slots(seq, pos)
    assert s.unique().numel() == 5 * 37
    assert int(s.max()) < kv.k[0].shape[0]
    # within a block the slots are consecutive
    assert torch.equal(s[:, 1:8] - s[:, :7], torch.ones(5, 7, dtype=s.dtype))


def _attn(lib, **kw):
    a = dict(q=1 << 20, k=1 << 20, v=1 << 20, n_slots=64, bt=1 << 20, max_blocks=4, lens=1 << 20, rows=2, hq=9, hkv=3,
             d=64, bs=16, maxc=64, out=1 << 20)
    a.update(kw)
    return lib.pba_decode_attention(a["q"], a["k"], a["v"], a["n_slots"], a["bt"], a["max_blocks"], a["lens"], a["rows"],
                                    a["hq"], a["hkv"], a["d"], a["bs"], a["maxc"], 0.125, a["out"], None)


@pytest.mark.parametrize("kw,msg", [
    ({"rows": -1}, "negative"),
    ({"q": None}, "null"),
    ({"d": 96}, "head_dim must be 64 or 128"),
    ({"hq": 10}, "multiple"),
    ({"hq": 27}, "at most 8"),
    ({"maxc": 65}, "max_context"),
    ({"maxc": (1 << 20) + 1, "max_blocks": 1 << 17}, "max_context"),
    ({"bs": 0}, "block_size"),
    ({"n_slots": 1 << 31}, "n_slots"),
    ({"q": (1 << 20) + 4}, "16-byte aligned"),
    ({"v": (1 << 20) + 8}, "16-byte aligned"),
])
def test_attention_abi_rejects_bad_arguments(kw, msg):
    lib = _lib.load()
    assert _attn(lib, **kw) == _lib.ERR_INVALID_ARGUMENT
    assert msg in _lib.last_error(lib)


def test_attention_abi_zero_rows_is_a_no_op():
    assert _attn(_lib.load(), rows=0) == _lib.OK


# ---------------------------------------------------------------- decode_attention's checks
def _attn_tensors(**kw):
    t = dict(q=torch.zeros(2, 9, 64), k=torch.zeros(64, 3, 64, dtype=torch.bfloat16),
             v=torch.zeros(64, 3, 64, dtype=torch.bfloat16), bt=torch.zeros(2, 4, dtype=torch.int32),
             lens=torch.ones(2, dtype=torch.int32))
    t.update(kw)
    return t


@pytest.mark.parametrize("kw,msg", [
    ({"q": torch.zeros(2, 9, 32)}, "head_dim must be 64 or 128"),
    ({"k": torch.zeros(64, 3, 32, dtype=torch.bfloat16), "v": torch.zeros(64, 3, 32, dtype=torch.bfloat16)},
     "head_dim 32 differs"),
    ({"v": torch.zeros(64, 3, 64)}, "v_cache must be a contiguous bf16"),
    ({"v": torch.zeros(32, 3, 64, dtype=torch.bfloat16)}, "differ in shape"),
    ({"bt": torch.zeros(3, 4, dtype=torch.int32)}, "one row per query row"),
    ({"lens": torch.ones(2, dtype=torch.int64)}, "context_lens"),
    ({"k": torch.zeros(64, 3, 64, dtype=torch.bfloat16, device="meta")}, "every operand must be on q's device"),
    ({"bt": torch.zeros(2, 4, dtype=torch.int32, device="meta")}, "every operand must be on q's device"),
    ({"k": torch.zeros(64 * 3 * 64 + 1, dtype=torch.bfloat16)[1:].view(64, 3, 64)}, "16-byte boundary"),
    ({}, "no CPU path"),
])
def test_decode_attention_rejects_bad_operands(kw, msg):
    """Every operand is checked before the kernel sees a pointer: a cache with another
    head size, a tensor on another device or on the host, a view off a 16-byte boundary."""
    from pagedbatch_amd.attention import decode_attention

    t = _attn_tensors(**kw)
    with pytest.raises(ValueError, match=msg):
        decode_attention(t["q"], t["k"], t["v"], t["bt"], t["lens"], block_size=16, max_context=64)


# ---------------------------------------------------------------- engine harness (host side)
def test_engine_graph_needs_the_fused_decode_step():
    from pagedbatch_amd import engine_step as es

    with pytest.raises(ValueError, match="fused_decode"):
        es.run(es.ModelShape.tiny(), num_seqs=2, prompt_len=4, output_len=2, block_size=4, device="cpu", graph=True)


def test_engine_forward_without_seq_slots_needs_context_lens():
    import torch

    from pagedbatch_amd import engine_step as es

    shape = es.ModelShape.tiny()
    model = es.Model(shape, torch.device("cpu"))
    cache = es.PagedKV(shape, 2, 8, 4, "cpu", torch.bfloat16)
    t = torch.zeros(2, dtype=torch.long)
    with pytest.raises(ValueError, match="context_lens"):
        model.forward(t, t, t, None, 1, cache, fused_decode=True)
