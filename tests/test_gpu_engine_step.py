"""The engine-step harness (pagedbatch_amd.engine_step) on the GPU.

* The configuration the engine benchmark runs (a smollm2-135m-shaped random bf16 model, 64
  requests of 128 prompt tokens, half greedy and half top-k=50 / top-p=0.9, block size 16):
  every captured step's tokens against the oracle on that step's own logits and
  uniforms (pagedbatch/engine.py:130-139 samples these rows one by one), greedy rows bit
  for bit, and the finish reasons the batched call brings back (engine.py:173-182).
* One batched sampling call per step gives the same tokens as one call per row (the
  reference's loop, engine.py:133-139); greedy rows follow the logits' argmax.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from oracle.compare import compare_rows
from pagedbatch_amd import engine_step as es
from pagedbatch_amd.sampling import sample_arrays

pytestmark = pytest.mark.gpu


def test_smollm2_64_requests_match_the_oracle(dev):
    """Prefill plus three decode steps at the benchmark's shape, decode attention through
    the paged-attention kernel; each step's sampling checked against the oracle."""
    steps = 4
    print("[case] engine step smollm2-135m shape, 64 requests, 4 steps", flush=True)
    times, out = es.run(es.ModelShape(), num_seqs=64, prompt_len=128, output_len=steps, block_size=16, device=dev,
                        fused_decode=True, capture_steps=range(steps))
    assert len(times.captures) == steps and all(len(o) == steps for o in out)
    for cap in times.captures:
        greedy = [t == 0 for t in cap.temperature]
        raw = cap.logits.cpu().view(torch.int16).numpy().view(np.uint16)
        refs = oracle.sample_batch(raw, "bfloat16", cap.temperature, cap.top_k, cap.top_p, cap.uniform,
                                   want_probs=True)
        dbg = sample_arrays(cap.logits, cap.temperature, cap.top_k, cap.top_p, cap.uniform, debug=True)
        # the engine's own call and the diagnostic call agree on the same inputs
        assert list(dbg.tokens) == cap.tokens
        assert (dbg.status == 0).all()
        rep = compare_rows(dbg.tokens, dbg.status, refs, greedy, probs=dbg.probs.cpu().numpy(),
                           kept=dbg.kept.cpu().numpy(), info=dbg.info, top_p=cap.top_p, uniform=cap.uniform)
        exact = rep.checked_tokens - sum(greedy)
        print(f"[case] step {cap.step}: {rep.summary()} exactly checked stochastic rows {exact}/32", flush=True)
        assert rep.ok(), rep.summary()
        assert [int(t) for t, g in zip(dbg.tokens, greedy) if g] == [r.token for r, g in zip(refs, greedy) if g]
        assert exact >= 16
    # every request reaches its 4 outputs together: no reason before the last step,
    # "length" for all at it (the random model has no EOS here)
    assert all(r is None for rs in times.reasons[:-1] for r in rs)
    assert times.reasons[-1] == ["length"] * 64


def test_batched_equals_per_row_tiny_model(dev):
    print("[case] engine step tiny model, batched vs per-row", flush=True)
    kw = dict(num_seqs=8, prompt_len=16, output_len=6, block_size=4, device=dev)
    tb, out_b = es.run(es.ModelShape.tiny(), **kw)
    tr, out_r = es.run(es.ModelShape.tiny(), **kw, per_row=True)
    assert out_b == out_r
    assert len(tb.forward_s) == 6 and all(len(o) == 6 for o in out_b)


def test_greedy_rows_take_the_argmax(dev):
    print("[case] engine step greedy argmax", flush=True)
    shape = es.ModelShape.tiny()
    model = es.Model(shape, torch.device(dev), seed=3)
    B, L = 4, 8
    cache = es.PagedKV(shape, B, L, 4, dev, torch.bfloat16)
    seq = torch.arange(B, device=dev).view(-1, 1)
    pos = torch.arange(L, device=dev).view(1, -1).expand(B, -1)
    tokens = torch.randint(0, shape.vocab_size, (B, L), generator=torch.Generator().manual_seed(0)).to(dev)
    slots = cache.slots(seq, pos)
    logits = model.forward(tokens.reshape(-1), pos.reshape(-1), slots.reshape(-1), slots, L, cache)
    from pagedbatch_amd import SamplingParams, sample
    toks = sample(logits, [SamplingParams(temperature=0.0)] * B, [torch.Generator()] * B)
    assert toks == [int(t) for t in torch.argmax(logits, dim=-1).cpu()]


@pytest.mark.parametrize("fused_head", [False, True])
def test_graph_replay_equals_eager_decode(dev, fused_head):
    """The decode forward replayed from a HIP graph (engine_step.DecodeGraph) runs the same
    kernels as the eager step: every step's logits (captured after each replay, with the
    eager sampling, stop check and input preparation between replays) are bit-identical to
    the eager run's, and so are the tokens and finish reasons."""
    print(f"[case] engine step graph replay vs eager, fused_head={fused_head}", flush=True)
    steps = 6
    # head_dim 64 (the paged-attention kernel's), three layers, 2 query heads per KV head
    shape = es.ModelShape(vocab_size=1000, hidden_size=256, intermediate_size=512, num_layers=3, num_heads=4,
                          num_kv_heads=2)
    kw = dict(num_seqs=8, prompt_len=16, output_len=steps, block_size=4, device=dev, fused_decode=True,
              fused_head=fused_head)
    if not fused_head:
        kw["capture_steps"] = range(steps)
    te, out_e = es.run(shape, **kw)
    tg, out_g = es.run(shape, **kw, graph=True)
    assert out_g == out_e
    assert tg.reasons == te.reasons
    for ce, cg in zip(te.captures, tg.captures):
        assert ce.step == cg.step
        assert torch.equal(ce.logits.view(torch.int16), cg.logits.view(torch.int16)), f"step {ce.step}"


def test_sampling_graph_matches_the_eager_call(dev):
    """sampling.SamplingGraph against sample_and_finish on the same logits buffer and the
    same generator states, over several replays with new logits, eager sampler calls and
    synchronisations between them; bf16 and fp32 logits, mixed rows, a row map, stop ids."""
    from pagedbatch_amd import SamplingGraph, SamplingParams, sample_and_finish
    from pagedbatch_amd.finish import FinishRule

    g = torch.Generator().manual_seed(5)
    for dtype in (torch.bfloat16, torch.float32):
        print(f"[case] sampling graph {dtype}", flush=True)
        B, V = 12, 3000
        buf = torch.empty(B, V, dtype=dtype, device=dev)
        rows = [0, 2, 3, 5, 7, 8, 9, 11]
        params = [SamplingParams(temperature=0.0), SamplingParams(temperature=0.7, top_k=20),
                  SamplingParams(temperature=1.0, top_p=0.9), SamplingParams(temperature=1.3),
                  SamplingParams(temperature=0.0), SamplingParams(temperature=1.0, top_k=5, top_p=0.8),
                  SamplingParams(temperature=0.9, top_p=0.95), SamplingParams(temperature=1.1, top_k=100)]
        shared = torch.Generator().manual_seed(11)
        seeded = torch.Generator().manual_seed(12)
        gens = [shared, shared, seeded, shared, shared, shared, seeded, shared]

        def rules(step):
            return [FinishRule(ignore_eos=(i % 3 == 0), stop_token_ids=(7, 11 + i), num_output=step + 1,
                               max_tokens=4, num_tokens=20 + step) for i in range(len(rows))]

        sg = SamplingGraph(buf, params, rows=rows, finish_rules=rules(0), eos_token_id=2, max_model_len=64)
        for step in range(4):
            x = torch.randn(B, V, generator=g) * 3.0
            x[:, 7] = 30.0 if step == 2 else x[:, 7]   # a step whose greedy rows hit a stop id
            buf.copy_(x.to(dtype))
            ref_state = [shared.get_state(), seeded.get_state()]
            want = sample_and_finish(buf, params, gens, rules(step), 2, 64, rows=rows)
            shared.set_state(ref_state[0])
            seeded.set_state(ref_state[1])
            got = sg(gens, rules(step))
            assert got == want, f"step {step}: {got} != {want}"
            torch.cuda.synchronize()
            sample_and_finish(buf, params, [torch.Generator().manual_seed(99)] * len(rows), rules(step), 2, 64,
                              rows=rows)  # eager work between replays
