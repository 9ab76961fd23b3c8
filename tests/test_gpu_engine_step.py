"""The engine-step harness (pagedbatch_amd.engine_step): one batched sampling call per step
gives the same tokens as one call per row (the reference's loop, engine.py:133-139), and
greedy rows follow the logits' argmax."""

from __future__ import annotations

import pytest
import torch

from pagedbatch_amd import engine_step as es

pytestmark = pytest.mark.gpu


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
