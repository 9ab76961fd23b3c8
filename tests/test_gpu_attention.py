"""Paged-attention decode kernel (pagedbatch/model.py:201-224) against the torch fp32
attention of the engine-step harness on the same cache, and the engine step run both ways."""

from __future__ import annotations

import math

import pytest
import torch

from pagedbatch_amd import _lib


def _torch_decode(q, kc, vc, block_table, lens, block_size, scale):
    """fp32 reference: gather each sequence's context through its block table, repeat the
    KV heads (model.py:214-216), softmax(q k^T * scale) v."""
    B, Hq, D = q.shape
    Hkv = kc.shape[1]
    rep = Hq // Hkv
    out = torch.empty(B, Hq, D, dtype=torch.float32)
    for b in range(B):
        L = int(lens[b])
        t = torch.arange(L)
        slots = block_table[b, t // block_size].long() * block_size + t % block_size
        k = kc[slots].float().repeat_interleave(rep, dim=1)  # [L, Hq, D]
        v = vc[slots].float().repeat_interleave(rep, dim=1)
        att = torch.einsum("hd,lhd->hl", q[b].float(), k) * scale
        out[b] = torch.einsum("hl,lhd->hd", torch.softmax(att, dim=-1), v)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("B,Hq,Hkv,bs,maxL,seed,D", [
    (4, 9, 3, 16, 200, 1, 64), (3, 8, 8, 8, 37, 2, 64), (2, 16, 2, 32, 1500, 3, 64), (5, 4, 1, 16, 1, 4, 64),
    (2, 16, 2, 16, 2048, 5, 64),
    (2, 9, 3, 16, 5000, 6, 64),      # a context past 2048
    (3, 32, 8, 16, 700, 7, 128),     # head_dim 128, four query heads per KV head (a Llama-3-8B layer)
    (2, 64, 8, 16, 300, 8, 128),     # eight per KV head (a Llama-3-70B layer)
    (3, 6, 1, 8, 90, 9, 128),        # six per KV head
])
def test_decode_matches_torch(B, Hq, Hkv, bs, maxL, seed, D):
    from pagedbatch_amd.attention import decode_attention

    print(f"[case] decode B={B} Hq={Hq} Hkv={Hkv} bs={bs} maxL={maxL} D={D}", flush=True)
    g = torch.Generator().manual_seed(seed)
    nblk = (maxL + bs - 1) // bs
    n_slots = B * nblk * bs + 3 * bs
    kc = (torch.randn(n_slots, Hkv, D, generator=g) * 0.5).to(torch.bfloat16)
    vc = torch.randn(n_slots, Hkv, D, generator=g).to(torch.bfloat16)
    perm = torch.randperm(n_slots // bs, generator=g)[: B * nblk].view(B, nblk).to(torch.int32)
    lens = torch.randint(1, maxL + 1, (B,), generator=g).to(torch.int32)
    lens[0] = maxL
    q = torch.randn(B, Hq, D, generator=g)
    scale = 1.0 / math.sqrt(D)
    want = _torch_decode(q, kc, vc, perm, lens, bs, scale)
    dev = torch.device("cuda", 0)
    got = decode_attention(q.to(dev), kc.to(dev), vc.to(dev), perm.to(dev), lens.to(dev), bs, maxL, scale).cpu()
    torch.testing.assert_close(got, want, rtol=2e-5, atol=2e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("B,Hq,Hkv,bs,maxL,seed,D", [(4, 9, 3, 16, 200, 11, 64), (3, 8, 2, 16, 700, 12, 64),
                                                     (2, 4, 4, 8, 1, 13, 64), (2, 32, 8, 16, 400, 14, 128)])
def test_decode_matches_reference_bf16_sdpa(B, Hq, Hkv, bs, maxL, seed, D):
    """Against the reference's own arithmetic (model.py:212-222): bf16 q, K and V gathered
    through the slot table, the KV heads repeated, F.scaled_dot_product_attention in bf16
    (on the CPU). The kernel computes in fp32 from the same bf16 inputs; torch's bf16 result
    differs from the exact one by at most a bf16 rounding of the weights and one of the
    output, so the bar is 2^-8 * (max |v| + |out|) per element."""
    import torch.nn.functional as F

    from pagedbatch_amd.attention import decode_attention

    print(f"[case] decode vs bf16 sdpa B={B} Hq={Hq} Hkv={Hkv} bs={bs} maxL={maxL} D={D}", flush=True)
    g = torch.Generator().manual_seed(seed)
    nblk = (maxL + bs - 1) // bs
    n_slots = B * nblk * bs + bs
    kc = (torch.randn(n_slots, Hkv, D, generator=g) * 0.5).to(torch.bfloat16)
    vc = torch.randn(n_slots, Hkv, D, generator=g).to(torch.bfloat16)
    perm = torch.randperm(n_slots // bs, generator=g)[: B * nblk].view(B, nblk).to(torch.int32)
    lens = torch.randint(1, maxL + 1, (B,), generator=g).to(torch.int32)
    lens[0] = maxL
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16)
    rep = Hq // Hkv
    want = torch.empty(B, Hq, D)
    bound = torch.empty(B, Hq, D)
    for b in range(B):
        L = int(lens[b])
        t = torch.arange(L)
        slots = perm[b, t // bs].long() * bs + t % bs
        keys = kc[slots].repeat_interleave(rep, dim=1).transpose(0, 1).unsqueeze(0)  # [1, Hq, L, D]
        values = vc[slots].repeat_interleave(rep, dim=1).transpose(0, 1).unsqueeze(0)
        o = F.scaled_dot_product_attention(q[b].view(1, Hq, 1, D), keys, values).view(Hq, D).float()
        want[b] = o
        vmax = values.float().abs().amax(dim=(2, 3)).view(Hq, 1)  # per head
        bound[b] = 2.0 ** -8 * (vmax + o.abs())
    dev = torch.device("cuda", 0)
    got = decode_attention(q.float().to(dev), kc.to(dev), vc.to(dev), perm.to(dev), lens.to(dev), bs, maxL).cpu()
    err = (got - want).abs()
    assert bool((err <= bound).all()), f"max err / bar {float((err / bound).max()):.3f}"
    if maxL == 1:  # a single position: the output is that V row, exactly
        assert torch.equal(got, want)


@pytest.mark.gpu
def test_decode_corrupt_block_table_gives_nan_not_a_fault():
    from pagedbatch_amd.attention import decode_attention

    dev = torch.device("cuda", 0)
    kc = torch.zeros(64, 1, 64, dtype=torch.bfloat16, device=dev)
    bt = torch.tensor([[0, 1], [0, 99]], dtype=torch.int32, device=dev)  # block 99 is past the 64 slots
    lens = torch.tensor([20, 20], dtype=torch.int32, device=dev)
    out = decode_attention(torch.ones(2, 2, 64, device=dev), kc, kc, bt, lens, 16, 32).cpu()
    assert torch.isfinite(out[0]).all() and torch.isnan(out[1]).all()


@pytest.mark.gpu
def test_decode_context_length_out_of_range_gives_nan():
    """A context length of 0 or past max_context: that sequence's output is NaN (no read),
    the others are computed."""
    from pagedbatch_amd.attention import decode_attention

    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(21)
    kc = torch.randn(64, 2, 128, generator=g).to(torch.bfloat16).to(dev)
    bt = torch.tensor([[0, 1], [2, 3], [1, 0]], dtype=torch.int32, device=dev)
    lens = torch.tensor([0, 20, 33], dtype=torch.int32, device=dev)  # max_context 32
    q = torch.randn(3, 4, 128, generator=g).to(dev)
    out = decode_attention(q, kc, kc, bt, lens, 16, 32).cpu()
    assert torch.isnan(out[0]).all() and torch.isnan(out[2]).all()
    assert torch.isfinite(out[1]).all()


@pytest.mark.gpu
def test_engine_decode_step_fused_matches_unfused():
    """One decode step of the tiny engine model on the same cache, attention fused or not:
    the same logits up to the bf16 rounding of the attention output (model.py:224's
    o_proj input), which is where the two fp32 results can first differ."""
    from pagedbatch_amd import engine_step as es

    dev = torch.device("cuda", 0)
    # a small model with the kernel's head_dim of 64
    shape = es.ModelShape(vocab_size=512, hidden_size=256, intermediate_size=256, num_layers=2, num_heads=4,
                          num_kv_heads=2)
    model = es.Model(shape, dev, seed=3)
    B, P, bs = 5, 21, 8
    cache = es.PagedKV(shape, B, P + 4, bs, dev, torch.bfloat16)
    seq = torch.arange(B, device=dev).view(-1, 1)
    g = torch.Generator().manual_seed(4)
    prompt = torch.randint(0, shape.vocab_size, (B, P), generator=g).to(dev)
    pos = torch.arange(P, device=dev).view(1, -1).expand(B, -1)
    model.forward(prompt.reshape(-1), pos.reshape(-1), cache.slots(seq, pos).reshape(-1), cache.slots(seq, pos), P, cache)
    tok = torch.randint(0, shape.vocab_size, (B, 1), generator=g).to(dev)
    pos1 = torch.full((B, 1), P, device=dev)
    ctx = torch.arange(P + 1, device=dev).view(1, -1).expand(B, -1)
    args = (tok.reshape(-1), pos1.reshape(-1), cache.slots(seq, pos1).reshape(-1), cache.slots(seq, ctx), 1, cache)
    plain = model.forward(*args).float()
    fused = model.forward(*args, fused_decode=True).float()
    torch.testing.assert_close(fused, plain, rtol=2e-2, atol=2e-3)
