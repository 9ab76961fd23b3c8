"""The fused lm_head + greedy kernel (pbs_lm_head_argmax) on the GPU against a float64
restatement of pagedbatch/model.py:283 (hidden @ weight.T) computed on the CPU, and its
greedy tokens against the oracle's torch.argmax restatement (pagedbatch/sampling.py:12-13)
applied to the kernel's own bf16 logits.

Bars: every logit within one bf16 ulp of the exact dot product plus the worst-case fp32
accumulation error (hidden_dim * 2^-24 * sum |h_k w_k|; the kernel rounds an fp32 sum to
bf16, nearest even), and equal to the correctly rounded value for all but 1 % of them; tokens bit-exact against the argmax of the returned logits, and equal
to the exact argmax wherever the exact top two values are more than two ulps apart."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from pagedbatch_amd import _lib
from pagedbatch_amd.lm_head import lm_head_argmax

pytestmark = pytest.mark.gpu


def bf16_bits(x: torch.Tensor) -> np.ndarray:
    return x.view(torch.int16).numpy().view(np.uint16)


def rne_bf16(x64: np.ndarray) -> np.ndarray:
    """float64 -> bf16 value (as float64): round to fp32 first is not what the kernel
    does, so round the exact value straight to 8 significant bits, ties to even."""
    x = np.asarray(x64, dtype=np.float64)
    m, e = np.frexp(x)                   # x = m * 2^e, 0.5 <= |m| < 1
    q = np.round(m * 256.0) / 256.0      # numpy rounds half to even
    return np.ldexp(q, e)


def ulp_bf16(x64: np.ndarray) -> np.ndarray:
    _, e = np.frexp(np.abs(x64))
    return np.ldexp(1.0, e - 8)


def check(dev, rows, hdim, vocab, seed, scale=1.0, plant=None):
    print(f"[case] lm_head rows={rows} hidden={hdim} vocab={vocab} seed={seed}", flush=True)
    g = torch.Generator().manual_seed(seed)
    hidden = (torch.randn(rows, hdim, generator=g) * scale).to(torch.bfloat16)
    weight = (torch.randn(vocab, hdim, generator=g) * 0.05).to(torch.bfloat16)
    if plant is not None:
        plant(hidden, weight)
    logits, tokens = lm_head_argmax(hidden.to(dev), weight.to(dev))
    _, tokens2 = lm_head_argmax(hidden.to(dev), weight.to(dev), want_logits=False)
    out = logits.cpu().float().numpy().astype(np.float64)
    tok = tokens.cpu().numpy()
    np.testing.assert_array_equal(tok, tokens2.cpu().numpy())
    h64, w64 = hidden.double().numpy(), weight.double().numpy()
    ref = h64 @ w64.T
    # the fp32 accumulation's worst-case error, hidden_dim * 2^-24 * sum |h_k w_k|, on top
    # of one bf16 ulp for the final rounding
    gamma = (np.abs(h64) @ np.abs(w64).T) * hdim * 2.0 ** -24
    fin = np.isfinite(ref)
    err = np.abs(out - ref)
    bar = ulp_bf16(ref) + gamma
    assert (err[fin] <= bar[fin]).all(), f"max err / bar {np.max(err[fin] / bar[fin]):.3f}"
    exact = out[fin] == rne_bf16(ref[fin])
    assert exact.mean() > 0.99, f"only {exact.mean():.4f} of the logits are the correctly rounded value"
    bits = bf16_bits(logits.cpu())
    for b in range(rows):
        row = oracle.bf16_bits_to_f32(bits[b])
        assert tok[b] == oracle.greedy_token(row), f"row {b}: token {tok[b]} != argmax of the returned logits"
        top2 = np.sort(ref[b])[-2:] if vocab > 1 else None
        if top2 is not None and np.all(np.isfinite(top2)) and top2[1] - top2[0] > 2 * ulp_bf16(top2[1]):
            assert tok[b] == int(np.argmax(ref[b])), f"row {b}: token {tok[b]} != exact argmax {np.argmax(ref[b])}"
    return logits, tok


@pytest.mark.parametrize("rows,hdim,vocab", [
    (64, 576, 49152),   # the smollm2-135m head at a 64-sequence decode step
    (1, 576, 49152),
    (7, 128, 1000),     # vocab not a multiple of the 64-column tile nor of 8
    (100, 576, 4099),   # two row blocks, the second partial
    (33, 64, 65),
    (130, 192, 2048),   # three row blocks
    (5, 256, 300),      # 4 chunks of 64: four in flight, a last group of four
    (9, 384, 777),      # 6 chunks: a last group of six
    (3, 448, 129),      # 7 chunks: a last group of seven
    (17, 960, 1500),    # 15 chunks: two groups, then seven
    (70, 1024, 640),    # the largest LDS-resident hidden block, two row blocks
    (8, 1088, 3000),    # 17 chunks: no equal slices of at most 1024, so the L2-fragment kernel
    (65, 2048, 700),    # two LDS-resident slices of 1024
    (33, 3072, 500),    # three slices of 1024
    (9, 1280, 999),     # two slices of 640 (ten chunks each: a last group of six)
])
def test_lm_head_matches_exact_dot_products(dev, rows, hdim, vocab):
    check(dev, rows, hdim, vocab, seed=rows * 7 + vocab)


def test_lm_head_ties_nan_and_negative_zero(dev):
    def plant(h, w):
        h[0] = 0.0625                    # row 0: columns 50 and 100 tie at the maximum
        w[50] = 1.0
        w[100] = 1.0
        h[1, 3] = float("nan")           # row 1: every logit NaN -> token 0 (first NaN)
        h[2] = 0.0                       # row 2: every logit +0 -> token 0
        w[7] = -w[7]
    logits, tok = check(dev, 5, 576, 3000, seed=3, plant=plant)
    assert tok[0] == 50
    assert tok[1] == 0 and torch.isnan(logits[1].float()).all()
    assert tok[2] == 0


def test_lm_head_rejects_bad_operands(dev):
    h = torch.zeros(4, 100, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(10, 100, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="multiple of 64"):
        lm_head_argmax(h, w)
    with pytest.raises(ValueError, match="bf16"):
        lm_head_argmax(torch.zeros(4, 64, device=dev), torch.zeros(10, 64, device=dev))
    lib = _lib.load()
    assert lib.pbs_lm_head_argmax(h.data_ptr(), 128, w.data_ptr(), 4, 128, 10, None, 1 << 20, 1 << 20, 16, None) \
        == _lib.ERR_WORKSPACE


def test_lm_head_back_to_back_calls(dev):
    """Calls of different sizes back to back share one workspace."""
    g = torch.Generator().manual_seed(8)
    w = (torch.randn(3000, 128, generator=g) * 0.05).to(torch.bfloat16)
    for rows in (40, 3, 70, 1):
        h = torch.randn(rows, 128, generator=g).to(torch.bfloat16)
        print(f"[case] lm_head back to back rows={rows}", flush=True)
        logits, tok = lm_head_argmax(h.to(dev), w.to(dev))
        bits = bf16_bits(logits.cpu())
        want = [oracle.greedy_token(oracle.bf16_bits_to_f32(bits[b])) for b in range(rows)]
        assert tok.cpu().tolist() == want


def test_engine_step_with_fused_head(dev):
    """The engine harness's fused-head path on the tiny model: greedy rows take the fused
    kernel's tokens, stochastic rows are sampled from its logits, and every request runs to
    its length limit with the stop check's reasons."""
    from pagedbatch_amd import engine_step as es

    shape = es.ModelShape.tiny()
    print("[case] engine step, tiny model, fused lm_head", flush=True)
    t, out = es.run(shape, num_seqs=8, prompt_len=16, output_len=6, block_size=4, device=dev, fused_head=True)
    assert all(len(o) == 6 for o in out)
    assert t.reasons[-1] == ["length"] * 8 and all(x is None for rs in t.reasons[:-1] for x in rs)
    assert all(0 <= tok < shape.vocab_size for o in out for tok in o)
    # against the unfused head (torch's bf16 matmul, then the sampler on every row): the
    # logits agree bit for bit but for a rare last-bit rounding, so the token streams agree
    _, ref = es.run(shape, num_seqs=8, prompt_len=16, output_len=6, block_size=4, device=dev)
    agree = sum(a == b for x, y in zip(out, ref) for a, b in zip(x, y)) / 48
    assert agree >= 0.9, agree
