"""Kernel-vs-oracle parity on the GPU, through the C ABI (pagedbatch_amd.sampling.sample_arrays).

Every case prints its name, dtype and shape before touching the GPU, so a failure names
itself. Bars (oracle/compare.py): greedy tokens bit-exact; stochastic tokens identical
unless u lies within 1e-6 of a CDF boundary, and then one whose CDF interval holds the
draw point up to 2e-6; kept sets identical unless top_p lies within 1e-6 of a cumulative
boundary, and then a prefix of the oracle's sampling order differing only at positions
whose exclusive mass is within 2e-6 of top_p; probabilities within 1e-5 absolute. Each
case also asserts how many of its stochastic rows met the exact bar.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from oracle.compare import compare_rows
from pagedbatch_amd import workloads
from pagedbatch_amd.sampling import sample_arrays

pytestmark = pytest.mark.gpu

DT_NAME = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}


def raw_numpy(x: torch.Tensor) -> np.ndarray:
    if x.dtype == torch.bfloat16:
        return x.view(torch.int16).numpy().view(np.uint16)
    return x.numpy()


def run_case(dev, name, logits_cpu, T, K, P, U, row_map=None, want_probs=True, info_only=False, min_checked=0.5):
    """One call through the C ABI against the oracle. Rows inside the 1e-6 bands are held
    to the band bar (oracle/compare.py); at least ``min_checked`` of the stochastic rows
    must meet the exact bar (token and kept set equal to the oracle's)."""
    print(f"[case] {name} dtype={logits_cpu.dtype} shape={tuple(logits_cpu.shape)} rows_out={len(T)}", flush=True)
    x = logits_cpu.to(dev)
    out = sample_arrays(x, T, K, P, U, row_map=row_map, debug=True)
    refs = oracle.sample_batch(raw_numpy(logits_cpu), DT_NAME[logits_cpu.dtype], T, K, P, U, row_map=row_map,
                               want_probs=want_probs or not info_only)
    greedy = [t == 0 for t in T]
    probs = None if info_only or not want_probs else out.probs.cpu().numpy()
    kept = None if info_only else out.kept.cpu().numpy()
    rep = compare_rows(out.tokens, out.status, refs, greedy, probs=probs, kept=kept, info=out.info, top_p=P,
                       uniform=U)
    stoch = [b for b, r in enumerate(refs) if not greedy[b] and r.status == oracle.ROW_OK]
    exact = rep.checked_tokens - sum(1 for b, r in enumerate(refs) if greedy[b] and r.status == oracle.ROW_OK)
    print(f"[case] {name}: {rep.summary()} exactly checked stochastic rows {exact}/{len(stoch)}", flush=True)
    assert rep.ok(), rep.summary()
    assert exact >= min_checked * len(stoch), f"only {exact} of {len(stoch)} stochastic rows met the exact bar"
    # the plain call (no diagnostics: the selecting lane writes the token itself) must give
    # the same tokens and statuses as the diagnostic call checked above
    tok, st = sample_arrays(x, T, K, P, U, row_map=row_map)
    np.testing.assert_array_equal(np.asarray(tok), np.asarray(out.tokens))
    np.testing.assert_array_equal(np.asarray(st), np.asarray(out.status))
    return out, refs, rep


def test_steps8_smollm_mixed(dev):
    w = workloads.steps8_smollm_mixed()
    run_case(dev, w.name, w.logits, w.temperature, w.top_k, w.top_p, w.uniform)


def test_greedy512_quantized_bit_exact(dev):
    w = workloads.greedy512_quantized()
    print(f"[case] {w.name}", flush=True)
    out = sample_arrays(w.logits.to(dev), w.temperature, w.top_k, w.top_p, w.uniform)
    ref = np.argmax(w.logits.numpy(), axis=1)
    assert (out[1] == 0).all()
    np.testing.assert_array_equal(out[0], ref)
    # the 1/4 grid puts a tie at the maximum in a good share of rows
    x = w.logits.numpy()
    assert ((x == x.max(axis=1, keepdims=True)).sum(axis=1) > 1).mean() > 0.25
    # and rows with the maximum planted at several random positions, first copy not at 0
    g = torch.Generator().manual_seed(11)
    y = w.logits[:64].clone()
    for r in range(64):
        pos = torch.randperm(y.shape[1], generator=g)[: 2 + r % 7]
        y[r, pos] = 9.0
    out = sample_arrays(y.to(dev), [0.0] * 64, [0] * 64, [1.0] * 64, [0.0] * 64)
    np.testing.assert_array_equal(out[0], np.argmax(y.numpy(), axis=1))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("vocab", [1, 7, 64, 1000, 4096, 32003, 65536])
def test_random_rows(dev, dtype, vocab):
    g = torch.Generator().manual_seed(vocab * 7 + int(DT_NAME[dtype] == "float16"))
    rows = 24
    x = torch.randn(rows, vocab, generator=g) * 1.5
    x[rows // 2:] = torch.round(x[rows // 2:] * 4) / 4  # heavy ties in half the rows
    logits = x.to(dtype)
    T = [0.0, 0.7, 1.0, 1.3] * (rows // 4)
    K = [0, 1, 2, 5, 50, vocab - 1, vocab, 0] * (rows // 8)
    P = [1.0, 0.5, 0.9, 0.95, 1e-6, 0.999] * (rows // 6)
    U = [float(v) for v in torch.rand(rows, generator=g)]
    U[3] = 0.0
    run_case(dev, f"random_{DT_NAME[dtype]}_{vocab}", logits, T, K, P, U)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_reference_known_answers(dev, dtype):
    """tests/test_engine.py:86-93 of the reference, through the kernel."""
    logits = torch.tensor([[0.1, 3.0, 0.2, 2.9]]).to(dtype)
    x = logits.to(dev)
    g = torch.Generator().manual_seed(0)
    for T, K, P in [(0.0, 0, 1.0), (1.0, 1, 1.0), (1.0, 0, 1e-6)]:
        u = float(torch.rand((), generator=g))
        tok, st = sample_arrays(x, [T], [K], [P], [u])
        assert st[0] == 0 and tok[0] == 1
    picks = set()
    for _ in range(50):
        u = float(torch.rand((), generator=g))
        tok, st = sample_arrays(x, [1.0], [2], [1.0], [u])
        picks.add(int(tok[0]))
    assert picks <= {1, 3} and len(picks) == 2


def test_edge_values(dev):
    nan, inf = float("nan"), float("inf")
    rows = [
        [1.0, nan, 3.0, nan],          # greedy -> first NaN; stochastic -> NaN status
        [-inf, -inf, -inf, -inf],      # greedy -> 0; stochastic -> nonfinite
        [-0.0, 0.0, -0.0, 0.0],        # -0 and +0 tie
        [inf, 1.0, 2.0, 3.0],          # greedy -> 0; stochastic -> nonfinite
        [-inf, 2.0, -inf, 2.0],        # -inf entries get zero mass
        [3e38, 3.3e38, -3e38, 0.0],    # overflow after /T for small T
    ]
    base = torch.tensor(rows, dtype=torch.float32)
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        logits = base.to(dtype)
        n = logits.shape[0]
        for T in (0.0, 1.0, 0.5):
            run_case(dev, f"edge_{DT_NAME[dtype]}_T{T}", logits, [T] * n, [0] * n, [1.0] * n, [0.3] * n)
        run_case(dev, f"edge_{DT_NAME[dtype]}_topk", logits, [1.0] * n, [2] * n, [0.7] * n, [0.6] * n)


def test_row_map_and_unaligned(dev):
    g = torch.Generator().manual_seed(5)
    big = torch.randn(6, 1003, generator=g)
    # a strided view with an odd row stride exercises the element-load path
    view = big[:, :1000]
    rm = [5, 0, 0, 3, 2, 5, 1]
    T = [1.0, 0.0, 0.8, 1.2, 1.0, 0.5, 1.0]
    K = [0, 0, 10, 0, 3, 0, 100]
    P = [0.9, 1.0, 1.0, 0.5, 1.0, 0.99, 0.8]
    U = [0.1, 0.0, 0.5, 0.9, 0.2, 0.7, 0.33]
    x = big.to(dev)[:, :1000]
    assert x.stride(0) == 1003
    out = sample_arrays(x, T, K, P, U, row_map=rm, debug=True)
    refs = oracle.sample_batch(view.contiguous().numpy(), "float32", T, K, P, U, row_map=rm, want_probs=True)
    rep = compare_rows(out.tokens, out.status, refs, [t == 0 for t in T], probs=out.probs.cpu().numpy(),
                       kept=out.kept.cpu().numpy(), info=out.info)
    assert rep.ok(), rep.summary()
    bad = sample_arrays(x, [1.0], [0], [1.0], [0.5], row_map=[6])
    assert bad[1][0] == oracle.ROW_BAD_PARAM


def test_mixed256_llama3_bf16(dev):
    w = workloads.mixed256_llama3_bf16()
    run_case(dev, w.name, w.logits, w.temperature, w.top_k, w.top_p, w.uniform, min_checked=0.85)


def test_nucleus1024_qwen_fp32_128_rows(dev):
    """The full 1024 x 151936 fp32 workload in one plain launch, and 128 of its rows (every
    eighth) through the diagnostic call against the oracle. The rows are flat (N(0, 0.5^2)):
    each token holds about 7e-6 of the mass, so the 1e-6 bands take in many rows; those are
    held to the band bar and a quarter of the rows must still meet the exact bar."""
    w = workloads.nucleus1024_qwen_fp32()
    print(f"[case] {w.name} full launch", flush=True)
    x = w.logits.to(dev)
    tok_all, st_all = sample_arrays(x, w.temperature, w.top_k, w.top_p, w.uniform)
    assert (np.asarray(st_all) == 0).all()
    rm = list(range(0, 1024, 8))
    T, K, P, U = ([v[r] for r in rm] for v in (w.temperature, w.top_k, w.top_p, w.uniform))
    out, _, _ = run_case(dev, w.name + "_128", w.logits, T, K, P, U, row_map=rm, want_probs=False, min_checked=0.25)
    np.testing.assert_array_equal(np.asarray(tok_all)[rm], np.asarray(out.tokens))


def test_bad_parameters_get_the_row_status(dev):
    """Every parameter the kernel validates (include/pbsample.h, PBS_ROW_BAD_PARAM), one
    per row, next to good rows that must still sample: a negative or NaN or infinite
    temperature, top_p of 0, above 1 or NaN, a negative top_k, a uniform of 1, below 0 or
    NaN, and a row_map entry past the logits."""
    g = torch.Generator().manual_seed(31)
    logits = torch.randn(4, 4096, generator=g).to(torch.bfloat16)
    nan, inf = float("nan"), float("inf")
    T = [-0.5, nan, inf, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 0.8, 0.0]
    K = [0, 0, 0, 0, 0, 0, -3, 0, 0, 0, 0, 20, 0]
    P = [1.0, 1.0, 1.0, 0.0, 1.5, nan, 1.0, 1.0, 1.0, 1.0, 1.0, 0.9, 1.0]
    U = [0.5, 0.5, 0.5, 0.5, 0.5, 0.5, 0.5, 1.0, -0.1, nan, 0.5, 0.4, 0.0]
    rm = [0, 1, 2, 3, 0, 1, 2, 3, 0, 1, 4, 2, 3]
    print("[case] bad parameters", flush=True)
    out = sample_arrays(logits.to(dev), T, K, P, U, row_map=rm, debug=True)
    refs = oracle.sample_batch(raw_numpy(logits), "bfloat16", T, K, P, U, row_map=rm)
    want = [oracle.ROW_BAD_PARAM] * 11 + [oracle.ROW_OK, oracle.ROW_OK]
    assert [r.status for r in refs] == want
    assert list(out.status) == want
    rep = compare_rows(out.tokens, out.status, refs, [t == 0 for t in T], info=out.info, top_p=P, uniform=U)
    assert rep.ok(), rep.summary()
    # the Python surface turns them into the reference's exceptions
    from pagedbatch_amd import sample

    gens = [torch.Generator().manual_seed(1)]
    with pytest.raises(RuntimeError, match="probability tensor"):
        sample(logits.to(dev)[:1], [_Params(nan, 0, 1.0)], gens)
    with pytest.raises(ValueError, match="finite"):
        sample(logits.to(dev)[:1], [_Params(inf, 0, 1.0)], gens)


class _Params:
    """A parameter object the reference's SamplingParams checks would let through."""

    def __init__(self, temperature, top_k, top_p):
        self.temperature, self.top_k, self.top_p = temperature, top_k, top_p


def test_counter_wrap_takes_general_path(dev):
    """A 16-bit value occurring more than 65535 times wraps its u16 histogram counter; such
    rows must go through the general (bisection) path and still match the oracle."""
    g = torch.Generator().manual_seed(21)
    V = 131072
    x = torch.zeros(4, V)
    x[:, :3000] = torch.randn(4, 3000, generator=g)  # everything else is exactly +0
    x[1, 5000:] = -0.0                                 # and -0, which ties with +0
    logits = x.to(torch.bfloat16)
    T = [1.0, 0.7, 1.3, 0.0]
    K = [0, 50, 0, 0]
    P = [0.9, 1.0, 0.5, 1.0]
    U = [0.99, 0.3, 0.7, 0.0]
    run_case(dev, "counter_wrap_bf16", logits, T, K, P, U, info_only=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_zero_ties_in_a_partial_chunk(dev, dtype):
    """Register rows whose length leaves the last chunk partly past the row end (those
    vectors load as zeros) while the draw lands in a tie group of +0: the selection must
    count only the real zeros. Also a +0 / -0 tie and a row whose tie group excludes 0."""
    g = torch.Generator().manual_seed(25)
    V = 5000  # 625 16-byte vectors: the second chunk of 512 lanes is 113 lanes full
    x = torch.zeros(6, V)
    x[:, ::50] = -torch.rand(6, 100, generator=g) - 0.5  # a few negatives; the maximum is 0
    x[2, 1::3] = -0.0                                     # -0 ties with +0
    x[3] = torch.randn(V, generator=g)                    # no zero ties at the draw
    x[4, V - 7:] = 0.25                                   # ties at the top in the last vector
    x[5, :] = 0.0                                         # one tie group of V
    logits = x.to(dtype)
    T = [1.0, 0.7, 1.0, 1.1, 1.0, 1.0]
    K = [0, 0, 0, 0, 3, 0]
    P = [1.0, 0.9, 1.0, 0.95, 1.0, 1.0]
    U = [0.7, 0.999, 0.5, 0.3, 0.9, 0.9999]
    run_case(dev, f"zero_ties_partial_{DT_NAME[dtype]}", logits, T, K, P, U)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_values_colliding_after_division(dev, dtype):
    """A huge temperature sends many distinct 16-bit values to the same (subnormal or zero)
    fp32 quotient: ties that span several histogram bins, including -0 and +0."""
    g = torch.Generator().manual_seed(22)
    V = 4096
    x = torch.randn(6, V, generator=g) * 1e-3
    x[3:, ::7] = 0.0
    x[4:, 1::7] = -0.0
    logits = x.to(dtype)
    T = [3e36, 1e37, 3e38, 3e36, 1e37, 1e30]
    K = [0, 10, 0, 100, 0, 5]
    P = [0.5, 1.0, 0.9, 0.3, 1.0, 0.6]
    U = [0.1, 0.5, 0.9, 0.25, 0.75, 0.4]
    # (huge temperatures leave few distinct weights: most draws sit on a boundary between
    # equal-mass tokens, which the band bar covers)
    run_case(dev, f"collide_{DT_NAME[dtype]}", logits, T, K, P, U, min_checked=0.15)


def test_fp32_window_paths(dev):
    """fp32 rows through each way the window path resolves: top-k within the top 4096 (one
    list), large top-k with and without top-p (the k-th element's bin gathered with the
    cutoff and draw windows), temperature 1 and not 1 (the division), and tie-heavy rows
    whose windows hold more elements than the LDS list (the general path)."""
    g = torch.Generator().manual_seed(24)
    V = 131072
    x = torch.randn(8, V, generator=g) * 0.5
    x[6:] = torch.round(x[6:] * 4) / 4  # few distinct values, tens of thousands of elements each
    T = [1.0, 0.8, 1.0, 1.3, 0.6, 1.0, 1.0, 0.9]
    K = [20, 3000, 60000, 90000, 0, 0, 0, 500]
    P = [0.9, 0.95, 0.8, 1.0, 0.95, 1.0, 0.9, 0.97]
    U = [float(v) for v in torch.rand(8, generator=g)]
    run_case(dev, "fp32_window_paths", x, T, K, P, U, want_probs=False, info_only=True)


@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, 128256), (torch.float16, 128256), (torch.bfloat16, 200000)])
def test_rows_masked_with_neg_inf(dev, dtype, V):
    """Rows whose vocabulary is masked with -inf (more than 65535 entries, so -inf's u16
    counter wraps and the rows take the general path): greedy rows, top-k inside and past
    the finite entries (the k-th is then -inf and everything is kept), top-p,
    temperatures, and a row where 70000 zeros wrap a finite counter too. Registers
    (V = 128256) and the re-read row (200000)."""
    g = torch.Generator().manual_seed(41)
    rows = 8
    nfin = [1000, 500, 3000, 800, 20, 2000, 1500, 600]
    x = torch.full((rows, V), float("-inf"))
    for r in range(rows):
        keep = torch.randperm(V, generator=g)[: nfin[r]]
        x[r, keep] = torch.randn(nfin[r], generator=g) * 2.0
    zeros = torch.randperm(V, generator=g)[:70000]
    x[7, zeros] = 0.0
    T = [0.0, 1.0, 0.8, 1.0, 1.0, 0.6, 1.2, 1.0]
    K = [0, 0, 20, 5000, 50, 0, 100, 0]
    P = [1.0, 1.0, 0.9, 1.0, 0.95, 0.8, 1.0, 0.9]
    U = [float(v) for v in torch.rand(rows, generator=g)]
    run_case(dev, f"masked_{DT_NAME[dtype]}_{V}", x.to(dtype), T, K, P, U, want_probs=False)


@pytest.mark.parametrize("V", [49152, 151936])
def test_fp32_windows_crowded_into_one_lane(dev, V):
    """fp32 rows whose windows are dense (the largest values, which hold the top-k, the
    top-p cutoff and the draw, are one element in 40) with every element of one thread
    among them (element i belongs to thread (i // 4) % 512): that lane's list column
    overflows, so the gather runs again with ballots. Registers (V = 49152) and the
    re-read row (V = 151936)."""
    g = torch.Generator().manual_seed(31)
    x = torch.randn(4, V, generator=g) * 0.5
    t0 = 5
    idx = torch.tensor([4 * (t0 + 512 * k) + e for k in range((V // 4 + 511) // 512) for e in range(4)
                        if 4 * (t0 + 512 * k) + e < V])
    others = torch.tensor(sorted(set(torch.randperm(V, generator=g)[: V // 40].tolist()) - set(idx.tolist())))
    top = torch.cat([idx, others])
    x[:, top] = 8.0 + torch.randn(4, len(top), generator=g) * 0.01
    T = [1.0, 1.0, 0.7, 1.0]
    K = [64, 0, 0, 30]
    P = [1.0, 0.5, 0.9, 0.8]
    U = [float(v) for v in torch.rand(4, generator=g)]
    run_case(dev, f"fp32_crowded_lane_{V}", x, T, K, P, U, want_probs=V <= 49152, info_only=V > 49152)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_register_row_sizes(dev, dtype):
    """Vocab sizes that land on each register-row width (and just past the largest)."""
    g = torch.Generator().manual_seed(23)
    sizes = (2048, 4096, 8192, 16384, 24576, 32768, 49152, 65536, 151936) if dtype == torch.float32 else \
        (4096, 8192, 12288, 24576, 49152, 128256, 131072, 151936)
    for V in sizes:
        x = (torch.randn(8, V, generator=g) * 2.0).to(dtype)
        T = [0.0, 0.9, 1.0, 1.2] * 2
        K = [0, 40, 0, V // 3, 1, 0, 7, 0]
        P = [1.0, 0.9, 0.5, 1.0, 1.0, 0.99, 0.8, 1.0]
        U = [float(v) for v in torch.rand(8, generator=g)]
        run_case(dev, f"width_{DT_NAME[dtype]}_{V}", x, T, K, P, U, want_probs=V <= 49152,
                 info_only=V > 49152)
