"""The all-greedy entry point ``pbs_argmax`` on the GPU, through the C ABI, against the
oracle's ``greedy_token`` (torch.argmax, pagedbatch/sampling.py:12-13: the first NaN if
the row holds one, else the first maximum) and against ``pbs_sample`` with temperature 0
on every row. Integer results: bit-exact."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from pagedbatch_amd import _lib, workloads
from pagedbatch_amd.sampling import _TORCH_DTYPE, sample, sample_arrays

pytestmark = pytest.mark.gpu

DT = [torch.bfloat16, torch.float16, torch.float32]


def argmax(x: torch.Tensor, row_map=None, n_logit_rows=None):
    """One pbs_argmax call on the device view ``x`` (rows may be strided)."""
    lib = _lib.load()
    rows = len(row_map) if row_map is not None else x.shape[0]
    tok = torch.full((rows,), -7, dtype=torch.int32, device=x.device)
    st = torch.full((rows,), -7, dtype=torch.int32, device=x.device)
    rm = torch.tensor(row_map, dtype=torch.int32, device=x.device) if row_map is not None else None
    rc = lib.pbs_argmax(x.data_ptr(), _TORCH_DTYPE[x.dtype], x.shape[0] if n_logit_rows is None else n_logit_rows,
                        rows, x.shape[1], x.stride(0), rm.data_ptr() if rm is not None else None, tok.data_ptr(),
                        st.data_ptr(), torch.cuda.current_stream(x.device).cuda_stream)
    assert rc == _lib.OK, _lib.last_error(lib)
    return tok.cpu().numpy(), st.cpu().numpy()


def want(x_cpu: torch.Tensor) -> np.ndarray:
    x = x_cpu.float().numpy()
    return np.array([oracle.greedy_token(r) for r in x], dtype=np.int32)


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("vocab", [1, 7, 8, 63, 4096, 32003, 49152, 65537, 128256, 151936])
def test_argmax_random_rows(dev, dtype, vocab):
    print(f"[case] argmax {dtype} vocab={vocab}", flush=True)
    g = torch.Generator().manual_seed(vocab + 3)
    rows = 16
    x = torch.randn(rows, vocab, generator=g) * 2
    x[rows // 2:] = torch.round(x[rows // 2:] * 2) / 2  # ties at the maximum
    # the maximum planted at the last element, the first element, and at two positions
    x[0, -1] = 50.0
    x[1, 0] = 50.0
    if vocab > 2:
        x[2, vocab // 2] = x[2, vocab - 2] = 50.0
    xd = x.to(dtype)
    tok, st = argmax(xd.to(dev))
    assert (st == 0).all()
    np.testing.assert_array_equal(tok, want(xd))
    # the same tokens as the sampler's greedy rows
    out = sample_arrays(xd.to(dev), [0.0] * rows, [0] * rows, [1.0] * rows, [0.0] * rows, debug=True)
    np.testing.assert_array_equal(tok, out.tokens)


@pytest.mark.parametrize("dtype", DT)
def test_argmax_special_values(dev, dtype):
    nan, inf = float("nan"), float("inf")
    V = 5000
    x = torch.zeros(8, V)
    x[0, 4000] = nan
    x[0, 17] = nan                # first NaN wins over everything
    x[0, 3] = inf
    x[1] = -inf                   # every value -inf: index 0
    x[2, ::2] = -0.0              # -0 and +0 tie: index 0
    x[3, 2500:] = inf             # first +inf
    x[4] = -inf
    x[4, V - 1] = -1e30           # the only finite value, last
    x[5] = torch.arange(V, dtype=torch.float32) * -1.0
    x[6, V - 1] = nan             # NaN at the end
    x[7, 1:] = 1.0
    xd = x.to(dtype)
    print(f"[case] argmax special values {dtype}", flush=True)
    tok, st = argmax(xd.to(dev))
    assert (st == 0).all()
    np.testing.assert_array_equal(tok, want(xd))
    assert tok.tolist()[:4] == [17, 0, 0, 2500]
    # the same rows behind an odd row stride: the element-load path
    wide = torch.zeros(8, V + 1, dtype=dtype)
    wide[:, :V] = xd
    view = wide.to(dev)[:, :V]
    assert view.stride(0) == V + 1
    tok, st = argmax(view)
    assert (st == 0).all()
    np.testing.assert_array_equal(tok, want(xd))


def test_argmax_row_map_stride_and_bad_rows(dev):
    g = torch.Generator().manual_seed(9)
    big = torch.randn(6, 1003, generator=g)
    x = big.to(dev)[:, :1000]           # odd row stride: the element-load path
    assert x.stride(0) == 1003
    rm = [5, 0, 0, 6, 2, -1, 1]
    print("[case] argmax row map, stride 1003, bad entries", flush=True)
    tok, st = argmax(x, row_map=rm)
    ref = want(big[:, :1000].contiguous())
    for b, r in enumerate(rm):
        if 0 <= r < 6:
            assert st[b] == 0 and tok[b] == ref[r]
        else:
            assert st[b] == _lib.ROW_BAD_PARAM and tok[b] == 0
    # aligned rows through a row map reading every row twice
    y = torch.randn(4, 4096, generator=g).to(torch.bfloat16)
    tok, st = argmax(y.to(dev), row_map=[3, 2, 1, 0, 0, 1, 2, 3])
    np.testing.assert_array_equal(tok, want(y)[[3, 2, 1, 0, 0, 1, 2, 3]])


def test_greedy512_quantized_through_sample(dev):
    """The 512 x 49152 quantized workload (ties at the maximum in a good share of rows)
    through sample(): every row greedy, so the call goes to pbs_argmax."""
    w = workloads.greedy512_quantized()
    print(f"[case] {w.name} via sample()", flush=True)
    x = w.logits.to(dev)

    class P:
        temperature, top_k, top_p = 0.0, 0, 1.0

    gens = [torch.Generator().manual_seed(0)] * w.rows
    toks = sample(x, [P()] * w.rows, gens)
    np.testing.assert_array_equal(np.array(toks, dtype=np.int32), want(w.logits))
    tok, st = argmax(x)
    np.testing.assert_array_equal(tok, want(w.logits))


def test_argmax_many_rows_large_vocab(dev):
    """2048 bf16 rows of 128256 (more workgroups than the chip holds at once)."""
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(2048, 128256, generator=g, dtype=torch.float32) * 3).to(torch.bfloat16)
    print("[case] argmax 2048 x 128256 bf16", flush=True)
    tok, st = argmax(x.to(dev))
    assert (st == 0).all()
    np.testing.assert_array_equal(tok, want(x))
