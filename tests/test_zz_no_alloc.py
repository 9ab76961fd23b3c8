"""pbs_lm_head_argmax_noalloc (the allocation-free variant of pbs_lm_head_argmax, which
runs on the library's own per-GPU scratch array) against pbs_lm_head_argmax with a
caller workspace, through the C ABI: the same logits bit for bit and the same tokens, on
two calls in a row (the second smaller, so it runs on what the first left in the scratch),
and sizes past the scratch rejected before any launch."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from pagedbatch_amd import _lib

pytestmark = pytest.mark.gpu


def _call(lib, hidden, weight, noalloc: bool):
    rows, hdim = hidden.shape
    vocab = weight.shape[0]
    logits = torch.full((rows, vocab), 7, dtype=torch.int16, device=hidden.device)
    tokens = torch.full((rows,), -5, dtype=torch.int32, device=hidden.device)
    stream = torch.cuda.current_stream(hidden.device).cuda_stream
    if noalloc:
        rc = lib.pbs_lm_head_argmax_noalloc(hidden.data_ptr(), hidden.stride(0), weight.data_ptr(), rows, hdim,
                                            vocab, logits.data_ptr(), tokens.data_ptr(), stream)
    else:
        nbytes = lib.pbs_lm_head_workspace_bytes(rows, vocab)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=hidden.device)
        rc = lib.pbs_lm_head_argmax(hidden.data_ptr(), hidden.stride(0), weight.data_ptr(), rows, hdim, vocab,
                                    logits.data_ptr(), tokens.data_ptr(), ws.data_ptr(), nbytes, stream)
    assert rc == _lib.OK, _lib.last_error(lib)
    torch.cuda.synchronize(hidden.device)
    return logits.cpu().numpy(), tokens.cpu().numpy()


def test_noalloc_matches_workspace_entry(dev):
    lib = _lib.load()
    g = torch.Generator().manual_seed(12)
    for rows, hdim, vocab in ((100, 576, 20000), (9, 576, 3001)):
        print(f"[case] lm_head no-alloc rows={rows} hidden={hdim} vocab={vocab}", flush=True)
        hidden = torch.randn(rows, hdim, generator=g).to(torch.bfloat16).to(dev)
        weight = (torch.randn(vocab, hdim, generator=g) * 0.05).to(torch.bfloat16).to(dev)
        ref_logits, ref_tok = _call(lib, hidden.view(torch.int16), weight.view(torch.int16), noalloc=False)
        got_logits, got_tok = _call(lib, hidden.view(torch.int16), weight.view(torch.int16), noalloc=True)
        np.testing.assert_array_equal(got_logits, ref_logits)
        np.testing.assert_array_equal(got_tok, ref_tok)
        assert ((0 <= got_tok) & (got_tok < vocab)).all()


def test_noalloc_rejects_sizes_past_its_scratch(dev):
    lib = _lib.load()
    # 1025 rows of a 32768 vocab: 1025 * 512 tiles > 2^19 keys; checked before any launch
    rc = lib.pbs_lm_head_argmax_noalloc(1 << 20, 64, 1 << 20, 1025, 64, 32768, None, 1 << 20, None)
    assert rc == _lib.ERR_WORKSPACE
    assert "scratch" in _lib.last_error(lib)
    assert lib.pbs_lm_head_argmax_noalloc(1 << 20, 64, 1 << 20, 0, 64, 32768, None, 1 << 20, None) == _lib.OK
