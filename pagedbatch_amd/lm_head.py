"""The step before the sampler, fused with the greedy decision: ``logits = hidden @
weight.T`` (pagedbatch/model.py:283, the bf16 ``lm_head`` Linear over each sequence's
last hidden state) on the matrix cores, with every row's ``torch.argmax`` over the bf16
logits (pagedbatch/sampling.py:12-13) taken in the same kernel.

``lm_head_argmax`` returns the greedy token of every row and, unless ``want_logits`` is
False, the bf16 logits themselves for the rows that still need sampling. A step whose
rows are all greedy then never writes the logits nor reads them back.
"""

from __future__ import annotations

import threading

import numpy as np
import torch

from . import _lib
from .sampling import SamplerError

KC = 64  # the kernel's hidden-dimension chunk: hidden_dim must be a multiple of it

_ws: dict[int, torch.Tensor] = {}
_ws_lock = threading.Lock()


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    with _ws_lock:
        ws = _ws.get(idx)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
            _ws[idx] = ws
        return ws


def _check(hidden: torch.Tensor, weight: torch.Tensor) -> None:
    if hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("hidden and weight must be bf16 (the model dtype of the reference's lm_head)")
    if hidden.dim() != 2 or weight.dim() != 2:
        raise ValueError("hidden must be [rows, hidden_dim] and weight [vocab, hidden_dim]")
    if hidden.shape[1] != weight.shape[1]:
        raise ValueError(f"hidden_dim differs: hidden {hidden.shape[1]}, weight {weight.shape[1]}")
    if hidden.shape[1] % KC:
        raise ValueError(f"hidden_dim {hidden.shape[1]} is not a multiple of {KC}")
    if not weight.is_contiguous() or hidden.stride(1) != 1 or hidden.stride(0) % 8:
        raise ValueError("weight must be contiguous and hidden rows contiguous with a stride that is a multiple of 8")
    if not hidden.is_cuda or weight.device != hidden.device:
        raise ValueError("hidden and weight must live on the same ROCm device; there is no CPU path")
    if hidden.data_ptr() % 16 or weight.data_ptr() % 16:
        raise ValueError("hidden and weight must start on a 16-byte boundary")


def lm_head_argmax(hidden: torch.Tensor, weight: torch.Tensor, want_logits: bool = True):
    """hidden: bf16 [rows, hidden_dim]; weight: bf16 [vocab, hidden_dim] (nn.Linear's
    layout). Returns ``(logits, tokens)``: bf16 [rows, vocab] logits (None when
    ``want_logits`` is False) and an int32 device tensor of the rows' greedy tokens."""
    _check(hidden, weight)
    rows, hdim = hidden.shape
    vocab = weight.shape[0]
    dev = hidden.device
    tokens = torch.empty(rows, dtype=torch.int32, device=dev)
    logits = torch.empty((rows, vocab), dtype=torch.bfloat16, device=dev) if want_logits else None
    if rows == 0:
        return logits, tokens
    lib = _lib.load()
    nbytes = lib.pbs_lm_head_workspace_bytes(rows, vocab)
    ws = _workspace(dev, nbytes)
    rc = lib.pbs_lm_head_argmax(hidden.data_ptr(), hidden.stride(0), weight.data_ptr(), rows, hdim, vocab,
                                logits.data_ptr() if logits is not None else None, tokens.data_ptr(),
                                ws.data_ptr(), ws.numel(), torch.cuda.current_stream(dev).cuda_stream)
    if rc != _lib.OK:
        msg = _lib.last_error(lib)
        if rc == _lib.ERR_INVALID_ARGUMENT:
            raise ValueError(msg)
        raise SamplerError(f"pbs_lm_head_argmax failed ({rc}): {msg}")
    return logits, tokens


def greedy_tokens(hidden: torch.Tensor, weight: torch.Tensor) -> np.ndarray:
    """The greedy token of every row, with no logits written (an all-greedy step)."""
    _, tokens = lm_head_argmax(hidden, weight, want_logits=False)
    return tokens.cpu().numpy()
