"""Next-token sampling on the GPU: greedy, temperature, top-k and top-p.

``sample_token`` keeps the signature of pagedbatch/sampling.py:10 so the reference engine
can import it unchanged. ``sample`` is the batched form the engine's per-row loop
(pagedbatch/engine.py:133-139) can be hoisted into: one kernel launch and one
device-to-host copy per step instead of one sync per row.

The draw consumes one uniform per stochastic row, taken from that row's generator with
``torch.rand`` in row order (greedy rows consume nothing, as in the reference), and picks
the token by inverse CDF over the kept tokens in the order pagedbatch's top-p sort uses
(probability descending, ties by ascending index). That is the same categorical
distribution pagedbatch's ``torch.multinomial`` samples from; the random stream it
consumes differs (one number per row instead of ``vocab``).
"""

from __future__ import annotations

import threading
from collections.abc import Sequence
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib

_TORCH_DTYPE = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16}

# torch.multinomial's message for an invalid distribution (what the reference raises)
_BAD_PROBS = "probability tensor contains either `inf`, `nan` or element < 0"


class SamplerError(RuntimeError):
    """The C ABI rejected a call."""


@dataclass
class DebugOutput:
    tokens: np.ndarray  # int32 [rows]
    status: np.ndarray  # int32 [rows]
    info: np.ndarray  # ROW_INFO_DTYPE [rows]
    probs: torch.Tensor | None  # float32 [rows, vocab] on the device
    kept: torch.Tensor | None  # uint8 [rows, vocab] on the device


class _Buffers:
    """Per-device staging: pinned host + device copies of the packed per-row arrays."""

    def __init__(self, device: torch.device):
        self.device = device
        self.cap = 0
        self.lock = threading.Lock()

    def ensure(self, n: int) -> None:
        if n <= self.cap:
            return
        cap = max(64, 1 << (n - 1).bit_length())
        # [temperature f32 | top_k i32 | top_p f32 | uniform f32 | row_map i32] x cap
        self.h_in = torch.empty(5 * cap, dtype=torch.int32, pin_memory=True)
        self.d_in = torch.empty(5 * cap, dtype=torch.int32, device=self.device)
        # [token i32 | status i32] x cap
        self.h_out = torch.empty(2 * cap, dtype=torch.int32, pin_memory=True)
        self.d_out = torch.empty(2 * cap, dtype=torch.int32, device=self.device)
        self.cap = cap


_buffers: dict[int, _Buffers] = {}
_buffers_lock = threading.Lock()


def _buffers_for(device: torch.device) -> _Buffers:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    with _buffers_lock:
        b = _buffers.get(idx)
        if b is None:
            b = _buffers[idx] = _Buffers(torch.device("cuda", idx))
        return b


def _check_logits(logits: torch.Tensor) -> torch.Tensor:
    if logits.dim() != 2:
        raise ValueError(f"logits must be [rows, vocab], got shape {tuple(logits.shape)}")
    if logits.dtype not in _TORCH_DTYPE:
        raise TypeError(f"logits dtype {logits.dtype} not supported (float32, float16, bfloat16)")
    if not logits.is_cuda:
        raise ValueError("logits must live on a ROCm device; this sampler has no CPU path")
    if logits.shape[1] < 1:
        raise ValueError("empty vocabulary")
    if logits.stride(1) != 1 or logits.stride(0) < logits.shape[1]:
        logits = logits.contiguous()
    return logits


def _top_k_code(k: int, vocab: int) -> int:
    # pagedbatch applies top-k only when 0 < k < vocab (sampling.py:15)
    return int(k) if 0 < int(k) < vocab else 0


def _launch(logits, h: np.ndarray, n: int, row_map_given: bool, debug: bool, bufs: _Buffers):
    """Copy packed params (host int32 view ``h``) and call the C ABI. Returns device outputs."""
    lib = _lib.load()
    hin = bufs.h_in.numpy()
    cap = bufs.cap
    for i in range(5):
        hin[i * cap : i * cap + n] = h[i]
    bufs.d_in.copy_(bufs.h_in, non_blocking=True)
    base = bufs.d_in.data_ptr()
    ptr = [base + 4 * i * cap for i in range(5)]
    out_tok = bufs.d_out.data_ptr()
    out_st = out_tok + 4 * cap
    stream = torch.cuda.current_stream(logits.device).cuda_stream
    args = [
        logits.data_ptr(),
        _TORCH_DTYPE[logits.dtype],
        logits.shape[0],
        n,
        logits.shape[1],
        logits.stride(0),
        ptr[4] if row_map_given else None,
        ptr[0],
        ptr[1],
        ptr[2],
        ptr[3],
        out_tok,
        out_st,
    ]
    probs = kept = info = None
    if debug:
        V = logits.shape[1]
        probs = torch.empty((n, V), dtype=torch.float32, device=logits.device)
        kept = torch.empty((n, V), dtype=torch.uint8, device=logits.device)
        info = torch.empty(n * _lib.ROW_INFO_DTYPE.itemsize, dtype=torch.uint8, device=logits.device)
        rc = lib.pbs_sample_debug(*args, probs.data_ptr(), kept.data_ptr(), info.data_ptr(), None, 0, stream)
    else:
        rc = lib.pbs_sample(*args, None, 0, stream)
    if rc != _lib.OK:
        msg = _lib.last_error(lib)
        if rc == _lib.ERR_INVALID_ARGUMENT:
            raise ValueError(msg)
        if rc == _lib.ERR_UNSUPPORTED_DTYPE:
            raise TypeError(msg)
        raise SamplerError(f"pbs_sample failed ({rc}): {msg}")
    bufs.h_out.copy_(bufs.d_out, non_blocking=True)
    torch.cuda.current_stream(logits.device).synchronize()
    hout = bufs.h_out.numpy()
    tokens = hout[:n].copy()
    status = hout[cap : cap + n].copy()
    return tokens, status, probs, kept, info


def _pack(n, temperature, top_k, top_p, uniform, row_map, vocab) -> np.ndarray:
    h = np.zeros((5, n), dtype=np.int32)
    h[0] = np.asarray(temperature, dtype=np.float32).view(np.int32)
    h[1] = np.asarray([_top_k_code(k, vocab) for k in top_k], dtype=np.int32)
    h[2] = np.asarray(top_p, dtype=np.float32).view(np.int32)
    h[3] = np.asarray(uniform, dtype=np.float32).view(np.int32)
    if row_map is not None:
        h[4] = np.asarray(row_map, dtype=np.int32)
    return h


def _raise_for_status(status: np.ndarray) -> None:
    bad = np.flatnonzero(status != _lib.ROW_OK)
    if bad.size == 0:
        return
    code = int(status[bad[0]])
    if code == _lib.ROW_BAD_PARAM:
        raise ValueError(f"invalid sampling parameters or row index for row {int(bad[0])}")
    raise RuntimeError(_BAD_PROBS)


def draw_uniforms(params: Sequence, generators: Sequence[torch.Generator]) -> list[float]:
    """One ``torch.rand`` draw per stochastic row, in row order; greedy rows draw nothing.

    Consecutive stochastic rows that share a generator (the engine's shared generator for
    unseeded requests, engine.py:58) take their draws from one ``torch.rand(n)`` call: torch
    fills it with the same numbers, in the same order, as n scalar draws, and leaves the
    generator in the same state.
    """
    out = [0.0] * len(params)
    i, n = 0, len(params)
    while i < n:
        if params[i].temperature == 0:
            i += 1
            continue
        g = generators[i]
        j = i + 1
        idx = [i]
        # extend the run over greedy rows (which draw nothing) while the generator repeats
        while j < n and (params[j].temperature == 0 or generators[j] is g):
            if params[j].temperature != 0:
                idx.append(j)
            j += 1
        vals = torch.rand(len(idx), generator=g, device=g.device).tolist()
        for k, v in zip(idx, vals):
            out[k] = float(v)
        i = j
    return out


def sample(logits: torch.Tensor, params: Sequence, generators: Sequence[torch.Generator],
           rows: Sequence[int] | None = None) -> list[int]:
    """Sample one token for each of ``rows`` (default: every row) of ``logits`` [B, vocab].

    ``params[i]`` and ``generators[i]`` belong to the i-th sampled row (the reference's
    ``seq.sampling`` and ``state.generator``, engine.py:138-139). Row order is the order
    uniforms are drawn in, matching the reference's per-row loop over one shared engine
    generator.
    """
    logits = _check_logits(logits)
    n = len(rows) if rows is not None else logits.shape[0]
    if len(params) != n or len(generators) != n:
        raise ValueError(f"need {n} params and generators, got {len(params)} and {len(generators)}")
    if n == 0:
        return []
    for sp in params:
        if sp.temperature < 0 or not 0 < sp.top_p <= 1 or sp.top_k < 0:
            raise ValueError("invalid SamplingParams")
    uniforms = draw_uniforms(params, generators)
    V = logits.shape[1]
    h = _pack(n, [sp.temperature for sp in params], [sp.top_k for sp in params], [sp.top_p for sp in params],
              uniforms, rows, V)
    bufs = _buffers_for(logits.device)
    with bufs.lock:
        bufs.ensure(n)
        tokens, status, _, _, _ = _launch(logits, h, n, rows is not None, False, bufs)
    _raise_for_status(status)
    return [int(t) for t in tokens]


def sample_token(logits: torch.Tensor, params, generator: torch.Generator) -> int:
    """Pick one token from a ``[vocab]`` logits row (pagedbatch/sampling.py:10)."""
    if logits.dim() != 1:
        raise ValueError(f"sample_token takes a [vocab] row, got shape {tuple(logits.shape)}")
    return sample(logits.unsqueeze(0), [params], [generator])[0]


def sample_arrays(logits: torch.Tensor, temperature, top_k, top_p, uniform, row_map=None,
                  debug: bool = False, check: bool = False):
    """Array-level entry: explicit per-row parameters and uniforms (tests, benchmarks).

    Returns ``(tokens, status)`` as int32 numpy arrays, or a ``DebugOutput`` with the
    final probabilities, the kept mask and per-row diagnostics when ``debug`` is set.
    """
    logits = _check_logits(logits)
    n = len(temperature)
    if n == 0:
        return (np.zeros(0, np.int32), np.zeros(0, np.int32))
    h = _pack(n, temperature, top_k, top_p, uniform, row_map, logits.shape[1])
    bufs = _buffers_for(logits.device)
    with bufs.lock:
        bufs.ensure(n)
        tokens, status, probs, kept, info = _launch(logits, h, n, row_map is not None, debug, bufs)
    if check:
        _raise_for_status(status)
    if not debug:
        return tokens, status
    info_np = np.frombuffer(info.cpu().numpy().tobytes(), dtype=_lib.ROW_INFO_DTYPE).copy()
    return DebugOutput(tokens=tokens, status=status, info=info_np, probs=probs, kept=kept)
