"""Next-token sampling on the GPU: greedy, temperature, top-k and top-p.

``sample_token`` keeps the signature of pagedbatch/sampling.py:10 so the reference engine
can import it unchanged. ``sample`` is the batched form the engine's per-row loop
(pagedbatch/engine.py:133-139) can be hoisted into: one kernel launch and one
device-to-host copy per step instead of one sync per row. ``sample_and_finish`` also runs
the step's stop check (engine.py:173-182) on the device and brings the finish reasons back
in the same copy as the tokens.

The draw consumes one uniform per stochastic row, taken from that row's generator with
``torch.rand`` in row order (greedy rows consume nothing, as in the reference), and picks
the token by inverse CDF over the kept tokens in the order pagedbatch's top-p sort uses
(probability descending, ties by ascending index). That is the same categorical
distribution pagedbatch's ``torch.multinomial`` samples from; the random stream it
consumes differs (one number per row instead of ``vocab``).
"""

from __future__ import annotations

import threading
import time
from collections.abc import Sequence
from dataclasses import dataclass
from operator import attrgetter

import numpy as np
import torch

from . import _lib

_TORCH_DTYPE = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16}

# torch.multinomial's message for an invalid distribution (what the reference raises)
_BAD_PROBS = "probability tensor contains either `inf`, `nan` or element < 0"

_TEMPERATURE, _TOP_K, _TOP_P = attrgetter("temperature"), attrgetter("top_k"), attrgetter("top_p")


class SamplerError(RuntimeError):
    """The C ABI rejected a call."""


@dataclass
class DebugOutput:
    tokens: np.ndarray  # int32 [rows]
    status: np.ndarray  # int32 [rows]
    info: np.ndarray  # ROW_INFO_DTYPE [rows]
    probs: torch.Tensor | None  # float32 [rows, vocab] on the device
    kept: torch.Tensor | None  # uint8 [rows, vocab] on the device


# staging layout, in int32 words of one pinned host block and its device copy:
#   inputs   temperature f32 | top_k i32 | top_p f32 | uniform f32 | row_map i32   (cap each)
#   finish   stop_offsets [cap + 1] | num_output | max_tokens | num_tokens  (cap each)
#            | ignore_eos u8 [cap] (cap / 4 words) | stop_ids [stop_cap]
#   outputs  token i32 | status i32 | reason i32   (cap each, a block of their own)
_IN_T, _IN_K, _IN_P, _IN_U, _IN_MAP = range(5)


class _Buffers:
    """Per-device staging: pinned host + device copies of the packed per-row arrays."""

    def __init__(self, device: torch.device):
        self.device = device
        self.cap = 0
        self.stop_cap = 0
        self.lock = threading.Lock()

    def ensure(self, n: int, nstop: int = 0) -> None:
        if n <= self.cap and nstop <= self.stop_cap:
            return
        cap = max(64, 1 << (max(n, self.cap) - 1).bit_length())
        stop_cap = max(self.stop_cap, 64, 1 << max(0, nstop - 1).bit_length())
        self.fin = 5 * cap  # start of the finish block
        self.stop_ids = self.fin + (cap + 1) + 3 * cap + cap // 4
        words = self.stop_ids + stop_cap
        self.h_in = torch.empty(words, dtype=torch.int32, pin_memory=True)
        self.d_in = torch.empty(words, dtype=torch.int32, device=self.device)
        self.h_in_np = self.h_in.numpy()
        self.h_out = torch.empty(3 * cap, dtype=torch.int32, pin_memory=True)
        self.d_out = torch.empty(3 * cap, dtype=torch.int32, device=self.device)
        self.h_out_np = self.h_out.numpy()
        self.cap = cap
        self.stop_cap = stop_cap


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


def _top_k_codes(top_k, vocab: int) -> np.ndarray:
    """The kernel's top_k argument: pagedbatch applies top-k only when 0 < k < vocab
    (sampling.py:15), so k >= vocab becomes 0 (off); a negative k stays negative (-1) so
    that the kernel reports the row as a bad parameter instead of switching top-k off."""
    k = np.asarray(top_k, dtype=np.int64)
    return np.where(k < 0, -1, np.where(k < vocab, k, 0)).astype(np.int32)


def _pack(n, temperature, top_k, top_p, uniform, row_map, vocab) -> np.ndarray:
    """The five per-row parameter arrays as one int32 [5, n] block (the staging layout)."""
    h = np.zeros((5, n), dtype=np.int32)
    h[_IN_T] = np.asarray(temperature, dtype=np.float32).view(np.int32)
    h[_IN_K] = _top_k_codes(top_k, vocab)
    h[_IN_P] = np.asarray(top_p, dtype=np.float32).view(np.int32)
    h[_IN_U] = np.asarray(uniform, dtype=np.float32).view(np.int32)
    if row_map is not None:
        h[_IN_MAP] = np.asarray(row_map, dtype=np.int32)
    return h


def _all_greedy(h: np.ndarray) -> bool:
    """True when every row of a packed block is greedy with valid parameters: then
    ``pbs_argmax`` returns exactly what ``pbs_sample`` would (it checks only the row map)."""
    t = h[_IN_T].view(np.float32)
    p = h[_IN_P].view(np.float32)
    return bool((t == 0).all() and (h[_IN_K] >= 0).all() and ((p > 0) & (p <= 1)).all())


def _stage_params(bufs: _Buffers, h: np.ndarray, n: int) -> None:
    cap = bufs.cap
    for i in range(5):
        bufs.h_in_np[i * cap : i * cap + n] = h[i]


def _stage_finish(bufs: _Buffers, rules, n: int) -> int:
    """The stop rules of n rows into the finish block; returns the number of stop ids."""
    return _write_finish(bufs.h_in_np, bufs.fin, bufs.cap, bufs.stop_ids, rules, n)


def _write_finish(hin: np.ndarray, base: int, cap: int, stop_base: int, rules, n: int) -> int:
    """Finish block layout (int32 words from ``base``): stop_offsets [cap + 1], num_output,
    max_tokens, num_tokens [cap each], ignore_eos bytes [cap]; stop ids from ``stop_base``."""
    lens = np.fromiter((len(r.stop_token_ids) for r in rules), np.int64, n)
    offs = hin[base : base + n + 1]
    offs[0] = 0
    offs[1:] = np.cumsum(lens)
    o = base + cap + 1
    hin[o : o + n] = np.fromiter((r.num_output for r in rules), np.int32, n)
    hin[o + cap : o + cap + n] = np.fromiter((r.max_tokens for r in rules), np.int32, n)
    hin[o + 2 * cap : o + 2 * cap + n] = np.fromiter((r.num_tokens for r in rules), np.int32, n)
    ign = hin[o + 3 * cap : o + 3 * cap + cap // 4].view(np.uint8)
    ign[:n] = np.fromiter((1 if r.ignore_eos else 0 for r in rules), np.uint8, n)
    nstop = int(offs[n])
    if nstop:
        hin[stop_base : stop_base + nstop] = [t for r in rules for t in r.stop_token_ids]
    return nstop


def _raise_for_status(status: np.ndarray, temperature: np.ndarray | None = None) -> None:
    bad = np.flatnonzero(status != _lib.ROW_OK)
    if bad.size == 0:
        return
    b = int(bad[0])
    code = int(status[b])
    if code == _lib.ROW_BAD_PARAM:
        if temperature is not None and np.isnan(temperature[b]):
            # a NaN temperature passes SamplingParams' check (config.py:146) and reaches
            # multinomial as NaN probabilities in the reference (sampling.py:27)
            raise RuntimeError(_BAD_PROBS)
        raise ValueError(f"invalid sampling parameters or row index for row {b} "
                         "(temperature must be finite, top_p in (0, 1], top_k >= 0)")
    raise RuntimeError(_BAD_PROBS)


def _args(logits, n: int, row_map_given: bool, bufs: _Buffers) -> list:
    """The C ABI arguments shared by pbs_sample, pbs_sample_debug and (the first seven)
    pbs_argmax: the logits, the staged per-row arrays on the device and the outputs."""
    cap = bufs.cap
    base = bufs.d_in.data_ptr()
    ptr = [base + 4 * i * cap for i in range(5)]
    out_tok = bufs.d_out.data_ptr()
    return [
        logits.data_ptr(),
        _TORCH_DTYPE[logits.dtype],
        logits.shape[0],
        n,
        logits.shape[1],
        logits.stride(0),
        ptr[_IN_MAP] if row_map_given else None,
        ptr[_IN_T],
        ptr[_IN_K],
        ptr[_IN_P],
        ptr[_IN_U],
        out_tok,
        out_tok + 4 * cap,
    ]


def _raise_for_rc(lib, rc: int, what: str) -> None:
    if rc == _lib.OK:
        return
    msg = _lib.last_error(lib)
    if rc == _lib.ERR_INVALID_ARGUMENT:
        raise ValueError(msg)
    if rc == _lib.ERR_UNSUPPORTED_DTYPE:
        raise TypeError(msg)
    raise SamplerError(f"{what} failed ({rc}): {msg}")


def _enqueue(logits, n: int, row_map_given: bool, bufs: _Buffers, finish, greedy: bool, sp) -> int:
    """The stream work of one (non-debug) sampling call on stream ``sp``: the staged
    arrays to the device, ``pbs_argmax`` (``greedy``: every row greedy with valid
    parameters) or ``pbs_sample``, with ``finish`` (eos id, max_model_len, number of stop
    ids) the stop check on the sampler's device tokens, and the outputs back to the pinned
    buffer. No allocation and no memset, so the whole sequence can be captured in a graph.
    Returns the number of output blocks copied back."""
    lib = _lib.load()
    cap = bufs.cap
    words = bufs.fin if finish is None else bufs.stop_ids + finish[2]
    bufs.d_in[:words].copy_(bufs.h_in[:words], non_blocking=True)
    args = _args(logits, n, row_map_given, bufs)
    out_tok = args[11]
    if greedy:
        _raise_for_rc(lib, lib.pbs_argmax(*args[:7], out_tok, args[12], sp), "pbs_argmax")
    else:
        _raise_for_rc(lib, lib.pbs_sample(*args, None, 0, sp), "pbs_sample")
    nout = 2
    if finish is not None:
        eos, max_model_len, nstop = finish
        base = bufs.d_in.data_ptr()
        f = base + 4 * bufs.fin
        o = f + 4 * (cap + 1)
        rc = lib.pbs_finish_reasons(out_tok, n, -1 if eos is None else int(eos), o + 4 * 3 * cap, f,
                                    base + 4 * bufs.stop_ids if nstop else None, o, o + 4 * cap, o + 8 * cap,
                                    int(max_model_len), out_tok + 8 * cap, sp)
        if rc != _lib.OK:
            raise SamplerError(f"pbs_finish_reasons failed ({rc}): {_lib.last_error(lib)}")
        nout = 3
    bufs.h_out[: nout * cap].copy_(bufs.d_out[: nout * cap], non_blocking=True)
    return nout


def _read_out(bufs: _Buffers, n: int, finish: bool):
    cap = bufs.cap
    hout = bufs.h_out_np
    tokens = hout[:n].copy()
    status = hout[cap : cap + n].copy()
    reasons = hout[2 * cap : 2 * cap + n].copy() if finish else None
    return tokens, status, reasons


def _launch(logits, n: int, row_map_given: bool, debug: bool, bufs: _Buffers, finish=None, timing=None,
            greedy: bool = False):
    """One sampling call on the current stream (``_enqueue``, or ``pbs_sample_debug`` with
    ``debug``), then one synchronisation. Returns host tokens, statuses and reasons (None
    without ``finish``) plus the device diagnostics of a debug call."""
    stream = torch.cuda.current_stream(logits.device)
    sp = stream.cuda_stream
    probs = kept = info = None
    if debug:
        if finish is not None:
            raise ValueError("the diagnostic call takes no stop check")
        lib = _lib.load()
        cap = bufs.cap
        bufs.d_in[: bufs.fin].copy_(bufs.h_in[: bufs.fin], non_blocking=True)
        args = _args(logits, n, row_map_given, bufs)
        V = logits.shape[1]
        probs = torch.empty((n, V), dtype=torch.float32, device=logits.device)
        kept = torch.empty((n, V), dtype=torch.uint8, device=logits.device)
        info = torch.empty(n * _lib.ROW_INFO_DTYPE.itemsize, dtype=torch.uint8, device=logits.device)
        rc = lib.pbs_sample_debug(*args, probs.data_ptr(), kept.data_ptr(), info.data_ptr(), None, 0, sp)
        _raise_for_rc(lib, rc, "pbs_sample")
        bufs.h_out[: 2 * cap].copy_(bufs.d_out[: 2 * cap], non_blocking=True)
    else:
        _enqueue(logits, n, row_map_given, bufs, finish, greedy, sp)
    stream.synchronize()
    if timing is not None:
        timing["launch_sync"] = time.perf_counter()
    tokens, status, reasons = _read_out(bufs, n, finish is not None)
    return tokens, status, reasons, probs, kept, info


def _uniforms(temperature: np.ndarray, generators: Sequence[torch.Generator]) -> np.ndarray:
    """One uniform per stochastic row (temperature != 0), in row order, float32."""
    n = temperature.shape[0]
    out = np.zeros(n, dtype=np.float32)
    idx = np.flatnonzero(temperature != 0)
    if idx.size == 0:
        return out
    g0 = generators[int(idx[0])]
    if all(generators[i] is g0 for i in idx.tolist()):
        # every stochastic row shares one generator (the engine's, engine.py:58): one call
        out[idx] = torch.rand(idx.size, generator=g0, device=g0.device).numpy()
        return out
    # runs of consecutive stochastic rows (greedy rows between them draw nothing) sharing a
    # generator: one torch.rand per run
    rows = idx.tolist()
    i = 0
    while i < len(rows):
        g = generators[rows[i]]
        j = i + 1
        while j < len(rows) and generators[rows[j]] is g:
            j += 1
        if j - i == 1:
            out[rows[i]] = float(torch.rand((), generator=g, device=g.device))
        else:
            out[rows[i:j]] = torch.rand(j - i, generator=g, device=g.device).numpy()
        i = j
    return out


def draw_uniforms(params: Sequence, generators: Sequence[torch.Generator]) -> list[float]:
    """One ``torch.rand`` draw per stochastic row, in row order; greedy rows draw nothing.

    Consecutive stochastic rows that share a generator (the engine's shared generator for
    unseeded requests, engine.py:58) take their draws from one ``torch.rand(n)`` call: torch
    fills it with the same numbers, in the same order, as n scalar draws, and leaves the
    generator in the same state.
    """
    t = np.fromiter(map(_TEMPERATURE, params), np.float64, len(params))
    return [float(v) for v in _uniforms(t, generators)]


def _param_arrays(params: Sequence, n: int):
    t = np.fromiter(map(_TEMPERATURE, params), np.float64, n)
    k = np.fromiter(map(_TOP_K, params), np.int64, n)
    p = np.fromiter(map(_TOP_P, params), np.float64, n)
    # SamplingParams' own checks (config.py:146-154), for objects built without them
    if (t < 0).any() or not ((p > 0) & (p <= 1)).all() or (k < 0).any():
        raise ValueError("invalid SamplingParams")
    return t, k, p


def _sample(logits, params, generators, rows, finish_rules=None, eos_token_id=None, max_model_len=0,
            timing=None):
    logits = _check_logits(logits)
    n = len(rows) if rows is not None else logits.shape[0]
    if len(params) != n or len(generators) != n:
        raise ValueError(f"need {n} params and generators, got {len(params)} and {len(generators)}")
    if finish_rules is not None and len(finish_rules) != n:
        raise ValueError(f"need {n} finish rules, got {len(finish_rules)}")
    if n == 0:
        return [], ([] if finish_rules is not None else None)
    if timing is not None:
        timing["start"] = time.perf_counter()
    t, k, p = _param_arrays(params, n)
    u = _uniforms(t, generators)
    if timing is not None:
        timing["uniforms"] = time.perf_counter()
    h = _pack(n, t, k, p, u, rows, logits.shape[1])
    bufs = _buffers_for(logits.device)
    with bufs.lock:
        nstop = sum(len(r.stop_token_ids) for r in finish_rules) if finish_rules is not None else 0
        bufs.ensure(n, nstop)
        _stage_params(bufs, h, n)
        fin = None
        if finish_rules is not None:
            fin = (eos_token_id, max_model_len, _stage_finish(bufs, finish_rules, n))
        if timing is not None:
            timing["pack"] = time.perf_counter()
        tokens, status, reasons, _, _, _ = _launch(logits, n, rows is not None, False, bufs, finish=fin,
                                                   timing=timing, greedy=_all_greedy(h))
    _raise_for_status(status, t)
    toks = tokens.tolist()
    if finish_rules is None:
        return toks, None
    from .finish import REASONS

    return toks, [REASONS[c] for c in reasons.tolist()]


def sample(logits: torch.Tensor, params: Sequence, generators: Sequence[torch.Generator],
           rows: Sequence[int] | None = None) -> list[int]:
    """Sample one token for each of ``rows`` (default: every row) of ``logits`` [B, vocab].

    ``params[i]`` and ``generators[i]`` belong to the i-th sampled row (the reference's
    ``seq.sampling`` and ``state.generator``, engine.py:138-139). Row order is the order
    uniforms are drawn in, matching the reference's per-row loop over one shared engine
    generator.
    """
    return _sample(logits, params, generators, rows)[0]


def sample_and_finish(logits: torch.Tensor, params: Sequence, generators: Sequence[torch.Generator],
                      rules: Sequence, eos_token_id: int | None, max_model_len: int,
                      rows: Sequence[int] | None = None) -> tuple[list[int], list[str | None]]:
    """``sample`` plus the stop check of each sampled sequence after its new token
    (pagedbatch/engine.py:173-182, with ``rules[i]`` a ``finish.FinishRule`` that counts
    the new token): the check runs on the device right after the sampling kernel and the
    reasons ("stop", "length" or None) come back in the tokens' copy."""
    return _sample(logits, params, generators, rows, finish_rules=rules, eos_token_id=eos_token_id,
                   max_model_len=max_model_len)


class SamplingGraph:
    """One engine step's sampling call for a fixed batch, captured in a HIP graph.

    The batch is fixed at construction: the logits buffer (which must keep its address,
    e.g. a captured decode step's output, and hold the step's logits at each call), the
    sampled rows, their parameters and, with ``finish_rules``, the stop rules' stop ids and
    eos. The graph holds the parameters' copy to the device, ``pbs_sample`` (``pbs_argmax``
    when every row is greedy), the stop check and the copy back; nothing in it allocates or
    clears memory. Each call draws the rows' uniforms from their generators on the host
    (as ``sample`` does, engine.py:138-139), writes them and the rules' per-step counts
    into the graph's own pinned staging buffer, replays the graph and synchronises once:
    the same tokens and reasons as ``sample_and_finish`` on the same logits and generators.
    """

    def __init__(self, logits: torch.Tensor, params: Sequence, rows: Sequence[int] | None = None,
                 finish_rules: Sequence | None = None, eos_token_id: int | None = None, max_model_len: int = 0):
        logits = _check_logits(logits)
        n = len(rows) if rows is not None else logits.shape[0]
        if n == 0:
            raise ValueError("a sampling graph needs at least one row")
        if len(params) != n:
            raise ValueError(f"need {n} params, got {len(params)}")
        if finish_rules is not None and len(finish_rules) != n:
            raise ValueError(f"need {n} finish rules, got {len(finish_rules)}")
        self.logits, self.n, self.rows = logits, n, rows
        self.t, k, p = _param_arrays(params, n)
        h = _pack(n, self.t, k, p, np.zeros(n, np.float32), rows, logits.shape[1])
        self.greedy = _all_greedy(h)
        self.bufs = _Buffers(logits.device)
        nstop = sum(len(r.stop_token_ids) for r in finish_rules) if finish_rules is not None else 0
        self.bufs.ensure(n, nstop)
        _stage_params(self.bufs, h, n)
        self.fin = None
        if finish_rules is not None:
            self.fin = (eos_token_id, max_model_len, _stage_finish(self.bufs, finish_rules, n))
        dev = logits.device
        # one call outside the capture (first launches), then the capture; the uniforms
        # staged meanwhile are zeros, and no generator is touched
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            _enqueue(logits, n, rows is not None, self.bufs, self.fin, self.greedy, side.cuda_stream)
        side.synchronize()
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            _enqueue(logits, n, rows is not None, self.bufs, self.fin, self.greedy,
                     torch.cuda.current_stream(dev).cuda_stream)
        torch.cuda.synchronize(dev)

    def __call__(self, generators: Sequence[torch.Generator], finish_rules: Sequence | None = None):
        """Tokens (and, with stop rules, reasons) of the rows for the logits the buffer holds
        now. ``finish_rules`` (required when the graph has a stop check) may change from call
        to call except in their total number of stop ids, which sizes the captured copy."""
        if len(generators) != self.n:
            raise ValueError(f"need {self.n} generators, got {len(generators)}")
        if (finish_rules is None) != (self.fin is None):
            raise ValueError("finish_rules must be given exactly when the graph was built with them")
        bufs, cap, n = self.bufs, self.bufs.cap, self.n
        u = _uniforms(self.t, generators)
        bufs.h_in_np[_IN_U * cap : _IN_U * cap + n] = u.view(np.int32)
        if finish_rules is not None:
            if len(finish_rules) != n:
                raise ValueError(f"need {n} finish rules, got {len(finish_rules)}")
            if _stage_finish(bufs, finish_rules, n) != self.fin[2]:
                raise ValueError("the number of stop ids changed since the graph was captured")
        self.graph.replay()
        torch.cuda.current_stream(self.logits.device).synchronize()
        tokens, status, reasons = _read_out(bufs, n, self.fin is not None)
        _raise_for_status(status, self.t)
        if self.fin is None:
            return tokens.tolist(), None
        from .finish import REASONS

        return tokens.tolist(), [REASONS[c] for c in reasons.tolist()]


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
        _stage_params(bufs, h, n)
        tokens, status, _, probs, kept, info = _launch(logits, n, row_map is not None, debug, bufs,
                                                       greedy=not debug and _all_greedy(h))
    if check:
        _raise_for_status(status, np.asarray(temperature, dtype=np.float64))
    if not debug:
        return tokens, status
    info_np = np.frombuffer(info.cpu().numpy().tobytes(), dtype=_lib.ROW_INFO_DTYPE).copy()
    return DebugOutput(tokens=tokens, status=status, info=info_np, probs=probs, kept=kept)
