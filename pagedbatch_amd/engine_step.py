"""A minimal batched decode loop around the sampler: the engine step of pagedbatch with the
per-row sampling loop hoisted into one ``sample()`` call per step.

It exists to measure the sampler inside an engine step (the reference's end-to-end
configuration: smollm2-135m-shaped random model, block size 16, 64 requests of 128
prompt tokens and 128 output tokens, half greedy and half top-k=50 / top-p=0.9). The model
is plain PyTorch and follows the Llama layout of pagedbatch/model.py:150-296 (RMSNorm,
rotate-half RoPE, grouped-query attention over a paged KV cache written through a slot
mapping, SwiGLU MLP, tied LM head, N(0, 0.02) initialisation); the sampling is this
package's kernel. What the engine does per step (pagedbatch/engine.py:104-139): one forward
over the scheduled tokens, logits of each sequence's last token, then one token per
sequence, here from a single batched call (the hoist of engine.py:133-139).

Out of scope: scheduling, preemption, chunked prefill, stop strings and the server; every
request here runs from prefill to its last token in lockstep.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass, field

import numpy as np

import torch
import torch.nn.functional as F

from .attention import decode_attention
from .config import SamplingParams
from .finish import FinishRule
from .sampling import SamplingGraph, _uniforms, sample_and_finish


@dataclass
class ModelShape:
    """pagedbatch/config.py:60-75 (the shape of HuggingFaceTB/SmolLM2-135M)."""

    vocab_size: int = 49152
    hidden_size: int = 576
    intermediate_size: int = 1536
    num_layers: int = 30
    num_heads: int = 9
    num_kv_heads: int = 3
    rms_norm_eps: float = 1e-5
    rope_theta: float = 100000.0

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads

    @classmethod
    def tiny(cls) -> "ModelShape":
        return cls(vocab_size=512, hidden_size=64, intermediate_size=128, num_layers=2, num_heads=4, num_kv_heads=2)


class Model:
    """Weights as plain tensors; forward over a flat token batch with a paged KV cache."""

    def __init__(self, shape: ModelShape, device: torch.device, dtype=torch.bfloat16, seed: int = 0,
                 max_positions: int = 4096):
        self.shape = shape
        g = torch.Generator().manual_seed(seed)
        H, I, D = shape.hidden_size, shape.intermediate_size, shape.head_dim

        def w(out_dim, in_dim):
            # [out, in] drawn like nn.Linear's weight, stored transposed ([in, out], contiguous)
            # so that every product is x @ W with no transposed operand
            return (torch.randn(out_dim, in_dim, generator=g) * 0.02).t().contiguous().to(device=device, dtype=dtype)

        embed = (torch.randn(shape.vocab_size, H, generator=g) * 0.02).to(device=device, dtype=dtype)
        self.embed = embed
        self.head = embed.t().contiguous()  # the tied LM head, [H, vocab]
        self.layers = []
        for _ in range(shape.num_layers):
            self.layers.append({
                "qkv": w((shape.num_heads + 2 * shape.num_kv_heads) * D, H),
                "o": w(H, shape.num_heads * D),
                "gate_up": w(2 * I, H),
                "down": w(H, I),
                "ln1": torch.ones(H, device=device, dtype=dtype),
                "ln2": torch.ones(H, device=device, dtype=dtype),
            })
        self.norm = torch.ones(H, device=device, dtype=dtype)
        inv = 1.0 / (shape.rope_theta ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
        f = torch.outer(torch.arange(max_positions, dtype=torch.float32), inv)
        emb = torch.cat([f, f], dim=-1)
        self.cos = emb.cos().to(device)
        self.sin = emb.sin().to(device)

    def _rms(self, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        x32 = x.float()
        return w * (x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + self.shape.rms_norm_eps)).to(x.dtype)

    def _rope(self, x: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        # x [T, heads, D] in fp32; rotate-half convention
        cos, sin = self.cos[pos].unsqueeze(1), self.sin[pos].unsqueeze(1)
        half = x.shape[-1] // 2
        rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
        return x * cos + rot * sin

    @torch.no_grad()
    def forward(self, tokens: torch.Tensor, pos: torch.Tensor, slots: torch.Tensor, seq_slots: torch.Tensor | None,
                q_len: int, cache: "PagedKV", fused_decode: bool = False, hidden_only: bool = False,
                context_lens: torch.Tensor | None = None, max_context: int | None = None) -> torch.Tensor:
        """``tokens``/``pos``/``slots``: [B * q_len] (sequence-major); ``seq_slots``: [B, L] the
        cache slots of each sequence's whole context, new tokens last. Returns [B, vocab]
        logits of each sequence's last token (with ``hidden_only``, its final hidden state
        [B, hidden] instead, for the fused lm_head). ``fused_decode`` runs decode steps
        (``q_len == 1``) through the paged-attention kernel (``attention.decode_attention``)
        instead of the gather + matmul + softmax below; it may take the context lengths as a
        device tensor ``context_lens`` with a fixed bound ``max_context`` instead of
        ``seq_slots`` (None), so that the step has the same shapes and kernel arguments every
        time (a captured graph)."""
        s = self.shape
        D, Hq, Hkv = s.head_dim, s.num_heads, s.num_kv_heads
        if seq_slots is not None:
            B, L = seq_slots.shape
        else:
            if not (fused_decode and q_len == 1 and context_lens is not None and max_context is not None):
                raise ValueError("without seq_slots the step must be a fused decode step with context_lens and "
                                 "max_context")
            B, L = tokens.numel(), None
        x = self.embed[tokens]
        scale = 1.0 / math.sqrt(D)
        causal = None
        if q_len > 1:
            qi = torch.arange(L - q_len, L, device=x.device).view(q_len, 1)
            causal = torch.arange(L, device=x.device).view(1, L) > qi  # True = masked
        for li, p in enumerate(self.layers):
            h = self._rms(x, p["ln1"])
            qkv = h @ p["qkv"]
            q = qkv[:, : Hq * D].view(-1, Hq, D).float()
            k = qkv[:, Hq * D : (Hq + Hkv) * D].view(-1, Hkv, D).float()
            v = qkv[:, (Hq + Hkv) * D :].view(-1, Hkv, D)
            q, k = self._rope(q, pos), self._rope(k, pos)
            cache.k[li].index_copy_(0, slots, k.to(cache.k[li].dtype))
            cache.v[li].index_copy_(0, slots, v)
            if fused_decode and q_len == 1:
                lens = context_lens if context_lens is not None else \
                    torch.full((B,), L, dtype=torch.int32, device=x.device)
                o = decode_attention(q.contiguous(), cache.k[li], cache.v[li], cache.block_table_i32, lens,
                                     cache.block_size, max_context if max_context is not None else L,
                                     scale).view(B, Hq * D)
            else:
                # attention in fp32 with contiguous operands: [B, Hkv, rep, q_len, D] x [B, Hkv, D, L]
                keys = cache.k[li][seq_slots].float().permute(0, 2, 3, 1).contiguous()  # [B, Hkv, D, L]
                vals = cache.v[li][seq_slots].float().permute(0, 2, 1, 3).contiguous()  # [B, Hkv, L, D]
                qh = q.view(B, q_len, Hkv, Hq // Hkv, D).permute(0, 2, 3, 1, 4).reshape(B, Hkv, -1, D).contiguous()
                att = torch.matmul(qh, keys) * scale  # [B, Hkv, rep * q_len, L]
                if causal is not None:
                    att = att.view(B, Hkv, Hq // Hkv, q_len, L).masked_fill(causal, float("-inf")).view(B, Hkv, -1, L)
                o = torch.matmul(torch.softmax(att, dim=-1), vals)  # [B, Hkv, rep * q_len, D]
                o = o.view(B, Hkv, Hq // Hkv, q_len, D).permute(0, 3, 1, 2, 4).reshape(B * q_len, Hq * D)
            x = x + o.to(x.dtype) @ p["o"]
            h = self._rms(x, p["ln2"])
            gu = h @ p["gate_up"]
            x = x + (F.silu(gu[:, : s.intermediate_size]) * gu[:, s.intermediate_size :]) @ p["down"]
        last = self._rms(x.view(B, q_len, -1)[:, -1], self.norm)
        return last.contiguous() if hidden_only else last @ self.head


class DecodeGraph:
    """The decode step's forward (one token per sequence, attention through the
    paged-attention kernel) captured once in a HIP graph and replayed every step. The
    per-step inputs (token ids, positions, cache slots, context lengths) live in fixed
    device buffers refilled before each replay, and the replay overwrites one fixed output
    buffer (the logits, or with ``hidden_only`` the final hidden state), which the caller
    consumes before the next replay. The capture's warm-up steps write the cache at slot 0
    with dummy values, so the graph is built before the prefill writes the prompts."""

    def __init__(self, model: Model, cache: "PagedKV", num_seqs: int, max_context: int, hidden_only: bool):
        dev = model.embed.device
        self.tokens = torch.zeros(num_seqs, dtype=torch.long, device=dev)
        self.pos = torch.zeros(num_seqs, dtype=torch.long, device=dev)
        self.slots = torch.zeros(num_seqs, dtype=torch.long, device=dev)
        self.lens = torch.ones(num_seqs, dtype=torch.int32, device=dev)

        def fwd():
            return model.forward(self.tokens, self.pos, self.slots, None, 1, cache, fused_decode=True,
                                 hidden_only=hidden_only, context_lens=self.lens, max_context=max_context)

        # warm-up on a side stream (libraries pick their kernels and workspaces outside the
        # capture), then the capture
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(2):
                fwd()
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out = fwd()
        torch.cuda.synchronize(dev)

    def __call__(self, tokens: torch.Tensor, pos: torch.Tensor, slots: torch.Tensor,
                 context_lens: torch.Tensor) -> torch.Tensor:
        self.tokens.copy_(tokens)
        self.pos.copy_(pos)
        self.slots.copy_(slots)
        self.lens.copy_(context_lens)
        self.graph.replay()
        return self.out


class PagedKV:
    """Per-layer K/V slot pools ([slots, kv_heads, head_dim]) in blocks of ``block_size``
    slots; each sequence owns whole blocks through its block table (block_manager.py:88-91:
    slot = block * block_size + offset)."""

    def __init__(self, shape: ModelShape, num_seqs: int, max_len: int, block_size: int, device, dtype):
        self.block_size = block_size
        blocks_per_seq = (max_len + block_size - 1) // block_size
        nslots = num_seqs * blocks_per_seq * block_size
        self.k = [torch.empty(nslots, shape.num_kv_heads, shape.head_dim, device=device, dtype=dtype)
                  for _ in range(shape.num_layers)]
        self.v = [torch.empty_like(t) for t in self.k]
        # block tables: sequence i holds blocks i, i + num_seqs, i + 2 num_seqs, ... (interleaved,
        # so that a sequence's blocks are not contiguous in the pool)
        self.block_table = torch.arange(blocks_per_seq, device=device).view(1, -1) * num_seqs + \
            torch.arange(num_seqs, device=device).view(-1, 1)
        self.block_table_i32 = self.block_table.to(torch.int32).contiguous()

    def slots(self, seq: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """Slots of positions ``pos`` of sequences ``seq`` (broadcast)."""
        blk = self.block_table[seq, pos // self.block_size]
        return blk * self.block_size + pos % self.block_size


@dataclass
class StepCapture:
    """What one step handed the sampler and got back: the logits (a device copy), the
    per-row parameters, the uniforms the rows drew and the tokens."""

    step: int
    logits: torch.Tensor
    temperature: list
    top_k: list
    top_p: list
    uniform: np.ndarray
    tokens: list


@dataclass
class StepTimes:
    """Per-step wall times (s): the forward (logits ready on the device) and the sampling
    call (params, uniforms, launch, kernel, stop check, tokens and reasons copied back).
    Step 0 is the prefill. ``reasons`` holds each step's finish reasons (engine.py:173-182)
    from the batched call; ``captures`` the steps asked for with ``capture_steps``."""

    forward_s: list = field(default_factory=list)
    sample_s: list = field(default_factory=list)
    tokens_per_step: int = 0
    reasons: list = field(default_factory=list)
    captures: list = field(default_factory=list)


def run(shape: ModelShape, num_seqs: int = 64, prompt_len: int = 128, output_len: int = 128, block_size: int = 16,
        device: str | torch.device = "cuda", seed: int = 0, per_row: bool = False,
        fused_decode: bool = False, capture_steps=(), fused_head: bool = False,
        graph: bool = False) -> tuple[StepTimes, list[list[int]]]:
    """Prefill every prompt, then decode in lockstep until each request has ``output_len``
    tokens. Half the requests are greedy, half top-k=50 / top-p=0.9 at temperature 1.0; the
    unseeded ones share one engine generator (engine.py:58). The batched path samples with
    one ``sample_and_finish`` call per step (the hoist of engine.py:133-139 with the stop
    check of engine.py:173-182 in the same launch sequence and copy back; the model has no
    EOS here, so every request runs to its length limit); ``per_row`` samples with one
    ``sample_token`` call per sequence (the reference loop, unhoisted). ``fused_decode``
    runs the decode steps' attention through the paged-attention kernel. ``fused_head``
    computes the logits with the fused lm_head + greedy kernel (``lm_head.lm_head_argmax``,
    model.py:283): greedy rows take its tokens, the stochastic rows are sampled from the
    logits it writes (``rows=``), and a step with no stochastic row writes no logits. The
    forward time then ends at the final hidden state and the sampling time includes the
    head. ``graph`` (with ``fused_decode``) replays the decode steps' forward from a HIP
    graph (``DecodeGraph``) instead of launching it op by op, and (without ``fused_head``)
    their sampling call from a second one (``sampling.SamplingGraph``): the host then only
    draws the uniforms, writes the stop rules' counts and synchronises. Returns the time
    split and the generated tokens."""
    if graph and not fused_decode:
        raise ValueError("graph replays the fused decode step: pass fused_decode=True")
    device = torch.device(device)
    model = Model(shape, device, seed=seed)
    cache = PagedKV(shape, num_seqs, prompt_len + output_len, block_size, device, torch.bfloat16)
    g = torch.Generator().manual_seed(seed + 1)
    prompts = torch.randint(3, shape.vocab_size, (num_seqs, prompt_len), generator=g)
    params = [SamplingParams(temperature=0.0) if i % 2 == 0 else SamplingParams(temperature=1.0, top_k=50, top_p=0.9)
              for i in range(num_seqs)]
    temps = np.array([p.temperature for p in params])
    engine_gen = torch.Generator().manual_seed(seed + 2)
    gens = [engine_gen] * num_seqs
    seq = torch.arange(num_seqs, device=device)
    out: list[list[int]] = [[] for _ in range(num_seqs)]
    times = StepTimes(tokens_per_step=num_seqs)
    capture_steps = set(capture_steps)
    dgraph = DecodeGraph(model, cache, num_seqs, prompt_len + output_len, hidden_only=fused_head) if graph else None
    # with the graph-replayed forward, the decode steps' sampling call is a graph too (on
    # the decode graph's fixed logits buffer); the stop rules' counts change every step
    sgraph = None
    if dgraph is not None and not fused_head and not per_row:
        rules0 = [FinishRule(ignore_eos=False, stop_token_ids=(), num_output=1, max_tokens=output_len,
                             num_tokens=prompt_len + 1)] * num_seqs
        sgraph = SamplingGraph(dgraph.out, params, finish_rules=rules0, max_model_len=prompt_len + output_len)

    def step(idx: int, tokens: torch.Tensor, start: int, q_len: int) -> list[int]:
        pos = torch.arange(start, start + q_len, device=device).view(1, -1).expand(num_seqs, -1)
        slots = cache.slots(seq.view(-1, 1), pos).reshape(-1)
        if dgraph is not None and q_len == 1:
            lens = torch.full((num_seqs,), start + 1, dtype=torch.int32, device=device)
            torch.cuda.synchronize(device)
            t0 = time.perf_counter()
            out_f = dgraph(tokens.reshape(-1), pos.reshape(-1), slots, lens)
        else:
            ctx = torch.arange(start + q_len, device=device).view(1, -1).expand(num_seqs, -1)
            seq_slots = cache.slots(seq.view(-1, 1), ctx)
            torch.cuda.synchronize(device)
            t0 = time.perf_counter()
            out_f = model.forward(tokens.reshape(-1), pos.reshape(-1), slots, seq_slots, q_len, cache, fused_decode,
                                  hidden_only=fused_head)
        torch.cuda.synchronize(device)
        t1 = time.perf_counter()
        if fused_head:
            toks, reasons = fused_head_step(model, out_f, params, gens, temps, n_out=len(out[0]) + 1)
            times.reasons.append(reasons)
            t2 = time.perf_counter()
            times.forward_s.append(t1 - t0)
            times.sample_s.append(t2 - t1)
            return toks
        logits = out_f
        cap = None
        if idx in capture_steps:
            # the uniforms this step's rows will draw: from a copy of the engine generator
            snap = torch.Generator().manual_seed(0)
            snap.set_state(engine_gen.get_state())
            cap = StepCapture(idx, logits.clone(), [p.temperature for p in params], [p.top_k for p in params],
                              [p.top_p for p in params], _uniforms(temps, [snap] * num_seqs), [])
            torch.cuda.synchronize(device)
            t1 = time.perf_counter()
        if per_row:
            from .sampling import sample_token
            toks = [sample_token(logits[i], params[i], gens[i]) for i in range(num_seqs)]
        else:
            n_out = len(out[0]) + 1  # outputs after this token (lockstep)
            rules = [FinishRule(ignore_eos=False, stop_token_ids=(), num_output=n_out, max_tokens=output_len,
                                num_tokens=prompt_len + n_out)] * num_seqs
            if sgraph is not None and q_len == 1:
                toks, reasons = sgraph(gens, rules)
            else:
                toks, reasons = sample_and_finish(logits, params, gens, rules, None, prompt_len + output_len)
            times.reasons.append(reasons)
        t2 = time.perf_counter()
        times.forward_s.append(t1 - t0)
        times.sample_s.append(t2 - t1)
        if cap is not None:
            cap.tokens = list(toks)
            times.captures.append(cap)
        return toks

    def fused_head_step(model, hidden, params, gens, temps, n_out):
        from .finish import finish_reasons
        from .lm_head import lm_head_argmax

        stoch = [i for i in range(num_seqs) if temps[i] != 0]
        greedy = [i for i in range(num_seqs) if temps[i] == 0]
        logits, gtok = lm_head_argmax(hidden, model.embed, want_logits=bool(stoch))
        rule = FinishRule(ignore_eos=False, stop_token_ids=(), num_output=n_out, max_tokens=output_len,
                          num_tokens=prompt_len + n_out)
        toks: list = [0] * num_seqs
        reasons: list = [None] * num_seqs
        if stoch:
            st, sr = sample_and_finish(logits, [params[i] for i in stoch], [gens[i] for i in stoch],
                                       [rule] * len(stoch), None, prompt_len + output_len, rows=stoch)
            for j, i in enumerate(stoch):
                toks[i], reasons[i] = st[j], sr[j]
        if greedy:
            # the stop check over every row's greedy token (as cheap as over the greedy rows,
            # and no device gather), then the greedy rows' entries on the host
            gr = finish_reasons(gtok, [rule] * num_seqs, None, prompt_len + output_len)
            gl = gtok.cpu().tolist()
            for i in greedy:
                toks[i], reasons[i] = gl[i], gr[i]
        return toks, reasons

    toks = step(0, prompts.to(device), 0, prompt_len)
    for i, t in enumerate(toks):
        out[i].append(t)
    for n in range(1, output_len):
        cur = torch.tensor([o[-1] for o in out], device=device).view(-1, 1)
        toks = step(n, cur, prompt_len + n - 1, 1)
        for i, t in enumerate(toks):
            out[i].append(t)
    return times, out
