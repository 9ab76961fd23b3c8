"""Paged-attention decode on the GPU: one kernel per layer and step instead of the
gather / repeat / SDPA sequence of pagedbatch/model.py:201-224.

``decode_attention`` takes one query token per sequence (a decode step), the layer's K/V
slot pools and the block tables, and returns the attention output in fp32. Query head h
reads KV head ``h // (n_heads // n_kv_heads)`` (the reference's ``repeat_interleave`` at
model.py:214-216); slots follow block_manager.py:88-91 (block * block_size + offset).
"""

from __future__ import annotations

import math

import torch

from . import _lib
from .sampling import SamplerError


HEAD_DIMS = (64, 128)  # the head sizes the kernel serves (k_decode indexes [slot][kv_head][head_dim])


def _check_args(q, k_cache, v_cache, block_table, context_lens) -> None:
    """Shapes, dtypes, devices and alignment of every operand, before anything reaches the
    kernel: it indexes the caches as [n_slots][n_kv_heads][64] bf16 through 16-byte loads
    and reads every pointer on q's device, so a smaller cache head size, a host tensor or
    a misaligned view would be read out of bounds instead of failing here."""
    if q.dtype != torch.float32 or q.dim() != 3 or not q.is_contiguous():
        raise ValueError("q must be a contiguous fp32 [rows, n_heads, head_dim] tensor")
    rows, n_heads, head_dim = q.shape
    if head_dim not in HEAD_DIMS:
        raise ValueError(f"head_dim must be 64 or 128, got {head_dim}")
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        if c.dtype != torch.bfloat16 or c.dim() != 3 or not c.is_contiguous():
            raise ValueError(f"{name} must be a contiguous bf16 [n_slots, n_kv_heads, head_dim] tensor")
    if k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache differ in shape")
    if k_cache.shape[2] != head_dim:
        raise ValueError(f"the caches' head_dim {k_cache.shape[2]} differs from q's {head_dim}")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or not block_table.is_contiguous():
        raise ValueError("block_table must be a contiguous int32 [rows, max_blocks] tensor")
    if context_lens.dtype != torch.int32 or context_lens.dim() != 1 or not context_lens.is_contiguous():
        raise ValueError("context_lens must be a contiguous int32 [rows] tensor")
    if block_table.shape[0] != rows or context_lens.shape[0] != rows:
        raise ValueError("block_table and context_lens need one row per query row")
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache), ("block_table", block_table),
                    ("context_lens", context_lens)):
        if t.device != q.device:
            raise ValueError(f"{name} is on {t.device}, q on {q.device}: every operand must be on q's device")
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        if t.data_ptr() % 16:
            raise ValueError(f"{name} must start on a 16-byte boundary (the kernel reads it in 16-byte loads)")
    if not q.is_cuda:
        raise ValueError("the operands must live on a ROCm device; decode_attention has no CPU path")


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_table: torch.Tensor,
                     context_lens: torch.Tensor, block_size: int, max_context: int,
                     scale: float | None = None) -> torch.Tensor:
    """q: fp32 [rows, n_heads, head_dim] (head_dim 64 or 128); k_cache / v_cache: bf16
    [n_slots, n_kv_heads, head_dim];
    block_table: int32 [rows, max_blocks]; context_lens: int32 [rows], each in
    [1, max_context]. Returns fp32 [rows, n_heads, head_dim]. Asynchronous on the current
    stream; a sequence whose block table points outside the pools gets NaN."""
    _check_args(q, k_cache, v_cache, block_table, context_lens)
    rows, n_heads, head_dim = q.shape
    n_slots, n_kv_heads, _ = k_cache.shape
    out = torch.empty_like(q)
    lib = _lib.load()
    rc = lib.pba_decode_attention(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), n_slots, block_table.data_ptr(), block_table.shape[1],
        context_lens.data_ptr(), rows, n_heads, n_kv_heads, head_dim, int(block_size), int(max_context),
        float(1.0 / math.sqrt(head_dim) if scale is None else scale), out.data_ptr(),
        torch.cuda.current_stream(q.device).cuda_stream)
    if rc != _lib.OK:
        raise SamplerError(f"pba_decode_attention failed ({rc}): {_lib.last_error(lib)}")
    return out
