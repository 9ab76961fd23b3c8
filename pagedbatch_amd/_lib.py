"""ctypes binding of the C ABI declared in include/pbsample.h.

The shared library is built in-tree (``pagedbatch_amd/libpbsample.so``, see
``pagedbatch_amd/build.py``). It is loaded after ``torch`` so that it binds to the HIP
runtime torch already loaded, which makes torch's device pointers and streams valid in it.
There is no fallback: without the library every sampling call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpbsample.so")

ABI_VERSION = 1

# dtype codes (PBS_DTYPE_*)
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2

# return codes (PBS_OK / PBS_ERR_*)
OK = 0
ERR_INVALID_ARGUMENT = -1
ERR_UNSUPPORTED_DTYPE = -2
ERR_HIP = -3
ERR_WORKSPACE = -4

# per-row status (PBS_ROW_*)
ROW_OK, ROW_NAN, ROW_NONFINITE, ROW_BAD_PARAM = 0, 1, 2, 3

# finish reasons (PBS_FINISH_*)
FINISH_NONE, FINISH_STOP, FINISH_LENGTH = 0, 1, 2

# the C symbols include/pbattn.h declares
ATTN_SYMBOLS = ("pba_decode_attention",)

# the C symbols include/pblmhead.h declares
LMHEAD_SYMBOLS = ("pbs_lm_head_workspace_bytes", "pbs_lm_head_argmax", "pbs_lm_head_argmax_noalloc")

# the C symbols include/pbsample.h declares, in declaration order
SYMBOLS = ("pbs_abi_version", "pbs_last_error", "pbs_workspace_bytes", "pbs_sample", "pbs_sample_debug",
           "pbs_argmax", "pbs_finish_reasons")

# layout of pbs_row_info
ROW_INFO_DTYPE = np.dtype(
    [
        ("token", "<i4"),
        ("status", "<i4"),
        ("x_max", "<f4"),
        ("x_kth", "<f4"),
        ("x_cut", "<f4"),
        ("n_cut_tie", "<i4"),
        ("n_cut_keep", "<i4"),
        ("n_kept", "<i4"),
        ("z_k", "<f8"),
        ("z_p", "<f8"),
        ("target", "<f8"),
    ]
)
assert ROW_INFO_DTYPE.itemsize == 56


class SamplerUnavailable(RuntimeError):
    """The HIP sampler library is missing or does not match this package."""


_lib = None
_lock = threading.Lock()

_c = ctypes
_SAMPLE_ARGS = [
    _c.c_void_p,  # logits
    _c.c_int,  # dtype
    _c.c_int64,  # n_logit_rows
    _c.c_int64,  # rows
    _c.c_int64,  # vocab
    _c.c_int64,  # row_stride
    _c.c_void_p,  # row_map
    _c.c_void_p,  # temperature
    _c.c_void_p,  # top_k
    _c.c_void_p,  # top_p
    _c.c_void_p,  # uniform
    _c.c_void_p,  # out_token
    _c.c_void_p,  # out_status
]


def load(path: str | None = None):
    """Load (once) and return the ctypes handle of libpbsample.so."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        import torch  # noqa: F401  (binds the library to torch's HIP runtime)

        p = path or LIB_PATH
        if not os.path.exists(p):
            raise SamplerUnavailable(
                f"{p} is missing: build it with `python -m pagedbatch_amd.build` (hipcc, gfx950)"
            )
        lib = ctypes.CDLL(p)
        lib.pbs_abi_version.restype = _c.c_int
        lib.pbs_abi_version.argtypes = []
        lib.pbs_last_error.restype = _c.c_char_p
        lib.pbs_last_error.argtypes = []
        lib.pbs_workspace_bytes.restype = _c.c_size_t
        lib.pbs_workspace_bytes.argtypes = [_c.c_int64, _c.c_int64, _c.c_int]
        lib.pbs_sample.restype = _c.c_int
        lib.pbs_sample.argtypes = _SAMPLE_ARGS + [_c.c_void_p, _c.c_size_t, _c.c_void_p]
        lib.pbs_sample_debug.restype = _c.c_int
        lib.pbs_sample_debug.argtypes = _SAMPLE_ARGS + [
            _c.c_void_p,  # out_probs
            _c.c_void_p,  # out_kept
            _c.c_void_p,  # out_info
            _c.c_void_p,  # workspace
            _c.c_size_t,  # workspace_bytes
            _c.c_void_p,  # stream
        ]
        lib.pbs_argmax.restype = _c.c_int
        lib.pbs_argmax.argtypes = [
            _c.c_void_p,  # logits
            _c.c_int,  # dtype
            _c.c_int64,  # n_logit_rows
            _c.c_int64,  # rows
            _c.c_int64,  # vocab
            _c.c_int64,  # row_stride
            _c.c_void_p,  # row_map
            _c.c_void_p,  # out_token
            _c.c_void_p,  # out_status
            _c.c_void_p,  # stream
        ]
        lib.pbs_finish_reasons.restype = _c.c_int
        lib.pbs_finish_reasons.argtypes = [
            _c.c_void_p,  # tokens
            _c.c_int64,  # rows
            _c.c_int32,  # eos_token_id
            _c.c_void_p,  # ignore_eos
            _c.c_void_p,  # stop_offsets
            _c.c_void_p,  # stop_ids
            _c.c_void_p,  # num_output
            _c.c_void_p,  # max_tokens
            _c.c_void_p,  # num_tokens
            _c.c_int32,  # max_model_len
            _c.c_void_p,  # out_reason
            _c.c_void_p,  # stream
        ]
        lib.pba_decode_attention.restype = _c.c_int
        lib.pba_decode_attention.argtypes = [
            _c.c_void_p,  # q
            _c.c_void_p,  # k_cache
            _c.c_void_p,  # v_cache
            _c.c_int64,  # n_slots
            _c.c_void_p,  # block_table
            _c.c_int64,  # max_blocks
            _c.c_void_p,  # context_lens
            _c.c_int64,  # rows
            _c.c_int,  # n_heads
            _c.c_int,  # n_kv_heads
            _c.c_int,  # head_dim
            _c.c_int,  # block_size
            _c.c_int,  # max_context
            _c.c_float,  # scale
            _c.c_void_p,  # out
            _c.c_void_p,  # stream
        ]
        lib.pbs_lm_head_workspace_bytes.restype = _c.c_size_t
        lib.pbs_lm_head_workspace_bytes.argtypes = [_c.c_int64, _c.c_int64]
        lib.pbs_lm_head_argmax.restype = _c.c_int
        lib.pbs_lm_head_argmax.argtypes = [
            _c.c_void_p,  # hidden
            _c.c_int64,  # hidden_stride
            _c.c_void_p,  # weight
            _c.c_int64,  # rows
            _c.c_int64,  # hidden_dim
            _c.c_int64,  # vocab
            _c.c_void_p,  # out_logits
            _c.c_void_p,  # out_token
            _c.c_void_p,  # workspace
            _c.c_size_t,  # workspace_bytes
            _c.c_void_p,  # stream
        ]
        lib.pbs_lm_head_argmax_noalloc.restype = _c.c_int
        lib.pbs_lm_head_argmax_noalloc.argtypes = lib.pbs_lm_head_argmax.argtypes[:8] + [_c.c_void_p]
        v = lib.pbs_abi_version()
        if v != ABI_VERSION:
            raise SamplerUnavailable(f"{p} has ABI version {v}, this package expects {ABI_VERSION}")
        if path is None:
            _lib = lib
        return lib


def last_error(lib) -> str:
    msg = lib.pbs_last_error()
    return msg.decode("utf-8", "replace") if msg else ""
