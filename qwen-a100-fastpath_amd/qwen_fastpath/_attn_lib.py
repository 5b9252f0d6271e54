"""ctypes binding of libqf_spec_attn.so, the C ABI declared in include/qf_spec_attn.h.

Built in-tree by qwen-a100-fastpath_amd/csrc/Makefile next to this file.  There is no fallback
implementation: if the library is missing, the attention entry point raises.
"""
from __future__ import annotations

import ctypes
import os

from ._lib import QFError

LIB_NAME = "libqf_spec_attn.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 1

MAX_ROWS = 64     # QF_SPEC_ATTN_MAX_ROWS
MIN_PAGE = 16     # QF_SPEC_ATTN_MIN_PAGE
KEY_BLOCK = 32    # QF_SPEC_ATTN_KEY_BLOCK
HEAD_SIZES = (64, 128, 256)

# Every symbol include/qf_spec_attn.h declares.
EXPORTS = (
    "qf_spec_attn_abi_version",
    "qf_spec_attn_workspace_bytes",
    "qf_spec_attention",
)

_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the library once.  Raises ImportError (never falls back) when it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `make -C qwen-a100-fastpath_amd/csrc` "
            "(or __graft_entry__.build()); the attention op has no non-HIP implementation")
    import torch  # noqa: F401  (its HIP runtime first, as for libqf_w8a16.so)
    L = ctypes.CDLL(LIB_PATH)
    p, i64, i32, sz, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t, ctypes.c_float
    L.qf_spec_attn_abi_version.argtypes = []
    L.qf_spec_attn_abi_version.restype = i32
    L.qf_spec_attn_workspace_bytes.argtypes = [i32] * 6
    L.qf_spec_attn_workspace_bytes.restype = sz
    L.qf_spec_attention.argtypes = [p, i64, i64,
                                    p, i64, i64, i64,
                                    p, i64, i64, i64,
                                    p, i64, p,
                                    p, i64, i64,
                                    i32, i32, i32, i32, i32, i32, f32, i32, i32,
                                    p, sz, p]
    L.qf_spec_attention.restype = i32
    v = L.qf_spec_attn_abi_version()
    if v != ABI_VERSION:
        raise ImportError(f"{LIB_PATH}: ABI version {v}, expected {ABI_VERSION}")
    _lib = L
    return L


def workspace_bytes(num_reqs: int, q_len: int, num_heads: int, num_kv_heads: int, head_size: int,
                    num_splits: int) -> int:
    return int(load().qf_spec_attn_workspace_bytes(num_reqs, q_len, num_heads, num_kv_heads, head_size,
                                                   num_splits))


def check(status: int, what: str) -> None:
    if status != 0:
        raise QFError(status, what)
