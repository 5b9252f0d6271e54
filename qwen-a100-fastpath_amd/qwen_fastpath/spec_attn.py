"""Split-KV, GQA-packed verification attention (QWEN_FAST_ATTN) on MI355X.

``gqa_packed_spec_attention`` has the signature and meaning of the reference's function
(plugin/qwen_fastpath/spec_attn.py:135-173): causal attention for a uniform decode batch of
``num_reqs`` requests x ``Q`` query tokens (token b*Q + qi) over a paged KV cache, written into
``out``.  Query qi of request b attends cached positions [0, seq_lens[b] - Q + qi]; this step's K/V
must already be in the cache.  The work runs in libqf_spec_attn.so (hand-written HIP for gfx950):
one launch streams each kv head's cached prefix once for the Q*G query rows sharing it, split across
workgroups (the last split also attends this step's in-flight positions, causally per row), and a
second merges the split partials by log-sum-exp.  Both grids are
fixed for a batch shape and nothing is read back to the host, so the call can be captured in a HIP
graph (its split workspace comes from torch's caching allocator, as the reference's does).
"""
from __future__ import annotations

import torch

from . import _attn_lib as AL

LOG2E = 1.4426950408889634

# Defaults of the reference's call (spec_attn.py:136), except two sizes:
# * num_splits: the reference fixes 64 (for an A100's 108 SMs); here None picks one prefix workgroup
#   per compute unit, CUs // (num_reqs * num_kv_heads) splits (64 for one request with 4 kv heads on
#   MI355X's 256 CUs).  A prefix workgroup holds a whole CU (128 KiB of LDS, one wavefront per SIMD),
#   so a grid larger than the CU count runs in two rounds: at 2 requests and 38K context, 32 splits
#   take 64.7 us and 64 take 71.7 us.
# * min_chunk: 64 positions instead of 128, so that short contexts spread over more workgroups (one
#   request: 1K context 12.4 us against 14.3 us, 2K 13.1 against 14.7 us; no change from 8K on).
# block_n / num_warps / num_stages / combine_warps are Triton launch knobs there; the HIP kernels
# have fixed shapes and ignore them.
DEFAULT_NUM_SPLITS = None
DEFAULT_MIN_CHUNK = 64

_cu_count: dict = {}


def auto_num_splits(device: torch.device, num_reqs: int, num_kv_heads: int) -> int:
    """Prefix splits that give one workgroup per compute unit of `device` (at least 1)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    n = _cu_count.get(idx)
    if n is None:
        n = _cu_count[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return max(1, n // max(1, int(num_reqs) * int(num_kv_heads)))


def _check_bf16_rows(t: torch.Tensor, name: str):
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {t.dtype}")
    if t.stride(-1) != 1:
        raise ValueError(f"{name} must be contiguous in its last dimension")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")


def supported(query: torch.Tensor, key_cache: torch.Tensor, Q: int, num_kv_heads: int,
              value_cache: torch.Tensor | None = None, out: torch.Tensor | None = None,
              num_reqs: int | None = None) -> bool:
    """Calls the library serves, the checks of qf_spec_attention (csrc/qf_spec_attn.hip) restated so
    that anything else takes the caller's original path instead of raising: head size 64/128/256,
    Q * (H / H_kv) <= 64 packed rows, pages of at least 16 positions, every row stride a multiple of
    8 elements, 16-byte aligned tensors, a grid of at most 65535 (request, kv head) pairs, a 32-bit
    token count and per-stage byte offsets, and the same head geometry in every tensor."""
    H, D = query.shape[1], query.shape[2]
    if D not in AL.HEAD_SIZES or num_kv_heads < 1 or H % num_kv_heads or Q < 1 or Q * (H // num_kv_heads) > AL.MAX_ROWS:
        return False
    if key_cache.shape[1] < AL.MIN_PAGE:
        return False
    tensors = [t for t in (query, key_cache, value_cache, out) if t is not None]
    for t in tensors:
        if t.dtype != torch.bfloat16 or t.stride(-1) != 1 or not t.is_cuda or t.data_ptr() % 16:
            return False
        if any(s < 0 or s % 8 for s in t.stride()[:-1]):
            return False
    if out is not None and (out.shape[1] != H or out.shape[2] != D):
        return False
    tok_strides = [key_cache.stride(1)] + ([value_cache.stride(1)] if value_cache is not None else [])
    if max(tok_strides) * 2 * AL.KEY_BLOCK >= 1 << 31:
        return False
    if num_reqs is not None and (num_reqs < 1 or num_reqs * num_kv_heads > 65535 or num_reqs * Q * H > 0x7FFFFFFF):
        return False
    return True


def gqa_packed_spec_attention(query, key_cache, value_cache, out, seq_lens, block_table, num_reqs, Q, num_kv_heads,
                              scale, num_splits=DEFAULT_NUM_SPLITS, min_chunk=DEFAULT_MIN_CHUNK, block_n=32,
                              num_warps=4, num_stages=2, combine_warps=2):
    """query/out [>= num_reqs*Q, H, D] bf16; key_cache/value_cache [num_blocks, PAGE, H_kv, D] bf16 (strided
    views are fine); seq_lens int32 [num_reqs]; block_table int32 [num_reqs, max_blocks].  num_splits None:
    one prefix workgroup per compute unit.  Returns out."""
    del block_n, num_warps, num_stages, combine_warps
    for t, n in ((query, "query"), (key_cache, "key_cache"), (value_cache, "value_cache"), (out, "out")):
        _check_bf16_rows(t, n)
    if seq_lens.dtype != torch.int32 or block_table.dtype != torch.int32:
        raise TypeError("seq_lens and block_table must be int32")
    if block_table.stride(-1) != 1:
        raise ValueError("block_table must be contiguous in its last dimension")
    B = int(num_reqs)
    H, D = query.shape[1], query.shape[2]
    if out.shape[1] != H or out.shape[2] != D or key_cache.shape[3] != D or value_cache.shape[3] != D:
        raise ValueError("query, out and the caches must share the head size and head count")
    if key_cache.shape[2] != num_kv_heads or value_cache.shape[2] != num_kv_heads:
        raise ValueError("cache kv-head count does not match num_kv_heads")
    if query.shape[0] < B * Q or out.shape[0] < B * Q or seq_lens.numel() < B or block_table.shape[0] < B:
        raise ValueError("batch tensors are smaller than num_reqs * Q")
    page = key_cache.shape[1]
    if num_splits is None:
        num_splits = auto_num_splits(query.device, B, num_kv_heads)
    L = AL.load()
    ws_bytes = AL.workspace_bytes(B, Q, H, num_kv_heads, D, num_splits)
    if ws_bytes == 0:
        raise ValueError("invalid attention sizes")
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=query.device)
    stream = torch.cuda.current_stream(query.device).cuda_stream
    rc = L.qf_spec_attention(
        query.data_ptr(), query.stride(0), query.stride(1),
        key_cache.data_ptr(), key_cache.stride(0), key_cache.stride(1), key_cache.stride(2),
        value_cache.data_ptr(), value_cache.stride(0), value_cache.stride(1), value_cache.stride(2),
        block_table.data_ptr(), block_table.stride(0), seq_lens.data_ptr(),
        out.data_ptr(), out.stride(0), out.stride(1),
        B, int(Q), H, int(num_kv_heads), D, page, float(scale), int(num_splits), int(min_chunk),
        ws.data_ptr(), ws_bytes, stream)
    AL.check(rc, "qf_spec_attention")
    return out
