"""Plugin surface of the decode fast paths (reference: plugin/qwen_fastpath/patches.py:10-189).

* ``patch_flash_attention`` -- routes uniform speculative-verification batches (every request has the
  same 1 < Q <= 8 query tokens) of an eligible attention layer to the split-KV, GQA-packed kernel
  (patches.py:10-69); everything else stays on the original forward.

* ``qf_int8_linear`` -- the dispatcher op (patches.py:84-106): M <= 16 bf16 activations on an int8
  weight with stride(0) == 1 and one fp32 scale per output channel go to the HIP W8A16 kernel;
  anything else goes to the W8A8 path the reference falls back to, except on TILED layers, whose
  M > 16 calls run the wide-M W8A16 kernel (up to TILED_WIDE_MAX_M rows) or the widened-weights
  library GEMM.
* ``patch_int8_linear`` -- swaps ``apply_weights(self, layer, x, bias)`` of vLLM's int8 scaled-mm
  kernel class (patches.py:72-116); ``W8A16LinearMethod.apply(layer, x, bias)`` is the same surface
  for callers that hold the layer directly.
* ``patch_draft_lm_head`` / ``quantize_lm_head`` / ``int8_logits`` / ``top_tokens`` -- the int8 MTP
  draft head (patches.py:119-189), running the same kernel form over a per-row int8 copy of the
  lm_head.

vLLM is an optional dependency: with vLLM absent the patch functions return False and log; the
ops, ``W8A16LinearMethod`` and the draft-head helpers work on plain tensors.
"""
from __future__ import annotations

import logging
import os
from typing import Callable, NamedTuple, Optional

import torch

from . import _lib as L
from .w8a16 import (ROWMAJOR, SMALL_M, TILED, _workspace, from_tiled, pick_config, to_tiled, w8a16_mm,
                    w8a16_mm_argmax, w8a16_mm_prefill, w8a8_mm)

logger = logging.getLogger("vllm.qwen_fastpath")

MAX_SPEC_QUERY_LEN = 8  # patches.py:7


# ------------------------------------------------------------------------------------------------
# verification attention (patches.py:10-69)
# ------------------------------------------------------------------------------------------------

def attn_switch_enabled() -> bool:
    """QWEN_FAST_ATTN, default "1" (plugin/qwen_fastpath/__init__.py:23)."""
    return os.environ.get("QWEN_FAST_ATTN", "1") == "1"


def _interleaved_kv_split(kv_cache: torch.Tensor, head_size: int):
    """The layer's cache as the reference reads it (patches.py:59): [blocks, H_kv, PAGE, 2D] with K
    and V interleaved per row, viewed as two [blocks, PAGE, H_kv, D] tensors.  None for another shape."""
    if kv_cache is None or kv_cache.dim() != 4 or kv_cache.shape[-1] != 2 * head_size:
        return None
    return kv_cache.transpose(1, 2).split(head_size, dim=-1)


def _stacked_kv_split(kv_cache: torch.Tensor, head_size: int):
    """A cache of shape [2, blocks, PAGE, H_kv, D] whose memory is laid out as its shape says (K then V,
    each [blocks][PAGE][H_kv][D]; vLLM's FlashAttention and ROCm AITER FlashAttention backends read it
    with ``kv_cache.unbind(0)``).  None for another shape."""
    if kv_cache is None or kv_cache.dim() != 5 or kv_cache.shape[0] != 2 or kv_cache.shape[-1] != head_size:
        return None
    return kv_cache.unbind(0)


def _paired_kv_split(kv_cache: torch.Tensor, head_size: int):
    """A cache of shape [blocks, 2, PAGE, H_kv, D] (K and V pages side by side per block; vLLM's Triton
    attention backend, the default on ROCm, reads it with ``kv_cache.unbind(1)``).  None for another
    shape."""
    if kv_cache is None or kv_cache.dim() != 5 or kv_cache.shape[1] != 2 or kv_cache.shape[-1] != head_size:
        return None
    return kv_cache.unbind(1)


def _flash_attn_kv_split(kv_cache: torch.Tensor, head_size: int):
    """vLLM's FlashAttention cache: the reference's interleaved 4-D layout, or the stacked 5-D one."""
    if kv_cache is not None and kv_cache.dim() == 5:
        return _stacked_kv_split(kv_cache, head_size)
    return _interleaved_kv_split(kv_cache, head_size)


def attn_impl_eligible(impl) -> bool:
    """The reference's per-layer predicate (patches.py:24-44), evaluated once per layer object;
    attributes a backend class does not define count as their neutral value."""
    ok = getattr(impl, "_qf_eligible", None)
    if ok is not None:
        return ok
    attn_type = getattr(impl, "attn_type", "decoder")
    decoder = str(getattr(attn_type, "value", attn_type)).lower() == "decoder"
    quantized = str(getattr(impl, "kv_cache_dtype", "auto")).startswith("fp8")
    window = getattr(impl, "sliding_window", None)
    ok = (decoder
          and getattr(impl, "dcp_world_size", 1) == 1
          and getattr(impl, "vllm_flash_attn_version", 2) == 2
          and not getattr(impl, "fa4_hd256", False)
          and (window is None or tuple(window) == (-1, -1))
          and getattr(impl, "alibi_slopes", None) is None
          and not getattr(impl, "logits_soft_cap", None)
          and getattr(impl, "sinks", None) is None
          and not quantized
          and impl.num_heads % impl.num_kv_heads == 0
          and impl.head_size in (64, 128, 256)
          and getattr(impl, "kv_sharing_target_layer_name", None) is None)
    impl._qf_eligible = ok
    return ok


def spec_batch_q_len(md) -> Optional[int]:
    """Q when the metadata describes a uniform verification batch the kernel serves (patches.py:49-58),
    else None."""
    if md is None or getattr(md, "causal", True) is not True or getattr(md, "use_cascade", False):
        return None
    if getattr(md, "mm_prefix_query_range_tensor", None) is not None or getattr(md, "rswa_prefix_lens", None) is not None:
        return None
    q_len = int(md.max_query_len)
    if not 1 < q_len <= MAX_SPEC_QUERY_LEN:
        return None
    num_reqs = md.query_start_loc.shape[0] - 1
    if md.num_actual_tokens != num_reqs * q_len:  # uniform: every request has exactly q_len tokens
        return None
    return q_len


def make_attention_forward(orig_forward: Callable, split_kv_cache: Callable = _interleaved_kv_split) -> Callable:
    """Replacement for ``forward(self, layer, query, key, value, kv_cache, attn_metadata, output,
    output_scale=None, output_block_scale=None)`` of an attention implementation class.
    ``split_kv_cache(kv_cache, head_size)`` returns the (key, value) [blocks, PAGE, H_kv, D] views of the
    layer's cache, or None when the cache is not in the layout it reads (the call then stays on the
    original forward)."""
    from .spec_attn import gqa_packed_spec_attention, supported

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output,
                output_scale=None, output_block_scale=None):
        md = attn_metadata
        q_len = spec_batch_q_len(md) if output_scale is None and output_block_scale is None else None
        if q_len is not None and attn_impl_eligible(self):
            num_reqs = md.query_start_loc.shape[0] - 1
            kv = split_kv_cache(kv_cache, self.head_size) if output is not None else None
            if kv is not None:
                key_cache, value_cache = kv
                q3 = query.view(query.shape[0], self.num_heads, self.head_size)
                o3 = output.view(output.shape[0], self.num_heads, self.head_size)
            if kv is not None and supported(q3, key_cache, q_len, self.num_kv_heads, value_cache, o3, num_reqs):
                gqa_packed_spec_attention(q3, key_cache, value_cache, o3, md.seq_lens, md.block_table,
                                          num_reqs, q_len, self.num_kv_heads, self.scale)
                return output
        return orig_forward(self, layer, query, key, value, kv_cache, attn_metadata, output,
                            output_scale, output_block_scale)

    forward._qwen_fastpath = True
    return forward


# The attention implementations patched by default, each with the adapter that reads its cache layout.
# FlashAttention is the class the reference patches (patches.py:13); on ROCm vLLM runs Triton attention
# by default, or AITER FlashAttention when AITER is enabled.  ROCm's paged-attention backend
# (rocm_attn:RocmAttentionImpl) is not listed: its cache keeps the legacy paged layout under a 5-D shape
# (each K row cut into 16-byte groups strided by the page, V stored transposed), which the kernel does
# not read.  An entry may also be a bare "module:Class" string, read with the reference's layout.
VLLM_ATTENTION_CLASSES = (
    ("vllm.v1.attention.backends.flash_attn:FlashAttentionImpl", _flash_attn_kv_split),
    ("vllm.v1.attention.backends.triton_attn:TritonAttentionImpl", _paired_kv_split),
    ("vllm.v1.attention.backends.rocm_aiter_fa:AiterFlashAttentionImpl", _stacked_kv_split),
)


def patch_flash_attention(impl_cls=None, split_kv_cache: Optional[Callable] = None) -> bool:
    """Install the verification-attention path on ``impl_cls``, or by default on every class of
    VLLM_ATTENTION_CLASSES that imports (the reference patches vLLM's FlashAttention implementation,
    patches.py:10-69).  Idempotent.  ``split_kv_cache(kv_cache, head_size) -> (key_cache, value_cache) or
    None`` gives the [blocks, PAGE, H_kv, D] views of the layer's cache (default for an explicit class:
    the reference's interleaved layout).  Returns False when no class could be patched."""
    classes = []
    if impl_cls is not None:
        classes.append((impl_cls, split_kv_cache or _interleaved_kv_split))
    else:
        for entry in VLLM_ATTENTION_CLASSES:
            path, adapter = (entry, _interleaved_kv_split) if isinstance(entry, str) else entry
            try:
                classes.append((_import_attr(path), split_kv_cache or adapter))
            except (ImportError, AttributeError, RuntimeError, OSError) as e:  # backend absent on this platform
                logger.debug("qwen_fastpath: %s not patched: %s", path, e)
                continue
    if not classes:
        logger.info("qwen_fastpath: vLLM attention implementation not found; split-KV attention available as "
                    "qwen_fastpath.gqa_packed_spec_attention only")
        return False
    for cls, adapter in classes:
        orig = cls.forward
        if not getattr(orig, "_qwen_fastpath", False):
            cls.forward = make_attention_forward(orig, adapter)
    logger.info("qwen_fastpath: split-KV GQA-packed attention enabled for speculative-decode verification")
    return True


def linear_switch_enabled() -> bool:
    """QWEN_FAST_LINEAR, default "1" (plugin/qwen_fastpath/__init__.py:25)."""
    return os.environ.get("QWEN_FAST_LINEAR", "1") == "1"


def draft_head_switch_enabled() -> bool:
    """QWEN_FAST_DRAFT_HEAD, default "1" (plugin/qwen_fastpath/__init__.py:27)."""
    return os.environ.get("QWEN_FAST_DRAFT_HEAD", "1") == "1"


# ------------------------------------------------------------------------------------------------
# W8A8 fallback (M > 16 or ineligible inputs on row-major layers)
# ------------------------------------------------------------------------------------------------

def _vllm_w8a8() -> Optional[Callable]:
    try:
        from vllm import _custom_ops as ops  # type: ignore
    except ImportError:
        return None

    def run(x2, w_q, w_s, bias, out_dtype):
        x_q, x_s, _ = ops.scaled_int8_quant(x2.contiguous(), None, None, symmetric=True)
        return ops.cutlass_scaled_mm(x_q, w_q, scale_a=x_s, scale_b=w_s, out_dtype=out_dtype, bias=bias)

    return run


def _int8_products(x_q: torch.Tensor, w_q: torch.Tensor) -> torch.Tensor:
    """fp32(x_q @ w_q) for integer-valued x_q in [-128, 127] and int8 w_q [K, N]: the exact integer
    sums rounded once to fp32.  On the GPU with M > 16 and K, N multiples of 8 the int8 GEMM of the
    library (torch._int_mm, int32 accumulation: |sum| <= K * 128 * 127 < 2^31 for K < 132000) gives them;
    otherwise an fp64 product does (sums of at most 2^53 are exact)."""
    M, K = x_q.shape
    N = w_q.shape[1]
    if x_q.is_cuda and M > 16 and K % 8 == 0 and N % 8 == 0 and K < 132000:
        try:
            return torch._int_mm(x_q.to(torch.int8), w_q).float()
        except RuntimeError:
            pass
    return (x_q.double() @ w_q.double()).float()


def w8a8_reference(x2: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor, bias: Optional[torch.Tensor],
                   out_dtype: torch.dtype) -> torch.Tensor:
    """Dynamic per-token symmetric int8 activations x int8 weights, exact integer accumulation, then
    fp32 scale_a * scale_b epilogue and optional bias -- the semantics of the scaled_int8_quant +
    cutlass_scaled_mm pair the reference falls back to (patches.py:99-100).  Used when vLLM is not
    installed; accuracy is pinned only by the reference's published W8A8 error statistic."""
    xf = x2.float()
    s_a = xf.abs().amax(dim=-1, keepdim=True) / 127.0
    x_q = torch.where(s_a > 0, torch.round(xf / torch.where(s_a > 0, s_a, torch.ones_like(s_a))),
                      torch.zeros_like(xf)).clamp_(-128, 127)
    acc = _int8_products(x_q, w_q)
    y = acc * s_a * w_s.reshape(1, -1).float()
    if bias is not None:
        y = y + bias.float()
    return y.to(out_dtype)


_fallback_impl: Optional[Callable] = None
TILED_WIDE_MAX_M = 1024


def prefill_arithmetic() -> str:
    """QWEN_FAST_LINEAR_PREFILL: the arithmetic of M > 16 calls on TILED layers.  "w8a8" (default) is the
    reference's own M > 16 arithmetic (per-token int8 activations, exact integer sums:
    scaled_int8_quant + cutlass_scaled_mm, patches.py:99-100) on the int8 MFMA; "w8a16" keeps the decode
    path's arithmetic (exact bf16 products, fp32 sums) at every M."""
    v = os.environ.get("QWEN_FAST_LINEAR_PREFILL", "w8a8").strip().lower()
    if v not in ("w8a8", "w8a16"):
        raise ValueError(f"QWEN_FAST_LINEAR_PREFILL must be w8a8 or w8a16, got {v!r}")
    return v


def _fallback(x2, w_q, w_s, bias, out_dtype, layout):
    if layout == TILED and x2.dtype != torch.bfloat16:
        # The library's kernels take bf16 activations.  Others (fp16 models) get the reference's W8A8
        # arithmetic restated in torch over the row-major weights recovered from the image (exact).
        N = w_s.numel()
        return w8a8_reference(x2, from_tiled(w_q, N, x2.shape[1]), w_s.reshape(-1).float(), bias, out_dtype)
    if layout == TILED and prefill_arithmetic() == "w8a8":
        # The reference's M > 16 arithmetic, on the TILED image CUTLASS cannot read: per-token int8
        # activations times the int8 weights on v_mfma_i32_16x16x64_i8 (gate_up M = 512: 169 us,
        # M = 2048: 565 us, against 241 / 723 us for the W8A16 routes below).
        y = w8a8_mm(x2, w_q, w_s.reshape(-1), out_dtype)
        return y if bias is None else y + bias
    if layout == TILED:
        # No W8A8 library kernel reads the permuted image.  Up to TILED_WIDE_MAX_M rows the wide-M
        # kernel runs (one launch, each weight fragment feeding up to 64 token rows); above, the
        # weights are widened to bf16 for a library bf16 GEMM (fp32 accumulation, scale after the K
        # reduction), whose MFMA tiles win once the product is that large.  Measured on the dense
        # 27B-class layer (gate_up / qkv / o_proj / down): at M = 1024 the wide kernel takes
        # 403 / 133 / 123 / 252 us against 478 / 136 / 116 / 277 us widened, at M = 2048
        # 806 / 241 / 205 / 427 us against 741 / 233 / 175 / 338 us.
        if x2.shape[0] <= TILED_WIDE_MAX_M:
            y = w8a16_mm(x2, w_q, w_s.reshape(-1), None, out_dtype, layout)
        else:
            y = w8a16_mm_prefill(x2.contiguous(), w_q, w_s, out_dtype, TILED)
        return y if bias is None else y + bias
    global _fallback_impl
    if _fallback_impl is None:
        _fallback_impl = _vllm_w8a8() or _w8a8_hip
    return _fallback_impl(x2, w_q, w_s, bias, out_dtype)


def _w8a8_hip(x2, w_q, w_s, bias, out_dtype):
    """Without vLLM: the same W8A8 arithmetic on the int8 MFMA (w8a8_mm on the row-major weight) when the
    library serves the shape -- K % 64 == 0, the [K, N] stride-(1, K) view, bf16 activations -- and the
    torch restatement otherwise, as the reference falls back when pick_config returns None."""
    M, K = x2.shape
    N = w_s.numel()
    if (x2.dtype == torch.bfloat16 and out_dtype in (torch.bfloat16, torch.float32) and w_q.dim() == 2
            and w_q.shape == (K, N) and w_q.stride(0) == 1 and w_q.stride(1) % 16 == 0 and w_q.data_ptr() % 16 == 0
            and w_q.is_cuda and w_s.dtype == torch.float32 and pick_config(N, K, ROWMAJOR) is not None):
        y = w8a8_mm(x2, w_q, w_s.reshape(-1), out_dtype, layout=ROWMAJOR)
        return y if bias is None else y + bias
    return w8a8_reference(x2, w_q, w_s, bias, out_dtype)


# ------------------------------------------------------------------------------------------------
# dispatcher op (patches.py:84-106)
# ------------------------------------------------------------------------------------------------

def weight_layout(w_q: torch.Tensor) -> int:
    """The layout a weight tensor holds: the TILED image is 1-D (to_tiled), the checkpoint's row-major
    weight the 2-D [K, N] view with stride (1, K) (w8a16.py:72)."""
    return TILED if w_q.dim() == 1 else ROWMAJOR


def out_features(w_q: torch.Tensor, w_s: torch.Tensor) -> int:
    """N: the [K, N] view's second dimension, or one per scale for the TILED image."""
    return w_s.numel() if w_q.dim() == 1 else w_q.shape[1]


def shape_eligible(x2: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor, layout: Optional[int] = None) -> bool:
    """The reference's predicate (patches.py:90-92): M <= SMALL_M, bf16 activations, w_q.stride(0) == 1
    (the [K, N] view of the row-major weight; the TILED image has no such stride), one scale per output
    channel, and a configuration for (N, K) (None when K % 64 != 0)."""
    layout = weight_layout(w_q) if layout is None else layout
    M, K = x2.shape
    if layout == ROWMAJOR:
        N = w_q.shape[1]
        layout_ok = w_q.stride(0) == 1
    else:
        N = w_s.numel()
        layout_ok = True
    return (M <= SMALL_M and x2.dtype == torch.bfloat16 and layout_ok and w_s.numel() == N
            and pick_config(N, K, layout) is not None)


def eligible(x2: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor, layout: Optional[int] = None) -> bool:
    """shape_eligible, and the tensors live on the GPU."""
    return x2.is_cuda and shape_eligible(x2, w_q, w_s, layout)


def _qf_int8_linear_impl(x: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor,
                         bias: Optional[torch.Tensor]) -> torch.Tensor:
    layout = weight_layout(w_q)
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    N = out_features(w_q, w_s)
    if x2.shape[0] == 0:  # no tokens
        y = x.new_empty((*lead, N))
        return y if bias is None else y + bias
    if eligible(x2, w_q, w_s, layout):
        if x2.stride(-1) != 1:
            x2 = x2.contiguous()
        s = w_s.reshape(-1)
        if s.dtype != torch.float32:
            s = s.float()
        y = w8a16_mm(x2, w_q, s, None, x.dtype, layout)
        if bias is not None:
            y = y + bias
        return y.view(*lead, N)
    y = _fallback(x2, w_q, w_s, bias, x.dtype, layout)
    return y.view(*lead, N)


def _qf_int8_linear_fake(x, w_q, w_s, bias):
    return x.new_empty((*x.shape[:-1], out_features(w_q, w_s)))


def _define_op(qualname: str):
    op = torch.library.custom_op(qualname, mutates_args=())(_op_body)
    op.register_fake(_qf_int8_linear_fake)
    return op


def _op_body(x: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor, bias: Optional[torch.Tensor]) -> torch.Tensor:
    """qf_int8_linear(x, w_q, w_s, bias): y [..., N] in x.dtype.  w_q is the [K, N] stride-(1, K) view of
    the checkpoint's int8 weight, or its TILED image (1-D); w_s holds the N fp32 per-channel scales."""
    return _qf_int8_linear_impl(x, w_q, w_s, bias)


# torch.ops.vllm.qf_int8_linear(x, w_q, w_s, bias): the reference's op (patches.py:84-106, registered
# there with vLLM's direct_register_custom_op), one opaque node under torch.compile with a fake impl;
# torch.ops.qwen_fastpath.qf_int8_linear is the same op under this package's namespace.
qf_int8_linear = _define_op("qwen_fastpath::qf_int8_linear")
try:
    qf_int8_linear_vllm = _define_op("vllm::qf_int8_linear")
except RuntimeError as e:  # another plugin already defined it
    qf_int8_linear_vllm = None
    logger.warning("qwen_fastpath: vllm::qf_int8_linear already defined (%s); using qwen_fastpath::qf_int8_linear", e)


def _linear_op():
    """The op the patched surfaces call: vllm::qf_int8_linear when this package defined it."""
    return torch.ops.vllm.qf_int8_linear if qf_int8_linear_vllm is not None else torch.ops.qwen_fastpath.qf_int8_linear


# ------------------------------------------------------------------------------------------------
# linear-layer surfaces (patches.py:108-116)
# ------------------------------------------------------------------------------------------------

def make_apply_weights(orig_apply: Callable) -> Callable:
    """Replacement for ``apply_weights(self, layer, x, bias=None)`` of an int8 scaled-mm kernel class
    whose ``_get_layer_params(layer)`` returns (w_q, w_s, i_s, i_zp, azp_adj)."""

    def apply_weights(self, layer, x, bias=None):
        w_q, w_s, i_s, i_zp, azp_adj = self._get_layer_params(layer)
        if i_s is None and i_zp is None and azp_adj is None:  # dynamic symmetric per-token
            return _linear_op()(x, w_q, w_s, bias)
        return orig_apply(self, layer, x, bias)

    apply_weights._qwen_fastpath = True
    return apply_weights


# vLLM classes whose apply_weights serve int8 W8A8 linears: the reference's CUTLASS class first,
# then the ROCm-side implementations of the same interface.
VLLM_INT8_KERNEL_CLASSES = (
    "vllm.model_executor.kernels.linear.scaled_mm.cutlass:CutlassInt8ScaledMMLinearKernel",
    "vllm.model_executor.layers.quantization.kernels.scaled_mm.cutlass:CutlassScaledMMLinearKernel",
    "vllm.model_executor.layers.quantization.kernels.scaled_mm.triton:TritonScaledMMLinearKernel",
    "vllm.model_executor.layers.quantization.kernels.scaled_mm.aiter:AiterScaledMMLinearKernel",
)


def _import_attr(path: str):
    mod, _, attr = path.partition(":")
    import importlib
    return getattr(importlib.import_module(mod), attr)


def tiled_layout_requested() -> bool:
    """QWEN_FAST_LINEAR_LAYOUT: "tiled" (default) repacks W8A8 linear weights into the TILED image at load
    time, in place of the row-major copy; "rowmajor" keeps the checkpoint layout, as the reference does
    (plugin/qwen_fastpath/w8a16.py:1-7)."""
    v = os.environ.get("QWEN_FAST_LINEAR_LAYOUT", "tiled").strip().lower()
    if v not in ("tiled", "rowmajor"):
        raise ValueError(f"QWEN_FAST_LINEAR_LAYOUT must be tiled or rowmajor, got {v!r}")
    return v == "tiled"


def repack_layer_weight(layer) -> bool:
    """Replace a dynamic-per-token int8 layer's [K, N] (stride (1, K)) weight by its TILED image, in
    place of the row-major copy (one weight copy is kept), and tag the layer.  Returns False and
    leaves the layer unchanged when it is not an eligible int8 layer."""
    w = getattr(layer, "weight", None)
    if getattr(layer, "_qf_layout", ROWMAJOR) == TILED:
        return True
    if w is None or w.dtype != torch.int8 or w.dim() != 2 or not w.is_cuda or w.stride(0) != 1:
        return False
    if any(getattr(layer, n, None) is not None for n in ("input_scale", "input_zero_point", "azp_adj")):
        return False
    # the image serves bf16 activations; a model in another dtype keeps the layout its fallback reads
    if getattr(layer, "params_dtype", torch.bfloat16) != torch.bfloat16:
        return False
    K, N = w.shape
    if pick_config(N, K, TILED) is None:
        return False
    img = to_tiled(w.detach())
    layer.weight = torch.nn.Parameter(img, requires_grad=False)
    layer._qf_layout = TILED
    return True


def make_process_weights_after_loading(orig: Callable) -> Callable:
    """Wrap a kernel class's ``process_weights_after_loading(self, layer)`` so that, once the
    original has laid the int8 weight out as [K, N] column-major (the CUTLASS view), the weight is
    repacked into the TILED image.  No reference counterpart: the reference streams the checkpoint
    layout as is (plugin/qwen_fastpath/w8a16.py:1-7)."""

    def process_weights_after_loading(self, layer):
        orig(self, layer)
        repack_layer_weight(layer)

    process_weights_after_loading._qwen_fastpath = True
    return process_weights_after_loading


def patch_int8_linear(kernel_cls=None, tiled: Optional[bool] = None) -> bool:
    """Install the W8A16 decode path on ``kernel_cls`` (default: vLLM's int8 scaled-mm kernel
    classes).  Idempotent (patches.py:80-82).  Returns False when no class could be patched.
    With ``tiled`` (default: QWEN_FAST_LINEAR_LAYOUT=tiled) the weights are also repacked into the
    TILED image after loading; M > 16 calls on such layers run the reference's W8A8 arithmetic on the
    int8 MFMA (w8a8_mm), or with QWEN_FAST_LINEAR_PREFILL=w8a16 the wide-M W8A16 kernel up to
    TILED_WIDE_MAX_M rows and a bf16 library GEMM over exactly widened weights above."""
    tiled = tiled_layout_requested() if tiled is None else bool(tiled)
    classes = [kernel_cls] if kernel_cls is not None else []
    if kernel_cls is None:
        for path in VLLM_INT8_KERNEL_CLASSES:
            try:
                classes.append(_import_attr(path))
            except (ImportError, AttributeError):
                continue
    if not classes:
        logger.info("qwen_fastpath: vLLM int8 linear kernel classes not found; W8A16 op available as "
                    "torch.ops.qwen_fastpath.qf_int8_linear only")
        return False
    for cls in classes:
        orig = cls.apply_weights
        if not getattr(orig, "_qwen_fastpath", False):
            cls.apply_weights = make_apply_weights(orig)
        pw = getattr(cls, "process_weights_after_loading", None)
        if tiled and pw is not None and not getattr(pw, "_qwen_fastpath", False):
            cls.process_weights_after_loading = make_process_weights_after_loading(pw)
    logger.info("qwen_fastpath: W8A16 decode path for W8A8-int8 linears (M <= %d), W8A8 above", SMALL_M)
    return True


class W8A16LinearMethod:
    """vLLM LinearMethod-style surface ``apply(layer, x, bias=None)`` over a W8A8 int8 layer.

    The layer holds ``weight`` (int8 [K, N] with stride(0) == 1, or the TILED image when
    ``layer._qf_layout == TILED``), ``weight_scale`` (fp32, N values) and optionally
    ``input_scale`` / ``input_zero_point`` / ``azp_adj`` (static or asymmetric activation
    quantisation, which keeps the original path).  The QWEN_FAST_LINEAR switch is read once at
    construction; "0" routes every call to ``fallback``."""

    def __init__(self, fallback: Optional[Callable] = None, enabled: Optional[bool] = None):
        self.enabled = linear_switch_enabled() if enabled is None else bool(enabled)
        self.fallback = fallback

    def _original(self, layer, x, bias):
        if self.fallback is not None:
            return self.fallback(layer, x, bias)
        x2 = x.reshape(-1, x.shape[-1])
        y = _fallback(x2, layer.weight, layer.weight_scale, bias, x.dtype, weight_layout(layer.weight))
        return y.view(*x.shape[:-1], y.shape[-1])

    def apply(self, layer, x: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        dynamic = all(getattr(layer, n, None) is None for n in ("input_scale", "input_zero_point", "azp_adj"))
        if self.enabled and dynamic:
            return _linear_op()(x, layer.weight, layer.weight_scale, bias)
        return self._original(layer, x, bias)


# ------------------------------------------------------------------------------------------------
# int8 MTP draft head (patches.py:119-189)
# ------------------------------------------------------------------------------------------------

class Int8Head(NamedTuple):
    """What the reference stores as draft_model._qf_head_i8 (patches.py:149)."""

    w_t: torch.Tensor      # int8 [H, V] view with stride (1, H) of the [V, H] quantised head, or its
                           # TILED image (layout == TILED)
    scale: torch.Tensor    # fp32 [V]
    num_pad: int           # padded vocabulary rows at the end
    cfg: object            # pick_config(V, H)
    layout: int = ROWMAJOR


def quantize_lm_head(weight: torch.Tensor):
    """Per-row int8 copy of a bf16 [V, H] lm_head on the GPU (HIP kernel; patches.py:139-147):
    s = max(amax|row|, 1e-8) / 127, q = clamp(round_half_even(row / s), -127, 127).
    Returns (w8 [V, H] int8, scale [V] fp32)."""
    if weight.dtype != torch.bfloat16 or weight.dim() != 2 or not weight.is_cuda:
        raise TypeError("quantize_lm_head expects a 2-D bf16 CUDA tensor")
    if weight.stride(1) != 1:
        weight = weight.contiguous()
    V, H = weight.shape
    w8 = torch.empty((V, H), dtype=torch.int8, device=weight.device)
    scale = torch.empty((V,), dtype=torch.float32, device=weight.device)
    stream = torch.cuda.current_stream(weight.device).cuda_stream
    L.check(L.load().qf_quantize_rows_int8(weight.data_ptr(), weight.stride(0), w8.data_ptr(), scale.data_ptr(),
                                           V, H, stream), "qf_quantize_rows_int8")
    return w8, scale


def make_int8_head(weight: torch.Tensor, num_pad: int = 0, layout: int = TILED) -> Int8Head:
    """The draft head's int8 copy.  The copy is this plugin's own (the checkpoint's bf16 head is left
    as it is), so it is kept in the TILED layout the kernel streams fastest; layout=ROWMAJOR keeps the
    reference's [V, H] row-major copy (patches.py:149)."""
    w8, scale = quantize_lm_head(weight)
    V, H = w8.shape
    cfg = pick_config(V, H, layout)
    if layout == TILED and cfg is not None:
        w_img = to_tiled(w8.t())
        del w8
        return Int8Head(w_img, scale, int(num_pad), cfg, TILED)
    return Int8Head(w8.t(), scale, int(num_pad), pick_config(V, H), ROWMAJOR)


def int8_logits(head: Optional[Int8Head], hidden_states: torch.Tensor, logits_as_input: bool = False,
                soft_cap=None, scale: float = 1.0, draft_id_to_target_id=None) -> Optional[torch.Tensor]:
    """Draft logits through the W8A16 kernel, or None when the guard of patches.py:160-163 fails
    (the caller then uses the bf16 head)."""
    if (head is None or hidden_states.dim() != 2 or hidden_states.shape[0] > SMALL_M
            or hidden_states.dtype != torch.bfloat16 or logits_as_input or soft_cap is not None
            or scale != 1.0 or draft_id_to_target_id is not None or head.cfg is None):
        return None
    x = hidden_states if hidden_states.stride(-1) == 1 else hidden_states.contiguous()
    return w8a16_mm(x, head.w_t, head.scale, head.cfg, torch.bfloat16, head.layout)


def int8_top_tokens(head: Optional[Int8Head], hidden_states: torch.Tensor, vocab_start: int = 0,
                    logits_as_input: bool = False, soft_cap=None, scale: float = 1.0,
                    draft_id_to_target_id=None, fused: bool = True) -> Optional[torch.Tensor]:
    """Draft token ids of the int8 head (patches.py:178-185); None when the guard of int8_logits fails.
    Two ways, same ids: the W8A16 logits, then the pad-masked argmax over them (two launches); or the
    argmax folded into the GEMM's epilogue (qf_w8a16_gemm_argmax: the logits are neither written nor
    re-read; a one-wavefront launch per token reads the folded slots; the default).  Measured on MI355X for
    the 151936 x 5120 head: 117.2 us fused vs 121.2 us two-launch at M = 1, 124.4 vs 128.0 us at M = 4.
    Shapes the fused path does not serve take the two-launch path."""
    if (head is None or hidden_states.dim() != 2 or hidden_states.shape[0] > SMALL_M
            or hidden_states.dtype != torch.bfloat16 or logits_as_input or soft_cap is not None
            or scale != 1.0 or draft_id_to_target_id is not None or head.cfg is None):
        return None
    x = hidden_states if hidden_states.stride(-1) == 1 else hidden_states.contiguous()
    n_valid = head.scale.numel() - int(head.num_pad)
    ids = w8a16_mm_argmax(x, head.w_t, head.scale, n_valid, vocab_start, head.cfg, head.layout) if fused else None
    if ids is None:
        ids = top_tokens(w8a16_mm(x, head.w_t, head.scale, head.cfg, torch.bfloat16, head.layout),
                         head.num_pad, vocab_start)
    return ids


def top_tokens(logits: torch.Tensor, num_pad: int = 0, vocab_start: int = 0) -> torch.Tensor:
    """argmax over the vocabulary with the last num_pad columns treated as -inf, plus the vocabulary
    start index (patches.py:182-185); HIP kernel, torch.argmax tie/NaN semantics."""
    if logits.dtype != torch.bfloat16 or logits.dim() != 2 or logits.stride(1) != 1:
        raise TypeError("top_tokens expects 2-D bf16 logits with unit column stride")
    M, N = logits.shape
    out = torch.empty((M,), dtype=torch.int64, device=logits.device)
    lib = L.load()
    ws = _workspace(logits.device, int(lib.qf_argmax_rows_workspace_bytes()))
    stream = torch.cuda.current_stream(logits.device).cuda_stream
    L.check(lib.qf_argmax_rows_bf16_ws(logits.data_ptr(), logits.stride(0) if M > 1 else N, M, N, N - int(num_pad),
                                       int(vocab_start), out.data_ptr(), ws.data_ptr(), ws.numel(), stream),
            "qf_argmax_rows_bf16_ws")
    return out


def patch_draft_lm_head(speculator_cls=None, mtp_cls=None) -> bool:
    """Give the MTP drafter an int8 per-row lm_head (patches.py:119-189).  With vLLM absent and no
    classes passed, returns False.  The classes need: speculator.load_draft_model(target_model,
    target_attn_layer_names) -> draft_model; draft_model.lm_head.weight / .tp_size /
    .shard_indices.(num_org_vocab_padding, org_vocab_start_index); draft_model.logits_processor
    with logits_as_input / soft_cap / scale / org_vocab_size; compute_logits / get_top_tokens."""
    if speculator_cls is None or mtp_cls is None:
        try:
            from vllm.model_executor.models import qwen3_5_mtp  # type: ignore
            from vllm.v1.worker.gpu.spec_decode.mtp.speculator import MTPSpeculator  # type: ignore
        except ImportError:
            logger.info("qwen_fastpath: vLLM MTP classes not found; int8 draft head helpers only")
            return False
        speculator_cls = speculator_cls or MTPSpeculator
        mtp_cls = mtp_cls or qwen3_5_mtp.Qwen3_5MTP

    orig_load = speculator_cls.load_draft_model
    if getattr(orig_load, "_qwen_fastpath", False):
        return True

    def load_draft_model(self, target_model, target_attn_layer_names):
        draft_model = orig_load(self, target_model, target_attn_layer_names)
        lm_head = getattr(draft_model, "lm_head", None)
        weight = getattr(lm_head, "weight", None)
        if (isinstance(draft_model, mtp_cls) and weight is not None and weight.dim() == 2
                and getattr(lm_head, "tp_size", 1) == 1):
            num_pad = lm_head.shard_indices.num_org_vocab_padding
            draft_model._qf_head_i8 = make_int8_head(weight, num_pad)
            logger.info("qwen_fastpath: int8 draft lm_head (%d x %d, %.2f GB) for MTP proposals",
                        weight.shape[0], weight.shape[1], weight.numel() / 1e9)
        return draft_model

    load_draft_model._qwen_fastpath = True
    speculator_cls.load_draft_model = load_draft_model

    def _logits(model, hidden_states):
        lp = model.logits_processor
        return int8_logits(model.__dict__.get("_qf_head_i8"), hidden_states, lp.logits_as_input, lp.soft_cap,
                           lp.scale, getattr(model, "draft_id_to_target_id", None))

    orig_logits = mtp_cls.compute_logits

    def compute_logits(self, hidden_states, spec_step_idx=0):
        logits = _logits(self, hidden_states)
        if logits is None:
            return orig_logits(self, hidden_states, spec_step_idx)
        return logits[..., : self.logits_processor.org_vocab_size]

    orig_top = mtp_cls.get_top_tokens

    def get_top_tokens(self, hidden_states):
        lp = self.logits_processor
        si = self.lm_head.shard_indices
        ids = int8_top_tokens(self.__dict__.get("_qf_head_i8"), hidden_states, si.org_vocab_start_index,
                              lp.logits_as_input, lp.soft_cap, lp.scale, getattr(self, "draft_id_to_target_id", None))
        if ids is None:
            return orig_top(self, hidden_states)
        return ids

    mtp_cls.compute_logits = compute_logits
    mtp_cls.get_top_tokens = get_top_tokens
    logger.info("qwen_fastpath: int8 draft lm_head enabled")
    return True
