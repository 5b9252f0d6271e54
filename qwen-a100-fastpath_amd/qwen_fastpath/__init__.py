"""qwen_fastpath on MI355X: the W8A16 decode GEMM behind QWEN_FAST_LINEAR, the int8 MTP draft head and
the split-KV verification attention behind QWEN_FAST_ATTN.

vLLM general plugin (entry point ``qwen_fastpath:register``, as plugin/qwen_fastpath/__init__.py:17-28
in the reference).  Each patch can be switched off with an environment variable read once at
register():

  QWEN_FAST_ATTN=0        keep the original attention for speculative-decode verification batches
  QWEN_FAST_LINEAR=0      keep the original W8A8 path for small-batch (decode) int8 linears
  QWEN_FAST_DRAFT_HEAD=0  keep the bf16 lm_head for MTP draft proposals
"""
import logging
import os

from .w8a16 import (  # noqa: F401
    AUTO, ROWMAJOR, SMALL_M, TILED, W8A16Config, dequant_bf16, from_tiled, pick_config, resolve_config, tiled_numel,
    quantize_tokens_int8, rms_norm_rows, scale_cast_bf16, to_tiled, w8a16_mm, w8a16_mm_argmax, w8a16_mm_prefill,
    w8a16_mm_rmsnorm,
    w8a8_mm)
from .spec_attn import gqa_packed_spec_attention  # noqa: F401
from .patches import (  # noqa: F401
    Int8Head,
    W8A16LinearMethod,
    eligible,
    int8_logits,
    int8_top_tokens,
    make_int8_head,
    patch_draft_lm_head,
    patch_flash_attention,
    patch_int8_linear,
    qf_int8_linear,
    quantize_lm_head,
    repack_layer_weight,
    shape_eligible,
    top_tokens,
    weight_layout,
    w8a8_reference,
)

logger = logging.getLogger("vllm.qwen_fastpath")
_registered = False


def register():
    """Idempotent plugin entry point (reference: plugin/qwen_fastpath/__init__.py:17-28)."""
    global _registered
    if _registered:
        return
    _registered = True
    if os.environ.get("QWEN_FAST_ATTN", "1") == "1":
        patch_flash_attention()
    if os.environ.get("QWEN_FAST_LINEAR", "1") == "1":
        patch_int8_linear()
    if os.environ.get("QWEN_FAST_DRAFT_HEAD", "1") == "1":
        patch_draft_lm_head()
