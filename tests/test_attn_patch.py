"""The verification-attention patch (qwen_fastpath.patches.patch_flash_attention), the counterpart of
the reference's FlashAttentionImpl.forward patch (plugin/qwen_fastpath/patches.py:10-69), on stand-in
implementation and metadata objects: which batches take the split-KV kernel, which keep the original
forward, the per-layer predicate, and (GPU) that the routed call writes the oracle's result into the
layer's output."""
import types

import numpy as np
import pytest
import torch

from qwen_fastpath import patches as P


class _Impl:
    """Stand-in with the attributes the reference's predicate reads (patches.py:24-44)."""
    calls = 0

    def __init__(self, H=24, HKV=4, D=256, **over):
        self.num_heads, self.num_kv_heads, self.head_size = H, HKV, D
        self.scale = D ** -0.5
        self.attn_type = "decoder"
        self.dcp_world_size = 1
        self.vllm_flash_attn_version = 2
        self.sliding_window = (-1, -1)
        self.alibi_slopes = None
        self.logits_soft_cap = 0
        self.sinks = None
        self.kv_cache_dtype = "auto"
        self.kv_sharing_target_layer_name = None
        for k, v in over.items():
            setattr(self, k, v)

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output, output_scale=None,
                output_block_scale=None):
        type(self).calls += 1
        output.fill_(-7.0)
        return output


def _md(B, Q, lens=None, **over):
    md = types.SimpleNamespace(
        max_query_len=Q, use_cascade=False, causal=True, mm_prefix_query_range_tensor=None,
        rswa_prefix_lens=None, num_actual_tokens=B * Q,
        query_start_loc=torch.arange(B + 1, dtype=torch.int32) * Q,
        seq_lens=None, block_table=None)
    for k, v in over.items():
        setattr(md, k, v)
    return md


def test_uniform_batch_detection():
    assert P.spec_batch_q_len(_md(2, 3)) == 3
    assert P.spec_batch_q_len(_md(1, 8)) == 8
    assert P.spec_batch_q_len(_md(1, 1)) is None            # Q == 1: plain decode stays on the original
    assert P.spec_batch_q_len(_md(1, 9)) is None            # beyond MAX_SPEC_QUERY_LEN
    assert P.spec_batch_q_len(_md(2, 3, num_actual_tokens=5)) is None   # mixed batch
    assert P.spec_batch_q_len(_md(2, 3, use_cascade=True)) is None
    assert P.spec_batch_q_len(_md(2, 3, causal=False)) is None
    assert P.spec_batch_q_len(_md(2, 3, rswa_prefix_lens=torch.zeros(1))) is None
    assert P.spec_batch_q_len(None) is None


def test_layer_predicate():
    assert P.attn_impl_eligible(_Impl())
    for over in ({"head_size": 96}, {"sliding_window": (128, 0)}, {"alibi_slopes": torch.zeros(1)},
                 {"logits_soft_cap": 30.0}, {"kv_cache_dtype": "fp8_e4m3"}, {"vllm_flash_attn_version": 3},
                 {"dcp_world_size": 2}, {"attn_type": "encoder"}, {"kv_sharing_target_layer_name": "l0"},
                 {"num_kv_heads": 5}):
        assert not P.attn_impl_eligible(_Impl(**over)), over
    impl = _Impl()
    P.attn_impl_eligible(impl)
    impl.head_size = 96  # evaluated once per layer object, as the reference caches it
    assert P.attn_impl_eligible(impl)


def test_patch_is_idempotent_and_falls_back():
    class Impl(_Impl):
        calls = 0
    assert P.patch_flash_attention(Impl)
    f = Impl.forward
    assert P.patch_flash_attention(Impl) and Impl.forward is f
    impl = Impl()
    out = torch.zeros(6, 24 * 256)
    # a mixed batch keeps the original forward (which writes -7)
    Impl.forward(impl, None, torch.zeros(6, 24 * 256), None, None, None, _md(2, 3, num_actual_tokens=5), out)
    assert Impl.calls == 1 and torch.all(out == -7)
    Impl.forward(impl, None, torch.zeros(6, 24 * 256), None, None, None, _md(2, 3), out, output_scale=1.0)
    assert Impl.calls == 2


@pytest.mark.gpu
def test_patched_forward_runs_the_kernel(oracle):
    from oracle import attn as A

    class Impl(_Impl):
        calls = 0
    P.patch_flash_attention(Impl)
    inp = A.gen_spec_inputs(3000, 3, 2, seed=4)
    dev = torch.device("cuda:0")
    kv = torch.from_numpy(inp.kv.view(np.int16)).to(dev).view(torch.bfloat16)   # [blocks, H_kv, PAGE, 2D]
    q = torch.from_numpy(inp.q.view(np.int16)).to(dev).view(torch.bfloat16).reshape(6, 24 * 256)
    out = torch.full_like(q, float("nan"))
    md = _md(2, 3, seq_lens=torch.from_numpy(inp.seq_lens).to(dev),
             block_table=torch.from_numpy(inp.block_table).to(dev))
    impl = Impl()
    res = Impl.forward(impl, None, q, None, None, kv, md, out)
    torch.cuda.synchronize()
    assert res is out and Impl.calls == 0
    ref = A.spec_attention(inp.query(), inp.key_cache(), inp.value_cache(), inp.seq_lens, inp.block_table,
                           2, 3, 4, 256 ** -0.5)
    rep = A.check_spec_attn(out.float().cpu().numpy().reshape(6, 24, 256), ref, inp.seq_lens, 3)
    assert rep.ok, rep
