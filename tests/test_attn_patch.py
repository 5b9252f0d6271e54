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
        if output is not None:
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


@pytest.mark.gpu
def test_unserved_calls_keep_the_original_forward(oracle):
    """Calls the library would refuse -- a misaligned query, a row stride that is not a multiple of 8
    elements, a cache whose token stride overflows the kernel's 32-bit stage offsets -- are recognised by
    spec_attn.supported (the C checks restated) and take the original forward instead of raising."""
    from oracle import attn as A
    from qwen_fastpath import spec_attn as S

    class Impl(_Impl):
        calls = 0
    P.patch_flash_attention(Impl)
    dev = torch.device("cuda:0")
    inp = A.gen_spec_inputs(300, 3, 2, seed=5)
    kv = torch.from_numpy(inp.kv.view(np.int16)).to(dev).view(torch.bfloat16)
    md = _md(2, 3, seq_lens=torch.from_numpy(inp.seq_lens).to(dev),
             block_table=torch.from_numpy(inp.block_table).to(dev))
    key_cache, value_cache = P._interleaved_kv_split(kv, 256)
    q = torch.zeros(6, 24 * 256, dtype=torch.bfloat16, device=dev)
    q3 = q.view(6, 24, 256)
    assert S.supported(q3, key_cache, 3, 4, value_cache, q3, 2)
    # misaligned query: a view one element into a larger buffer
    big = torch.zeros(6 * 24 * 256 + 8, dtype=torch.bfloat16, device=dev)
    qm = big[1:1 + 6 * 24 * 256].view(6, 24 * 256)
    assert not S.supported(qm.view(6, 24, 256), key_cache, 3, 4, value_cache, q3, 2)
    out = torch.zeros(6, 24 * 256, dtype=torch.bfloat16, device=dev)
    Impl.forward(Impl(), None, qm, None, None, kv, md, out)
    assert Impl.calls == 1 and torch.all(out == -7)
    # the same call on an aligned query takes the kernel
    Impl.forward(Impl(), None, q, None, None, kv, md, out)
    torch.cuda.synchronize()
    assert Impl.calls == 1 and not torch.any(out == -7)


class _Desc:
    """A tensor descriptor with the attributes spec_attn.supported reads, standing for a device tensor
    without allocating one, so each refusal is exercised on the host."""

    def __init__(self, shape, stride=None, ptr=0, dtype=torch.bfloat16):
        self.shape = tuple(shape)
        if stride is None:
            stride, acc = [], 1
            for n in reversed(self.shape):
                stride.insert(0, acc)
                acc *= n
        self._stride, self._ptr, self.dtype, self.is_cuda = tuple(stride), ptr, dtype, True

    def stride(self, dim=None):
        return self._stride if dim is None else self._stride[dim]

    def data_ptr(self):
        return self._ptr


def _cache(page=16, hkv=4, d=256, tok_stride=None):
    # [blocks, PAGE, H_kv, D] view of the interleaved [blocks, H_kv, PAGE, 2D] cache
    ts = 2 * d if tok_stride is None else tok_stride
    return _Desc((10, page, hkv, d), (hkv * page * 2 * d, ts, page * 2 * d, 1))


@pytest.mark.parametrize("case,expect", [
    ("served", True),
    ("misaligned query", False),
    ("query row stride not a multiple of 8", False),
    ("fp16 cache", False),
    ("host tensors", False),
    ("page of 8 positions", False),
    ("head size 96", False),
    ("Q x group rows above 64", False),
    ("token stride overflows 32-bit stage offsets", False),
    ("more than 65535 (request, kv head) pairs", False),
    ("output head geometry differs", False),
    ("negative stride", False),
])
def test_supported_restates_the_library_checks(case, expect):
    """spec_attn.supported refuses exactly the calls the library's own checks reject, so the patched
    forward falls back instead of raising; one refusal per case, on host-side descriptors."""
    from qwen_fastpath import spec_attn as S
    q = _Desc((6, 24, 256), ptr=4096)
    kc, vc = _cache(), _cache()
    o = _Desc((6, 24, 256), ptr=8192)
    Q, hkv, nreq = 3, 4, 2
    if case == "misaligned query":
        q._ptr = 4098
    elif case == "query row stride not a multiple of 8":
        q._stride = (24 * 256 + 4, 256, 1)
    elif case == "fp16 cache":
        kc.dtype = torch.float16
    elif case == "host tensors":
        vc.is_cuda = False
    elif case == "page of 8 positions":
        kc, vc = _cache(page=8), _cache(page=8)
    elif case == "head size 96":
        q, o = _Desc((6, 24, 96), ptr=4096), _Desc((6, 24, 96), ptr=8192)
    elif case == "Q x group rows above 64":
        Q = 11   # 11 x 6 = 66 packed rows
    elif case == "token stride overflows 32-bit stage offsets":
        vc = _cache(tok_stride=1 << 25)
    elif case == "more than 65535 (request, kv head) pairs":
        nreq = 16384 + 1
    elif case == "output head geometry differs":
        o = _Desc((6, 12, 256), ptr=8192)
    elif case == "negative stride":
        kc._stride = (-kc._stride[0],) + kc._stride[1:]
    assert S.supported(q, kc, Q, hkv, vc, o, nreq) is expect, case


@pytest.mark.gpu
def test_w8a8_fallback_predicate_takes_misaligned_weights():
    """A row-major weight view that is not 16-byte aligned fails _w8a8_hip's predicate and is served by
    the torch restatement instead of raising from the library."""
    dev = torch.device("cuda:0")
    M, N, K = 20, 256, 1024
    x = torch.randn(M, K, device=dev).to(torch.bfloat16)
    buf = torch.randint(-127, 128, (N * K + 16,), dtype=torch.int8, device=dev)
    w = buf[1:1 + N * K].view(N, K).t()  # [K, N] view, stride (1, K), data_ptr % 16 == 1
    s = torch.rand(N, device=dev) * 0.002 + 1e-4
    assert w.data_ptr() % 16
    y = P._w8a8_hip(x, w, s, None, torch.bfloat16)
    assert torch.equal(y, P.w8a8_reference(x, w, s, None, torch.bfloat16))


def _kv_layouts(nblk=3, page=16, hkv=2, d=64):
    """One cache's contents in the three layouts: K[b, t, h, :] = 1000 b + 10 t + h + d-index / 1000 and
    V the same, negated."""
    b = torch.arange(nblk).view(-1, 1, 1, 1).float()
    t = torch.arange(page).view(1, -1, 1, 1).float()
    h = torch.arange(hkv).view(1, 1, -1, 1).float()
    e = torch.arange(d).view(1, 1, 1, -1).float()
    K = 1000 * b + 10 * t + h + e / 1000
    V = -K
    inter = torch.cat([K, V], dim=-1).transpose(1, 2).contiguous()   # [blocks, H_kv, PAGE, 2D]
    stacked = torch.stack([K, V]).contiguous()                       # [2, blocks, PAGE, H_kv, D]
    paired = torch.stack([K, V], dim=1).contiguous()                 # [blocks, 2, PAGE, H_kv, D]
    return K, V, inter, stacked, paired


def test_cache_layout_adapters():
    K, V, inter, stacked, paired = _kv_layouts()
    for fn, cache in ((P._interleaved_kv_split, inter), (P._stacked_kv_split, stacked),
                      (P._paired_kv_split, paired), (P._flash_attn_kv_split, inter),
                      (P._flash_attn_kv_split, stacked)):
        k, v = fn(cache, 64)
        assert k.shape == K.shape and torch.equal(k, K) and torch.equal(v, V), fn.__name__
        assert k.data_ptr() >= cache.data_ptr() and k.stride(-1) == 1  # views of the cache, no copy
    # a cache in another layout (or head size) is declined, so the call keeps the original forward
    assert P._interleaved_kv_split(stacked, 64) is None and P._interleaved_kv_split(inter, 128) is None
    assert P._stacked_kv_split(inter, 64) is None and P._stacked_kv_split(paired, 64) is None
    assert P._paired_kv_split(stacked, 64) is None and P._paired_kv_split(inter, 64) is None
    assert P._stacked_kv_split(None, 64) is None


def test_default_classes_each_with_its_adapter(monkeypatch):
    """Every class of VLLM_ATTENTION_CLASSES that imports is patched with its own adapter; a bare string
    entry reads the reference's layout; classes that do not import are skipped."""
    import sys
    mod = types.ModuleType("qf_standin_attn_backends")

    class FA(_Impl):
        calls = 0

    class Triton(_Impl):
        calls = 0

    class Legacy(_Impl):
        calls = 0

    mod.FA, mod.Triton, mod.Legacy = FA, Triton, Legacy
    monkeypatch.setitem(sys.modules, "qf_standin_attn_backends", mod)
    seen = []

    def spy(name, fn):
        def adapter(kv_cache, head_size):
            seen.append(name)
            return fn(kv_cache, head_size)
        return adapter

    monkeypatch.setattr(P, "VLLM_ATTENTION_CLASSES", (
        ("qf_standin_attn_backends:FA", spy("fa", P._flash_attn_kv_split)),
        ("qf_standin_attn_backends:Triton", spy("triton", P._paired_kv_split)),
        "qf_standin_attn_backends:Legacy",
        ("qf_standin_attn_backends:Missing", P._stacked_kv_split),
        ("qf_no_such_module:X", P._stacked_kv_split),
    ))
    assert P.patch_flash_attention()
    for cls in (FA, Triton, Legacy):
        assert getattr(cls.forward, "_qwen_fastpath", False)
    f = Triton.forward
    assert P.patch_flash_attention() and Triton.forward is f
    # host tensors never take the kernel: each call reaches its adapter, then the original forward
    _, _, inter, stacked, paired = _kv_layouts(page=16, hkv=4, d=256)
    out = torch.zeros(6, 24 * 256)
    for cls, cache in ((FA, stacked), (Triton, paired)):
        cls.forward(cls(), None, torch.zeros(6, 24 * 256), None, None, cache, _md(2, 3), out)
        assert cls.calls == 1 and torch.all(out == -7)
    assert seen == ["fa", "triton"]
    # no output buffer: the original forward, without reading the cache
    Triton.forward(Triton(), None, torch.zeros(6, 24 * 256), None, None, paired, _md(2, 3), None)
    assert Triton.calls == 2 and seen == ["fa", "triton"]


@pytest.mark.gpu
def test_patched_forward_on_each_cache_layout(oracle):
    """The same batch through the patched forward with the cache in the reference's interleaved layout,
    the stacked [2, blocks, PAGE, H_kv, D] layout and the paired [blocks, 2, PAGE, H_kv, D] layout: all
    three take the kernel, give the same bits, and pass the oracle."""
    from oracle import attn as A

    inp = A.gen_spec_inputs(2000, 3, 2, seed=6)
    dev = torch.device("cuda:0")
    kv = torch.from_numpy(inp.kv.view(np.int16)).to(dev).view(torch.bfloat16)   # [blocks, H_kv, PAGE, 2D]
    K = kv[..., :256].transpose(1, 2)
    V = kv[..., 256:].transpose(1, 2)
    caches = {"interleaved": (kv, P._flash_attn_kv_split),
              "stacked": (torch.stack([K, V]).contiguous(), P._stacked_kv_split),
              "paired": (torch.stack([K, V], dim=1).contiguous(), P._paired_kv_split)}
    q = torch.from_numpy(inp.q.view(np.int16)).to(dev).view(torch.bfloat16).reshape(6, 24 * 256)
    md = _md(2, 3, seq_lens=torch.from_numpy(inp.seq_lens).to(dev),
             block_table=torch.from_numpy(inp.block_table).to(dev))
    ref = A.spec_attention(inp.query(), inp.key_cache(), inp.value_cache(), inp.seq_lens, inp.block_table,
                           2, 3, 4, 256 ** -0.5)
    outs = {}
    for name, (cache, adapter) in caches.items():
        class Impl(_Impl):
            calls = 0
        P.patch_flash_attention(Impl, adapter)
        out = torch.full_like(q, float("nan"))
        Impl.forward(Impl(), None, q, None, None, cache, md, out)
        torch.cuda.synchronize()
        assert Impl.calls == 0, name
        rep = A.check_spec_attn(out.float().cpu().numpy().reshape(6, 24, 256), ref, inp.seq_lens, 3)
        print(f"{name}: {rep}", flush=True)
        assert rep.ok, (name, rep)
        outs[name] = out
    assert torch.equal(outs["stacked"], outs["interleaved"]) and torch.equal(outs["paired"], outs["interleaved"])
