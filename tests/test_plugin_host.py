"""CPU tests of the plugin contract (reference: plugin/qwen_fastpath/__init__.py:17-28 and
patches.py:72-116): register() is idempotent and reads each switch once, QWEN_FAST_LINEAR=0 leaves the
kernel class untouched, re-patching wraps once, the op is registered as vllm::qf_int8_linear(x, w_q,
w_s, bias) with its fake impl, and the dispatcher's eligibility predicate routes each of the fallback
cases the reference's tests would force to the fallback.  No GPU: the library is
loaded for its host-only configuration queries, nothing is launched."""
import pytest
import torch

import qwen_fastpath as qf
from qwen_fastpath import patches as P


class StandInKernel:
    """Stand-in for vLLM's int8 scaled-mm kernel class (patches.py:72-116)."""

    def __init__(self, params):
        self.params = params

    def _get_layer_params(self, layer):
        return self.params

    def apply_weights(self, layer, x, bias=None):
        return ("original", layer, x, bias)

    def process_weights_after_loading(self, layer):
        layer.loaded = True


class StandInAttention:
    def forward(self, *args, **kwargs):
        return "original attention"


ORIG_APPLY = StandInKernel.apply_weights
ORIG_PWAL = StandInKernel.process_weights_after_loading
ORIG_FORWARD = StandInAttention.forward


@pytest.fixture
def fresh(monkeypatch):
    """A process-fresh plugin: register() not yet run, the stand-ins as vLLM's classes."""
    monkeypatch.setattr(qf, "_registered", False)
    monkeypatch.setattr(P, "VLLM_INT8_KERNEL_CLASSES", (f"{__name__}:StandInKernel",))
    monkeypatch.setattr(P, "VLLM_ATTENTION_CLASSES", (f"{__name__}:StandInAttention",))
    for k in ("QWEN_FAST_LINEAR", "QWEN_FAST_ATTN", "QWEN_FAST_DRAFT_HEAD", "QWEN_FAST_LINEAR_LAYOUT"):
        monkeypatch.delenv(k, raising=False)
    yield
    StandInKernel.apply_weights = ORIG_APPLY
    StandInKernel.process_weights_after_loading = ORIG_PWAL
    StandInAttention.forward = ORIG_FORWARD


def test_register_default_patches_once(fresh):
    qf.register()
    patched = StandInKernel.apply_weights
    assert patched is not ORIG_APPLY and getattr(patched, "_qwen_fastpath", False)
    # the default weight layout is the TILED image: the load-time hook is installed too
    assert getattr(StandInKernel.process_weights_after_loading, "_qwen_fastpath", False)
    assert getattr(StandInAttention.forward, "_qwen_fastpath", False)
    qf.register()  # idempotent: nothing is wrapped twice
    assert StandInKernel.apply_weights is patched
    assert P.patch_int8_linear() and StandInKernel.apply_weights is patched


def test_linear_switch_off_leaves_class_untouched(fresh, monkeypatch):
    monkeypatch.setenv("QWEN_FAST_LINEAR", "0")
    qf.register()
    assert StandInKernel.apply_weights is ORIG_APPLY
    assert StandInKernel.process_weights_after_loading is ORIG_PWAL
    # the switch is read once, at register(): turning it on afterwards changes nothing
    monkeypatch.setenv("QWEN_FAST_LINEAR", "1")
    qf.register()
    assert StandInKernel.apply_weights is ORIG_APPLY


def test_attention_switch_off(fresh, monkeypatch):
    monkeypatch.setenv("QWEN_FAST_ATTN", "0")
    qf.register()
    assert StandInAttention.forward is ORIG_FORWARD
    assert StandInKernel.apply_weights is not ORIG_APPLY


def test_rowmajor_layout_keeps_loader(fresh, monkeypatch):
    monkeypatch.setenv("QWEN_FAST_LINEAR_LAYOUT", "rowmajor")
    qf.register()
    assert StandInKernel.process_weights_after_loading is ORIG_PWAL
    assert StandInKernel.apply_weights is not ORIG_APPLY


def test_layout_switch_rejects_unknown(monkeypatch):
    monkeypatch.setenv("QWEN_FAST_LINEAR_LAYOUT", "columnmajor")
    with pytest.raises(ValueError):
        P.tiled_layout_requested()


def test_static_quantisation_keeps_original_apply(fresh):
    """A layer with a static input scale (i_s not None) keeps the original apply_weights
    (patches.py:110-112); the dynamic per-token case goes to the op."""
    P.patch_int8_linear()
    layer, x = object(), torch.zeros(2, 64)
    k = StandInKernel((None, None, torch.ones(1), None, None))
    assert k.apply_weights(layer, x)[0] == "original"
    k = StandInKernel((None, None, None, torch.zeros(1), None))
    assert k.apply_weights(layer, x)[0] == "original"
    k = StandInKernel((None, None, None, None, torch.zeros(1)))
    assert k.apply_weights(layer, x)[0] == "original"


def test_linear_method_switch():
    calls = []
    m = P.W8A16LinearMethod(fallback=lambda layer, x, bias: calls.append("orig") or "orig", enabled=False)

    class Layer:
        weight = torch.zeros(64, 16, dtype=torch.int8)
        weight_scale = torch.ones(16)
        input_scale = input_zero_point = azp_adj = None

    assert m.apply(Layer(), torch.zeros(2, 64, dtype=torch.bfloat16)) == "orig" and calls == ["orig"]


def test_op_identity_and_fake():
    """torch.ops.vllm.qf_int8_linear(x, w_q, w_s, bias) exists with the reference's four arguments,
    and its fake impl gives (*x.shape[:-1], N) in x.dtype for both weight layouts."""
    op = torch.ops.vllm.qf_int8_linear
    schema = op.default._schema
    assert [a.name for a in schema.arguments] == ["x", "w_q", "w_s", "bias"]
    assert str(schema.arguments[3].type) == "Optional[Tensor]"
    assert [a.name for a in torch.ops.qwen_fastpath.qf_int8_linear.default._schema.arguments] == ["x", "w_q", "w_s",
                                                                                                   "bias"]
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x = torch.empty(2, 3, 5120, dtype=torch.bfloat16)
        w = torch.empty(1024, 5120, dtype=torch.int8).t()
        s = torch.empty(1024, dtype=torch.float32)
        y = op(x, w, s, None)
        assert tuple(y.shape) == (2, 3, 1024) and y.dtype == torch.bfloat16
        img = torch.empty(qf.tiled_numel(1000, 5120), dtype=torch.int8)  # N not a multiple of 16
        y = op(x, img, torch.empty(1000, dtype=torch.float32), None)
        assert tuple(y.shape) == (2, 3, 1000)
        y = op(torch.empty(0, 5120, dtype=torch.bfloat16), w, s, torch.empty(1024, dtype=torch.bfloat16))
        assert tuple(y.shape) == (0, 1024)


def test_weight_layout_inference():
    w = torch.zeros(1024, 512, dtype=torch.int8).t()
    assert P.weight_layout(w) == qf.ROWMAJOR and P.out_features(w, torch.ones(1024)) == 1024
    img = torch.zeros(qf.tiled_numel(1000, 512), dtype=torch.int8)
    assert P.weight_layout(img) == qf.TILED and P.out_features(img, torch.ones(1000)) == 1000


def _case(M=5, K=5120, N=1024, dtype=torch.bfloat16, wstride=True, ns=None):
    x = torch.zeros(M, K, dtype=dtype)
    w = torch.zeros(N, K, dtype=torch.int8).t() if wstride else torch.zeros(K, N, dtype=torch.int8)
    s = torch.ones(N if ns is None else ns)
    return x, w, s


@pytest.mark.parametrize("name,args,expect", [
    ("M=16 (largest decode width)", dict(M=16), True),
    ("M=1", dict(M=1), True),
    ("M=17", dict(M=17), False),
    ("fp16 activations", dict(dtype=torch.float16), False),
    ("fp32 activations", dict(dtype=torch.float32), False),
    ("w_q.stride(0) != 1", dict(wstride=False), False),
    ("w_s.numel() != N", dict(ns=1023), False),
    ("K % 64 != 0", dict(K=5100), False),
])
def test_dispatch_predicate_truth_table(name, args, expect):
    """The reference's eligibility (patches.py:90-92) case by case; the remaining two fallback cases of
    the reference's list, QWEN_FAST_LINEAR=0 and a non-None input scale, are covered above."""
    x, w, s = _case(**args)
    assert P.shape_eligible(x, w, s) is expect, name
    assert not P.eligible(x, w, s)  # CPU tensors never take the HIP path


def test_cpu_tensors_take_the_fallback(monkeypatch):
    seen = []
    monkeypatch.setattr(P, "_fallback", lambda x2, w_q, w_s, bias, dt, layout: seen.append(layout) or
                        torch.zeros(x2.shape[0], w_s.numel(), dtype=dt))
    x, w, s = _case()
    y = P._qf_int8_linear_impl(x.view(1, 5, -1), w, s, None)
    assert tuple(y.shape) == (1, 5, 1024) and seen == [qf.ROWMAJOR]


def test_zero_tokens_need_no_device():
    x, w, s = _case(M=0)
    b = torch.ones(1024, dtype=torch.bfloat16)
    y = P._qf_int8_linear_impl(x, w, s, b)
    assert tuple(y.shape) == (0, 1024) and y.dtype == torch.bfloat16


def test_repack_refuses_other_model_dtypes():
    class Layer:
        weight = torch.zeros(1024, 512, dtype=torch.int8).t()
        input_scale = input_zero_point = azp_adj = None
        params_dtype = torch.float16

    assert P.repack_layer_weight(Layer()) is False


def test_library_wrappers_refuse_host_tensors():
    """Every wrapper that hands pointers to the library refuses tensors in host memory before any call: a host
    pointer reaching a kernel would fault the device."""
    x = torch.zeros(5, 512, dtype=torch.bfloat16)
    w = torch.zeros(1024, 512, dtype=torch.int8)
    s = torch.ones(1024, dtype=torch.float32)
    calls = [lambda: qf.rms_norm_rows(x), lambda: qf.quantize_tokens_int8(x), lambda: qf.to_tiled(w.t()),
             lambda: qf.w8a8_mm(x, w.t(), s, torch.bfloat16, layout=qf.ROWMAJOR),
             lambda: qf.dequant_bf16(w.t(), 1024, 512),
             lambda: qf.scale_cast_bf16(torch.zeros(5, 1024), s, torch.zeros(5, 1024, dtype=torch.bfloat16)),
             lambda: qf.w8a16_mm_argmax(x, w.t(), s, 1024)]
    for call in calls:
        with pytest.raises(TypeError, match="GPU tensor"):
            call()
