"""GPU tests of the plugin surface: the qf_int8_linear dispatcher (plugin/qwen_fastpath/patches.py:84-116
in the reference), W8A16LinearMethod.apply, the patched apply_weights, and the int8 MTP draft head
(patches.py:119-189): quantiser, draft logits and the pad-masked argmax."""
import numpy as np
import pytest
import torch

import qwen_fastpath as qf
from qwen_fastpath import patches as P
from helpers import bf16_bits, dev_inputs, to_dev_bf16

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


class _Layer:
    def __init__(self, w_t, w_s, layout=qf.ROWMAJOR):
        self.weight = w_t
        self.weight_scale = w_s
        self.input_scale = None
        self.input_zero_point = None
        self.azp_adj = None
        self._qf_layout = layout


@pytest.fixture
def no_fallback(monkeypatch):
    """Fail the test if an eligible call reaches the W8A8 fallback."""
    def boom(*a, **k):
        raise AssertionError("eligible input reached the fallback path")
    monkeypatch.setattr(P, "_fallback", boom)


def test_dispatcher_eligible_runs_hip_kernel(oracle, no_fallback):
    M, N, K = 5, 1024, 2048
    inp = oracle.gen_inputs(M, N, K, seed=1)
    x, w, s = dev_inputs(inp, DEV)
    x3 = x.view(1, M, K)  # leading dims are flattened and restored
    y = torch.ops.qwen_fastpath.qf_int8_linear(x3, w, s.view(N, 1), None)
    torch.cuda.synchronize()
    assert y.shape == (1, M, N) and y.dtype == torch.bfloat16
    rep = oracle.check_w8a16(bf16_bits(y.view(M, N)), inp.x, inp.w, inp.s)
    assert rep.ok, rep
    # bias is added after the product, in bf16 (patches.py:96-97)
    b = torch.randn(N, device=DEV).to(torch.bfloat16)
    yb = torch.ops.qwen_fastpath.qf_int8_linear(x, w, s, b)
    assert torch.equal(yb, (y.view(M, N) + b))


def test_linear_method_apply_and_tiled_layer(oracle, no_fallback):
    M, N, K = 3, 2048, 5120
    inp = oracle.gen_inputs(M, N, K, seed=2)
    x, w, s = dev_inputs(inp, DEV)
    method = P.W8A16LinearMethod(enabled=True)
    y_rm = method.apply(_Layer(w, s), x)
    y_t = method.apply(_Layer(qf.to_tiled(w), s, qf.TILED), x)
    torch.cuda.synchronize()
    for y in (y_rm, y_t):
        assert oracle.check_w8a16(bf16_bits(y), inp.x, inp.w, inp.s).ok


def test_patched_apply_weights_routes_by_quant_scheme(oracle):
    class Kernel:  # stand-in for vLLM's int8 scaled-mm kernel class
        calls = []

        def _get_layer_params(self, layer):
            return layer.weight, layer.weight_scale, layer.input_scale, None, None

        def apply_weights(self, layer, x, bias=None):
            Kernel.calls.append("orig")
            return torch.zeros(x.shape[0], layer.weight.shape[1], device=x.device, dtype=x.dtype)

    assert P.patch_int8_linear(Kernel)
    assert P.patch_int8_linear(Kernel)  # idempotent
    M, N, K = 2, 512, 1024
    inp = oracle.gen_inputs(M, N, K, seed=3)
    x, w, s = dev_inputs(inp, DEV)
    layer = _Layer(w, s)
    y = Kernel().apply_weights(layer, x)
    assert oracle.check_w8a16(bf16_bits(y), inp.x, inp.w, inp.s).ok and Kernel.calls == []
    layer.input_scale = torch.ones(1, device=DEV)  # static activation scale: original path
    Kernel().apply_weights(layer, x)
    assert Kernel.calls == ["orig"]


def test_ineligible_m17_uses_w8a8_fallback(oracle):
    """M > 16 takes the W8A8 path; its error against the exact product is the reference's published
    W8A8 statistic (0.0083-0.0094 rel-L2, data/measurements.json:420-427), not the W8A16 one."""
    M, N, K = 17, 5120, 6144
    inp = oracle.gen_inputs(M, N, K, seed=4, dist="reftest")
    x, w, s = dev_inputs(inp, DEV)
    y = torch.ops.qwen_fastpath.qf_int8_linear(x, w, s, None)
    torch.cuda.synchronize()
    ex = oracle.w8a16_f64(inp.x, inp.w, inp.s)
    yf = y.float().cpu().numpy().astype(np.float64)
    rel = np.linalg.norm(yf - ex) / np.linalg.norm(ex)
    assert 0.006 <= rel <= 0.012, rel


@pytest.mark.parametrize("M,N,K", [(17, 5120, 6144), (64, 1000, 2048), (300, 512, 17408)])
def test_w8a8_integer_products_library_gemm_matches_fp64(M, N, K):
    """The W8A8 restatement's integer sums through the library int8 GEMM (int32) equal the fp64 ones bit
    for bit after the one rounding to fp32, extremes included (-128 activations, +-127 weights)."""
    from qwen_fastpath import patches as P
    g = torch.Generator(device=DEV)
    g.manual_seed(M + N)
    x_q = torch.randint(-128, 128, (M, K), device=DEV, generator=g).float()
    x_q[0] = -128.0
    w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=DEV, generator=g)
    w[0] = 127
    got = P._int8_products(x_q, w.t())
    ref = (x_q.double() @ w.t().double()).float()
    direct = torch._int_mm(x_q.to(torch.int8), w.t())  # the library path itself runs for these shapes
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.equal(direct.float(), ref)


def test_quantize_lm_head_bit_exact(oracle):
    V, H = 3000, 5120
    rng = np.random.default_rng(5)
    wf = rng.standard_normal((V, H)) * np.exp2(rng.integers(-6, 3, (V, 1)))
    wf[7] = 0.0
    wb = oracle.bf16_from_f64(wf)
    q_ref, s_ref = oracle.quantize_rows(wb)
    w8, sc = qf.quantize_lm_head(to_dev_bf16(wb, DEV))
    torch.cuda.synchronize()
    assert np.array_equal(sc.cpu().numpy(), s_ref)
    assert np.array_equal(w8.cpu().numpy(), q_ref)


@pytest.mark.parametrize("H", [8, 5120, 8192, 5124, 8200])
def test_quantizer_kernels_bit_exact(oracle, H):
    """Both quantiser kernels: the single-pass vector one (16-byte-aligned rows, H % 8 == 0, H <= 8192) and
    the general one (H = 5124, 8200), with zero rows, huge and tiny magnitudes and values at exact ties."""
    V = 257
    rng = np.random.default_rng(H)
    wf = rng.standard_normal((V, H)) * np.exp2(rng.integers(-20, 20, (V, 1)))
    wf[3] = 0.0
    wf[5, :] = 2.5                # amax 127: scale ~1, so 2.5 / s sits on (or next to) a half step
    wf[5, 0] = 127.0
    wb = oracle.bf16_from_f64(wf)
    q_ref, s_ref = oracle.quantize_rows(wb)
    w8, sc = qf.quantize_lm_head(to_dev_bf16(wb, DEV))
    torch.cuda.synchronize()
    assert np.array_equal(sc.cpu().numpy(), s_ref)
    assert np.array_equal(w8.cpu().numpy(), q_ref)


def test_draft_head_logits_and_argmax(oracle):
    """int8 draft logits through the W8A16 kernel (patches.py:157-166) and the pad-masked argmax
    (patches.py:182-185), against the oracle.  A row whose top-2 exact logits are within 2 bf16 ulp
    cannot have a guaranteed argmax and is reported instead of compared."""
    V, H, num_pad, start = 151936, 5120, 64, 1000
    rng = np.random.default_rng(6)
    g = torch.Generator(device=DEV)
    g.manual_seed(6)
    w_dev = (torch.randn(V, H, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    wb = bf16_bits(w_dev)
    head = qf.make_int8_head(w_dev, num_pad)  # TILED copy
    head_rm = qf.make_int8_head(w_dev, num_pad, qf.ROWMAJOR)  # the reference's row-major copy
    assert head.layout == qf.TILED and head_rm.layout == qf.ROWMAJOR
    q, s = oracle.quantize_rows(wb)
    assert np.array_equal(head.scale.cpu().numpy(), s)
    assert np.array_equal(qf.from_tiled(head.w_t, V, H).cpu().numpy(), head_rm.w_t.cpu().numpy())
    for M in (1, 4):
        hb = oracle.bf16_from_f64(rng.standard_normal((M, H)))
        logits = qf.int8_logits(head, to_dev_bf16(hb, DEV))
        assert logits is not None and logits.shape == (M, V)
        rep = oracle.check_w8a16(bf16_bits(logits), hb, q, s)
        assert rep.ok, rep
        rep_rm = oracle.check_w8a16(bf16_bits(qf.int8_logits(head_rm, to_dev_bf16(hb, DEV))), hb, q, s)
        assert rep_rm.ok, rep_rm
        ids = qf.top_tokens(logits, num_pad, start).cpu().numpy()
        want = oracle.argmax_rows(bf16_bits(logits), V - num_pad, start)
        assert np.array_equal(ids, want)  # same logits: argmax semantics must agree exactly
        ex_bits, ex64 = oracle.w8a16_exact(hb, q, s)
        ex_ids = oracle.argmax_rows(ex_bits, V - num_pad, start)
        for m in range(M):
            row = ex64[m, : V - num_pad]
            top2 = np.sort(row)[-2:]
            gap_ulp = (top2[1] - top2[0]) / oracle.bf16_ulp(np.array([top2[1]]))[0]
            if gap_ulp >= 2:
                assert ids[m] == ex_ids[m], (M, m, gap_ulp)
            else:
                print(f"draft head M={M} row {m}: top-2 gap {gap_ulp:.2f} ulp, argmax not guaranteed")
    # guards of patches.py:160-163
    hb = torch.zeros((17, H), dtype=torch.bfloat16, device=DEV)
    assert qf.int8_logits(head, hb) is None
    assert qf.int8_logits(head, hb[:2], soft_cap=30.0) is None
    assert qf.int8_logits(None, hb[:2]) is None


def test_top_tokens_semantics():
    v = torch.full((4, 300), -1.0)
    v[0, 10] = v[0, 20] = 3.0          # tie -> first
    v[1, 299] = 9.0                    # inside the pad -> ignored
    v[1, 5] = 2.0
    v[2, 7] = float("nan")             # NaN is the maximum
    v[2, 8] = 100.0
    v[3, :] = -float("inf")            # all -inf -> first index
    ids = qf.top_tokens(v.to(torch.bfloat16).to(DEV), num_pad=4, vocab_start=10).cpu().tolist()
    assert ids == [20, 15, 17, 10]


def test_top_tokens_vector_path(oracle):
    """Rows whose stride allows 16-byte loads (8 logits per load) plus a scalar tail."""
    N, num_pad, start = 41000, 5, 17
    v = np.full((5, N), -1.0)
    v[0, 100] = v[0, 40000] = 4.0          # tie across vector groups -> first
    v[1, N - 2] = 9.0                      # in the pad
    v[1, N - num_pad - 1] = 8.0            # last valid column, in the scalar tail
    v[2, 33333] = np.nan
    v[2, 9999] = np.nan                    # first NaN wins
    v[3, :] = -np.inf
    v[4, 7] = v[4, N - num_pad - 2] = 6.0  # tie between a vector group and the tail -> first
    bits = oracle.bf16_from_f64(v)
    logits = torch.from_numpy(bits.view(np.int16)).to(DEV).view(torch.bfloat16)
    ids = qf.top_tokens(logits, num_pad, start).cpu().numpy()
    want = oracle.argmax_rows(bits, N - num_pad, start)
    assert np.array_equal(ids, want)
    assert list(ids) == [100 + start, N - num_pad - 1 + start, 9999 + start, start, 7 + start]


@pytest.mark.parametrize("M,N,num_pad", [(1, 16384, 0), (16, 16392, 3), (3, 151936, 64), (16, 8192 * 64, 1)])
def test_top_tokens_row_split(oracle, M, N, num_pad):
    """Rows cut into 8192-logit chunks across workgroups, folded by the last one: random rows with a
    planted maximum in a random chunk and a tie later in the row, against the oracle."""
    rng = np.random.default_rng(M * 100 + N % 97)
    v = rng.standard_normal((M, N))
    for m in range(M):
        j = int(rng.integers(0, N - num_pad))
        v[m, j] = 50.0 + m
        v[m, min(j + 1 + int(rng.integers(0, 9000)), N - num_pad - 1)] = 50.0 + m  # tie: first wins
        if num_pad:
            v[m, N - 1] = 1e4                                                       # pad ignored
    bits = oracle.bf16_from_f64(v)
    logits = torch.from_numpy(bits.view(np.int16)).to(DEV).view(torch.bfloat16)
    for _ in range(2):  # the arrival counters are back at zero for the next call
        ids = qf.top_tokens(logits, num_pad, 5).cpu().numpy()
        assert np.array_equal(ids, oracle.argmax_rows(bits, N - num_pad, 5))


def test_load_time_tiled_repack(oracle, monkeypatch):
    """QWEN_FAST_LINEAR_LAYOUT=tiled: after the kernel class's own process_weights_after_loading has
    laid the checkpoint's [N, K] weight out as the [K, N] column-major view, the weight is replaced by
    its TILED image (one copy); decode calls and M > 16 calls (the reference's W8A8 arithmetic by
    default, the W8A16 one with QWEN_FAST_LINEAR_PREFILL=w8a16) both stay correct."""
    class Kernel:  # stand-in for vLLM's int8 scaled-mm kernel class
        def process_weights_after_loading(self, layer):
            layer.weight = torch.nn.Parameter(layer.weight.t(), requires_grad=False)

        def _get_layer_params(self, layer):
            return layer.weight, layer.weight_scale, layer.input_scale, None, None

        def apply_weights(self, layer, x, bias=None):
            raise AssertionError("the original path must not run for a dynamic int8 layer")

    assert P.patch_int8_linear(Kernel, tiled=True)
    M, N, K = 5, 1000, 2048
    inp = oracle.gen_inputs(M, N, K, seed=8)
    layer = _Layer(torch.from_numpy(inp.w).to(DEV), torch.from_numpy(inp.s).to(DEV))
    Kernel().process_weights_after_loading(layer)
    assert layer._qf_layout == qf.TILED and layer.weight.numel() == qf.tiled_numel(N, K)
    x = to_dev_bf16(inp.x, DEV)
    y = Kernel().apply_weights(layer, x)
    torch.cuda.synchronize()
    assert oracle.check_w8a16(bf16_bits(y), inp.x, inp.w, inp.s).ok
    rng = np.random.default_rng(9)
    x20 = oracle.bf16_from_f64(rng.standard_normal((20, K)))
    monkeypatch.setenv("QWEN_FAST_LINEAR_PREFILL", "w8a16")
    y20 = Kernel().apply_weights(layer, to_dev_bf16(x20, DEV))
    torch.cuda.synchronize()
    assert y20.shape == (20, N) and oracle.check_w8a16(bf16_bits(y20), x20, inp.w, inp.s).ok
    monkeypatch.delenv("QWEN_FAST_LINEAR_PREFILL")
    y20 = Kernel().apply_weights(layer, to_dev_bf16(x20, DEV))
    ref = P.w8a8_reference(to_dev_bf16(x20, DEV), torch.from_numpy(inp.w).to(DEV).t(), torch.from_numpy(inp.s).to(DEV),
                           None, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(y20.view(torch.int16), ref.view(torch.int16))
    assert not qf.repack_layer_weight(_Layer(torch.zeros(4, 4, dtype=torch.float32, device=DEV), None))


def test_draft_head_baseline_inputs_full_size(oracle):
    """The draft-head configuration's own inputs at full size: V = 151936, H = 5120, int8 weights uniform in
    [-127, 127] and per-row fp32 scales |N(0,1)| * 0.002 + 1e-4 (the oracle's generator, seed 0), bf16 N(0,1)
    hidden rows, M = 1 and 4, the head in its TILED copy.  The logits pass oracle.check_w8a16 against the exact
    product; the ids of the fused epilogue (qf_w8a16_gemm_argmax) and of logits-then-argmax equal the argmax of
    the kernel's own logits, and equal the exact product's argmax on every row whose top-2 exact logits are 2
    bf16 ulp or more apart (a row under that gap is reported, not compared)."""
    V, H, num_pad, start = 151936, 5120, 64, 0
    for M in (1, 4):
        inp = oracle.gen_inputs(M, V, H, seed=0)
        w_dev = torch.from_numpy(inp.w).to(DEV)
        head = qf.Int8Head(qf.to_tiled(w_dev.t()), torch.from_numpy(inp.s).to(DEV), num_pad,
                           qf.pick_config(V, H, qf.TILED), qf.TILED)
        del w_dev
        hb = to_dev_bf16(inp.x, DEV)
        print(f"draft head baseline inputs M={M}", flush=True)
        logits = qf.int8_logits(head, hb)
        fused = qf.int8_top_tokens(head, hb, start, fused=True)
        two = qf.int8_top_tokens(head, hb, start, fused=False)
        torch.cuda.synchronize()
        lb = bf16_bits(logits)
        ex_bits, ex64 = oracle.w8a16_exact(inp.x, inp.w, inp.s)
        rep = oracle.check_w8a16(lb, inp.x, inp.w, inp.s, exact=(ex_bits, ex64))
        print(f"  logits: {rep}", flush=True)
        assert rep.ok, rep
        own = oracle.argmax_rows(lb, V - num_pad, start)
        assert np.array_equal(fused.cpu().numpy(), own) and np.array_equal(two.cpu().numpy(), own), M
        ex_ids = oracle.argmax_rows(ex_bits, V - num_pad, start)
        for m in range(M):
            row = ex64[m, : V - num_pad]
            top2 = np.sort(row)[-2:]
            gap_ulp = (top2[1] - top2[0]) / oracle.bf16_ulp(np.array([top2[1]]))[0]
            print(f"  row {m}: exact argmax {ex_ids[m]}, kernel {own[m]}, top-2 gap {gap_ulp:.2f} ulp", flush=True)
            if gap_ulp >= 2:
                assert own[m] == ex_ids[m], (M, m, gap_ulp)
        del head
