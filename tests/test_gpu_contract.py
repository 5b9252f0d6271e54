"""GPU tests of the op contract the reference's callers rely on (plugin/qwen_fastpath/patches.py:84-116):

* torch.ops.vllm.qf_int8_linear(x, w_q, w_s, bias) passes torch.library.opcheck (schema, fake impl,
  dynamic-shape tracing) on both weight layouts and on a fallback call, and traces as one opaque node
  under torch.compile(fullgraph=True);
* zero-token calls return an empty [..., N] result on both layouts;
* the fallback cases reach the reference's W8A8 arithmetic (fp16 activations, a weight whose stride(0)
  is not 1, K not a multiple of 64), including fp16 activations on a TILED layer;
* calls on two streams at once, each with its own workspace (fused split-K GEMM, row-split argmax), match
  the same calls run one after the other; a split-K call captured into a graph with no eager call on the
  capture stream before replays correctly."""
import numpy as np
import pytest
import torch

import qwen_fastpath as qf
from qwen_fastpath import _lib as L
from qwen_fastpath import patches as P
from helpers import bf16_bits, dev_inputs

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _inputs(oracle, M, N, K, seed):
    inp = oracle.gen_inputs(M, N, K, seed=seed)
    x, w, s = dev_inputs(inp, DEV)
    return inp, x, w, s


def test_opcheck_vllm_op(oracle):
    M, N, K = 5, 1024, 2048
    _, x, w, s = _inputs(oracle, M, N, K, 11)
    img = qf.to_tiled(w)
    b = torch.randn(N, device=DEV).to(torch.bfloat16)
    x17 = torch.randn(17, K, device=DEV).to(torch.bfloat16)
    for args in ((x, w, s, None), (x.view(1, M, K), img, s, b), (x17, w, s, None), (x17, img, s, None)):
        torch.library.opcheck(torch.ops.vllm.qf_int8_linear.default, args)


def test_compile_fullgraph_one_opaque_node(oracle):
    M, N, K = 4, 1024, 2048
    inp, x, w, s = _inputs(oracle, M, N, K, 12)
    img = qf.to_tiled(w)
    graphs = []

    def backend(gm, example_inputs):
        graphs.append(gm)
        return gm.forward

    def f(a, wq, ws):
        y = torch.ops.vllm.qf_int8_linear(a, wq, ws, None)
        return y * 2

    for wq in (w, img):
        torch._dynamo.reset()
        graphs.clear()
        cf = torch.compile(f, backend=backend, fullgraph=True)
        y = cf(x, wq, s)
        torch.cuda.synchronize()
        assert torch.equal(y, f(x, wq, s))
        calls = [n for gm in graphs for n in gm.graph.nodes
                 if n.op == "call_function" and "qf_int8_linear" in str(n.target)]
        assert len(calls) == 1, [str(n.target) for gm in graphs for n in gm.graph.nodes]
        assert oracle.check_w8a16(bf16_bits(y / 2), inp.x, inp.w, inp.s).ok
    # the same function through AOT autograd (fake-tensor tracing of the op, eager execution)
    torch._dynamo.reset()
    cf = torch.compile(f, backend="aot_eager", fullgraph=True)
    assert torch.equal(cf(x, img, s), f(x, img, s))


def test_zero_tokens_both_layouts(oracle):
    _, x, w, s = _inputs(oracle, 3, 512, 1024, 13)
    b = torch.randn(512, device=DEV).to(torch.bfloat16)
    for wq in (w, qf.to_tiled(w)):
        for x0 in (x[:0], x[:0].view(1, 0, 1024)):
            y = torch.ops.vllm.qf_int8_linear(x0, wq, s, b)
            assert tuple(y.shape) == (*x0.shape[:-1], 512) and y.dtype == torch.bfloat16
    assert tuple(qf.w8a16_mm(x[:0], w, s, None, torch.bfloat16).shape) == (0, 512)
    assert tuple(qf.w8a8_mm(x[:0], qf.to_tiled(w), s, torch.bfloat16).shape) == (0, 512)


def test_fallback_cases_reach_w8a8(oracle, monkeypatch):
    """Each ineligible call goes to the W8A8 arithmetic of the reference's fallback (scaled_int8_quant +
    cutlass_scaled_mm, patches.py:99-100; here its torch restatement w8a8_reference, or the library's
    W8A8 kernels where they serve the call, bit-identical to it) and never to the W8A16 kernel."""
    monkeypatch.setattr(P, "_fallback_impl", None)
    M, N, K = 4, 256, 1024
    _, x, w, s = _inputs(oracle, M, N, K, 14)

    def no_w8a16(*a, **k):
        raise AssertionError("ineligible call reached the W8A16 kernel")

    monkeypatch.setattr(P, "w8a16_mm", no_w8a16)
    # fp16 activations, row-major and TILED (the image is unpacked for the restatement)
    xh = x.to(torch.float16)
    want = P.w8a8_reference(xh, w, s, None, torch.float16)
    assert torch.equal(torch.ops.vllm.qf_int8_linear(xh, w, s, None), want)
    assert torch.equal(torch.ops.vllm.qf_int8_linear(xh, qf.to_tiled(w), s, None), want)
    # a weight with stride(0) != 1 (a [K, N] row-major copy)
    wc = w.contiguous()
    assert wc.stride(0) != 1
    assert torch.equal(torch.ops.vllm.qf_int8_linear(x, wc, s, None), P.w8a8_reference(x, wc, s, None, torch.bfloat16))
    # K not a multiple of 64
    K2 = 1000
    x2 = torch.randn(M, K2, device=DEV).to(torch.bfloat16)
    w2 = torch.randint(-127, 128, (N, K2), dtype=torch.int8, device=DEV).t()
    assert torch.equal(torch.ops.vllm.qf_int8_linear(x2, w2, s, None), P.w8a8_reference(x2, w2, s, None, torch.bfloat16))


def test_two_streams_overlap_with_own_workspaces(oracle):
    """Fused split-K GEMMs (down's shape at M = 5, K split three ways) and row-split argmaxes issued on two
    same-priority streams without synchronisation between them equal the same calls run in order."""
    N, K = 5120, 17408
    img = torch.randint(-127, 128, (qf.tiled_numel(N, K),), dtype=torch.int8, device=DEV)
    s = torch.rand(N, device=DEV) * 0.002 + 1e-4
    cfg = qf.resolve_config(5, N, K, qf.TILED)
    assert cfg.split_k > 1 and cfg.reduce == 0, cfg
    xs = [torch.randn(5, K, device=DEV).to(torch.bfloat16) for _ in range(8)]
    logits = [torch.randn(4, 40000, device=DEV).to(torch.bfloat16) for _ in range(8)]
    want_y = [qf.w8a16_mm(x, img, s, None, torch.bfloat16, qf.TILED) for x in xs]
    want_i = [P.top_tokens(lg, 7, 100) for lg in logits]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    got_y, got_i = [None] * 8, [None] * 8
    for rep in range(3):
        for j in range(8):
            with torch.cuda.stream(streams[j % 2]):
                got_y[j] = qf.w8a16_mm(xs[j], img, s, None, torch.bfloat16, qf.TILED)
                got_i[j] = P.top_tokens(logits[j], 7, 100)
        torch.cuda.synchronize()
        for j in range(8):
            assert torch.equal(got_y[j], want_y[j]), f"rep {rep} call {j}: split-K result differs"
            assert torch.equal(got_i[j], want_i[j]), f"rep {rep} call {j}: argmax differs"
    ref = torch.argmax(torch.where(torch.arange(40000, device=DEV) < 40000 - 7, logits[0].float(),
                                   torch.tensor(float("-inf"), device=DEV)), dim=-1) + 100
    assert torch.equal(want_i[0], ref)


def test_two_streams_w8a8_tile_split_overlap():
    """W8A8 calls on the LDS-tiled kernel with its K split three ways (the last split of each tile adds the
    others' int32 partials through the stream's workspace) issued on two same-priority streams without
    synchronisation between them equal the same calls run in order, and the restatement."""
    M, N, K = 512, 1024, 8192
    w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=DEV)
    wt = qf.to_tiled(w.t())
    s = torch.rand(N, device=DEV) * 0.002 + 1e-4
    cfg = (L.KERNEL_MFMA_W8A8_TILE, 3, 8, 8, 4, 1, 1, 0)
    xs = [torch.randn(M, K, device=DEV).to(torch.bfloat16) for _ in range(6)]
    want = [qf.w8a8_mm(x, wt, s, torch.bfloat16, cfg) for x in xs]
    ref0 = P.w8a8_reference(xs[0], w.t(), s, None, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(want[0].view(torch.int16), ref0.view(torch.int16))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    got = [None] * 6
    for rep in range(3):
        for j in range(6):
            with torch.cuda.stream(streams[j % 2]):
                got[j] = qf.w8a8_mm(xs[j], wt, s, torch.bfloat16, cfg)
        torch.cuda.synchronize()
        for j in range(6):
            assert torch.equal(got[j].view(torch.int16), want[j].view(torch.int16)), f"rep {rep} call {j}"


def test_capture_without_warmup(oracle):
    """The first split-K call on a fresh stream happens inside the capture: its workspace is the
    capture's own, its counters cleared by a fill kernel recorded into the graph."""
    N, K = 1024, 17408
    inp, x, w, s = _inputs(oracle, 5, N, K, 15)
    img = qf.to_tiled(w)
    cfg = qf.W8A16Config(2, 4, 1, 8, 4, 1, 2, 0)  # fused four-way K split
    eager = qf.w8a16_mm(x, img, s, cfg, torch.bfloat16, qf.TILED)
    st = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        y = qf.w8a16_mm(x, img, s, cfg, torch.bfloat16, qf.TILED)
    for _ in range(4):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
        qf.w8a16_mm(x, img, s, cfg, torch.bfloat16, qf.TILED)  # eager call between replays
    assert oracle.check_w8a16(bf16_bits(eager), inp.x, inp.w, inp.s).ok


def test_capture_workspaces_released_between_captures(oracle):
    """A capture's workspace is held by the package only while that capture is the latest on its stream.
    Three graphs captured one after another on one stream (split-K calls of three widths, whose workspaces
    differ in size; the third shares the second's memory pool) replay correctly, in any order and with
    eager calls between replays, after the earlier captures' workspaces were released; the package then
    holds the buffers of the last capture only."""
    from qwen_fastpath import w8a16 as W
    N, K = 1024, 17408
    inp, x16, w, s = _inputs(oracle, 16, N, K, 21)
    img = qf.to_tiled(w)
    cfg = qf.W8A16Config(2, 4, 1, 8, 4, 1, 2, 0)  # fused four-way K split: partials sized by M
    st = torch.cuda.Stream()
    graphs, outs, want = [], [], []
    for i, M in enumerate((5, 16, 9)):
        x = x16[:M]
        want.append(qf.w8a16_mm(x, img, s, cfg, torch.bfloat16, qf.TILED))
        g = torch.cuda.CUDAGraph()
        pool = graphs[1].pool() if i == 2 else None
        with torch.cuda.graph(g, stream=st, pool=pool):
            outs.append(qf.w8a16_mm(x, img, s, cfg, torch.bfloat16, qf.TILED))
        graphs.append(g)
        held = [k for k in W._capture_ws if k[1] == st.cuda_stream]
        assert len(held) == 1 and len(W._capture_ws[held[0]][1]) == 1, W._capture_ws
    torch.cuda.synchronize()
    junk = [torch.randn(1 << 20, device=DEV) for _ in range(8)]  # allocations between capture and replay
    for rep, order in enumerate(((0, 1, 2), (2, 0, 1), (1, 2, 0))):
        for j in order:
            outs[j].zero_()
            graphs[j].replay()
            torch.cuda.synchronize()
            assert torch.equal(outs[j], want[j]), (rep, j)
            qf.w8a16_mm(x16[:7], img, s, cfg, torch.bfloat16, qf.TILED)  # eager call between replays
    del junk
    for M, y in zip((5, 16, 9), want):
        assert oracle.check_w8a16(bf16_bits(y), inp.x[:M], inp.w, inp.s).ok
