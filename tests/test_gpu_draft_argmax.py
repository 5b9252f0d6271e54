"""The draft head's argmax fused into the W8A16 kernel (qf_w8a16_gemm_argmax): the ids must equal the
pad-masked argmax of the bf16 logits the plain kernel writes (plugin/qwen_fastpath/patches.py:178-185),
and the oracle's argmax of those logits, bit for bit -- with planted ties (first index wins, -0.0 and
+0.0 tie), a NaN row (NaN is the maximum), rows of negative logits, a winner planted in the pad columns
(ignored), several grid sizes, repeated calls (the per-token slots are cleared for the next call) and
graph replay."""
import numpy as np
import pytest
import torch

import qwen_fastpath as qf
from qwen_fastpath import patches as P

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _head(N, K, seed, plant=True):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=DEV, generator=g)
    s = (torch.rand(N, device=DEV, generator=g) * 0.002 + 1e-4).float()
    if plant:
        w[7] = 127                     # a strong row ...
        w[N // 2 + 3] = 127            # ... and an identical later row: the tie goes to row 7
        s[N // 2 + 3] = s[7]
        w[N - 2] = 127                 # a winner inside the pad columns (ignored when num_pad >= 2)
        s[N - 2] = 1.0
    return w, s


def _ref_ids(y_bits, n_valid, offset, oracle):
    return oracle.argmax_rows(y_bits, n_valid, offset)


@pytest.mark.parametrize("layout", [qf.TILED, qf.ROWMAJOR])
@pytest.mark.parametrize("M", [1, 2, 4, 7, 8, 12, 16])
@pytest.mark.parametrize("N,K", [(151936, 5120), (5000, 1024), (1000, 256)])
def test_fused_ids_equal_unfused(oracle, layout, M, N, K):
    w, s = _head(N, K, seed=N + M)
    wt = w.t()
    wl = qf.to_tiled(wt) if layout == qf.TILED else wt
    g = torch.Generator(device=DEV)
    g.manual_seed(M)
    x = torch.rand(M, K, device=DEV, generator=g).to(torch.bfloat16)  # positive: row 7 is a clear maximum
    x[M - 1] = torch.randn(K, device=DEV, generator=g).to(torch.bfloat16)  # a random row too
    num_pad, offset = 64, 1234
    y = qf.w8a16_mm(x, wl, s, None, torch.bfloat16, layout)
    torch.cuda.synchronize()
    ref = qf.top_tokens(y, num_pad, offset).cpu().numpy()
    y_bits = y.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(ref, _ref_ids(y_bits, N - num_pad, offset, oracle))
    for rep in range(2):  # the per-token slots are back at zero for the next call
        res = qf.w8a16_mm_argmax(x, wl, s, N - num_pad, offset, None, layout, with_logits=True)
        if res is None:  # configurations without the fused epilogue (GEMV, split K)
            assert qf.w8a16_mm_argmax(x, wl, s, N - num_pad, offset, None, layout) is None
            return
        ids, y2 = res
        torch.cuda.synchronize()
        assert np.array_equal(ids.cpu().numpy(), ref), (rep, ids.cpu().numpy(), ref)
        assert torch.equal(y2.view(torch.int16), y.view(torch.int16))
        ids_only = qf.w8a16_mm_argmax(x, wl, s, N - num_pad, offset, None, layout)
        assert np.array_equal(ids_only.cpu().numpy(), ref)


def test_nan_row_and_all_pad_winner(oracle):
    N, K, M = 3000, 512, 3
    w, s = _head(N, K, seed=5, plant=False)
    s[11] = float("nan")               # every logit of column 11 is NaN: NaN is the maximum
    wl = qf.to_tiled(w.t())
    x = torch.randn(M, K, device=DEV).to(torch.bfloat16)
    ids = qf.w8a16_mm_argmax(x, wl, s, N, 0, None, qf.TILED)
    assert ids is not None
    assert ids.cpu().tolist() == [11] * M
    ids = qf.w8a16_mm_argmax(x, wl, s, 11, 0, None, qf.TILED)   # NaN column excluded by n_valid
    y = qf.w8a16_mm(x, wl, s, None, torch.bfloat16, qf.TILED)
    ref = qf.top_tokens(y, N - 11, 0)
    assert torch.equal(ids, ref)


def test_graph_replay():
    N, K, M = 151936, 5120, 1
    w, s = _head(N, K, seed=3)
    wl = qf.to_tiled(w.t())
    x = torch.randn(M, K, device=DEV).to(torch.bfloat16)
    eager = qf.w8a16_mm_argmax(x, wl, s, N - 64, 7, None, qf.TILED)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        qf.w8a16_mm_argmax(x, wl, s, N - 64, 7, None, qf.TILED)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = qf.w8a16_mm_argmax(x, wl, s, N - 64, 7, None, qf.TILED)
    for i in range(3):
        out.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i


def test_int8_top_tokens_matches_two_step(oracle):
    V, H = 151936, 5120
    wf = (torch.randn(V, H, device=DEV) * 0.02).to(torch.bfloat16)
    head = P.make_int8_head(wf, num_pad=64)
    del wf
    for M in (1, 4):
        hs = torch.randn(M, H, device=DEV).to(torch.bfloat16)
        ids = P.int8_top_tokens(head, hs, 100)
        dflt = P.int8_top_tokens(head, hs, 100, fused=False)
        two = P.top_tokens(P.int8_logits(head, hs), 64, 100)
        torch.cuda.synchronize()
        assert torch.equal(ids, two) and torch.equal(dflt, two)


@pytest.mark.parametrize("layout", [qf.TILED, qf.ROWMAJOR])
def test_signed_zero_tie_and_negative_logits(oracle, layout):
    """-0.0 and +0.0 are equal maxima (the first index wins, as in torch.argmax), and a row whose logits are
    all negative picks the least negative one."""
    N, K, M = 3000, 512, 2
    g = torch.Generator(device=DEV)
    g.manual_seed(17)
    w = torch.full((N, K), 127, dtype=torch.int8, device=DEV)
    w[5] = 0
    w[9] = 0
    s = torch.full((N,), -0.01, dtype=torch.float32, device=DEV)
    s[9] = 0.01                       # column 9: +0.0; column 5: -0.0 (a zero sum times a negative scale)
    wl = qf.to_tiled(w.t()) if layout == qf.TILED else w.t()
    x = (torch.rand(M, K, device=DEV, generator=g) + 0.1).to(torch.bfloat16)
    y = qf.w8a16_mm(x, wl, s, None, torch.bfloat16, layout)
    torch.cuda.synchronize()
    yb = y.view(torch.int16).cpu().numpy().view(np.uint16)
    assert (yb[:, 5] == 0x8000).all() and (yb[:, 9] == 0).all()
    ref = qf.top_tokens(y, 0, 0)
    assert ref.cpu().tolist() == [5] * M
    ids = qf.w8a16_mm_argmax(x, wl, s, N, 0, None, layout)
    if ids is None:
        pytest.skip("no fused epilogue for this configuration")
    assert torch.equal(ids, ref)
    # all logits negative: random positive weights, negative scales
    w2 = torch.randint(1, 128, (N, K), dtype=torch.int8, device=DEV, generator=g)
    s2 = -(torch.rand(N, device=DEV, generator=g) * 0.002 + 1e-4).float()
    wl2 = qf.to_tiled(w2.t()) if layout == qf.TILED else w2.t()
    y2 = qf.w8a16_mm(x, wl2, s2, None, torch.bfloat16, layout)
    torch.cuda.synchronize()
    assert (y2.float() < 0).all()
    ref2 = qf.top_tokens(y2, 0, 3)
    y2b = y2.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(ref2.cpu().numpy(), _ref_ids(y2b, N, 3, oracle))
    ids2 = qf.w8a16_mm_argmax(x, wl2, s2, N, 3, None, layout)
    assert torch.equal(ids2, ref2)


@pytest.mark.parametrize("M,N,K", [(1, 151936, 5120), (16, 151936, 5120), (7, 1000, 4096), (5, 5000, 1024)])
def test_caller_workspace_prefix_back_at_zero(M, N, K):
    """Through the C ABI with a caller workspace: after every call the counter prefix (the per-token slots) is all
    zero again, and bytes past the prefix (split-K partials of earlier calls on a shared workspace) do not matter;
    grids of more and fewer workgroups than slots."""
    import ctypes
    from qwen_fastpath import _lib as L
    lib = L.load()
    w, s = _head(N, K, seed=M + N)
    wl = qf.to_tiled(w.t())
    g = torch.Generator(device=DEV)
    g.manual_seed(K)
    x = torch.randn(M, K, device=DEV, generator=g).to(torch.bfloat16)
    n_valid = N - 64
    ref = qf.top_tokens(qf.w8a16_mm(x, wl, s, None, torch.bfloat16, qf.TILED), 64, 11)
    cfg = L.Config.from_seq((0,) * 8)
    need = int(lib.qf_w8a16_argmax_workspace_bytes(M, N, K, qf.TILED, ctypes.byref(cfg)))
    assert need == L.COUNTER_BYTES
    ws = torch.full((need + (1 << 20),), 0xA5, dtype=torch.uint8, device=DEV)
    ws[:L.COUNTER_BYTES].zero_()
    stream = torch.cuda.current_stream().cuda_stream
    print(f"argmax workspace M={M} N={N} K={K}", flush=True)
    for rep in range(3):
        ids = torch.full((M,), -1, dtype=torch.int64, device=DEV)
        rc = lib.qf_w8a16_gemm_argmax(x.data_ptr(), K, wl.data_ptr(), K, qf.TILED, s.data_ptr(), None, N,
                                      L.DTYPE_BF16, M, N, K, n_valid, 11, ids.data_ptr(), ctypes.byref(cfg),
                                      ws.data_ptr(), ws.numel(), stream)
        assert rc == L.OK, rc
        torch.cuda.synchronize()
        assert torch.equal(ids, ref), (rep, ids.tolist(), ref.tolist())
        assert int(torch.count_nonzero(ws[:L.COUNTER_BYTES])) == 0, rep
