"""GPU test of qf_w8a16_gemm_noalloc, the entry point that allocates nothing (its split-K workspace is a
static device array): through the C ABI it gives the bits of qf_w8a16_gemm with the same configuration,
on two calls in a row of which the second is smaller (and reads scratch the first left behind), for a
fused last-arrival K split and a second-pass K split; a call needing more than the scratch is refused
before anything is launched."""
import ctypes

import pytest
import torch

import qwen_fastpath as qf
from qwen_fastpath import _lib as L

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _gemm(lib, x, img, s, N, K, cfg, noalloc):
    M = x.shape[0]
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    c = L.Config.from_seq(cfg)
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.qf_w8a16_gemm_noalloc(x.data_ptr(), K, img.data_ptr(), K, L.LAYOUT_TILED, s.data_ptr(), y.data_ptr(),
                                       N, L.DTYPE_BF16, M, N, K, ctypes.byref(c), stream)
    else:
        nbytes = int(lib.qf_w8a16_workspace_bytes(M, N, K, L.LAYOUT_TILED, ctypes.byref(c)))
        ws = torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=DEV)
        rc = lib.qf_w8a16_gemm(x.data_ptr(), K, img.data_ptr(), K, L.LAYOUT_TILED, s.data_ptr(), y.data_ptr(), N,
                               L.DTYPE_BF16, M, N, K, ctypes.byref(c), ws.data_ptr(), ws.numel(), stream)
    L.check(rc, "noalloc" if noalloc else "gemm")
    torch.cuda.synchronize()
    return y


def _case(M, N, K, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    x = torch.randn(M, K, device=DEV, generator=g).to(torch.bfloat16)
    img = torch.randint(-127, 128, (qf.tiled_numel(N, K),), dtype=torch.int8, device=DEV, generator=g)
    s = torch.rand(N, device=DEV, generator=g) * 0.002 + 1e-4
    return x, img, s


def test_noalloc_first_call_inside_graph_capture():
    """The file's first test, so that in a fresh process the library's first no-alloc call on the device
    happens inside a graph capture: the scratch address is fetched there and its counter-clearing kernel is
    recorded into the graph.  The graph, replayed three times with eager calls of both entry points between
    the replays, equals qf_w8a16_gemm bit for bit (a fused four-way K split, whose counters must start at zero
    on every replay)."""
    lib = L.load()
    M, N, K, cfg = 5, 1024, 17408, (2, 4, 1, 8, 4, 1, 2, 0)
    x, img, s = _case(M, N, K, 7)
    c = L.Config.from_seq(cfg)
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    st = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    print("noalloc: capturing the first call", flush=True)
    with torch.cuda.graph(g, stream=st):
        rc = lib.qf_w8a16_gemm_noalloc(x.data_ptr(), K, img.data_ptr(), K, L.LAYOUT_TILED, s.data_ptr(),
                                       y.data_ptr(), N, L.DTYPE_BF16, M, N, K, ctypes.byref(c),
                                       torch.cuda.current_stream().cuda_stream)
    L.check(rc, "noalloc inside capture")
    want = _gemm(lib, x, img, s, N, K, cfg, noalloc=False)
    for rep in range(3):
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16)), rep
        eager = _gemm(lib, x, img, s, N, K, cfg, noalloc=True)
        assert torch.equal(eager.view(torch.int16), want.view(torch.int16)), rep


# (M, N, K, config): the first call of each pair is the larger one
PAIRS = [
    ((5, 5120, 17408, (2, 3, 1, 8, 4, 1, 2, 0)), (3, 1024, 8192, (2, 4, 1, 8, 4, 1, 2, 0))),   # fused split
    ((16, 10240, 5120, (2, 3, 1, 8, 4, 1, 1, 1)), (7, 2048, 5120, (2, 2, 1, 8, 4, 1, 1, 1))),  # second pass
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_gemm_two_calls(first, second):
    lib = L.load()
    for (M, N, K, cfg), seed in ((first, 1), (second, 2)):
        need = int(lib.qf_w8a16_workspace_bytes(M, N, K, L.LAYOUT_TILED, ctypes.byref(L.Config.from_seq(cfg))))
        assert 0 < need <= L.SCRATCH_BYTES
        x, img, s = _case(M, N, K, seed)
        want = _gemm(lib, x, img, s, N, K, cfg, noalloc=False)
        got = _gemm(lib, x, img, s, N, K, cfg, noalloc=True)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (M, N, K, cfg)
        again = _gemm(lib, x, img, s, N, K, cfg, noalloc=True)  # counters were left at zero
        assert torch.equal(again.view(torch.int16), want.view(torch.int16)), (M, N, K, cfg)


def test_noalloc_refuses_oversize_before_launch():
    lib = L.load()
    M, N, K = 16, 34816, 5120
    c = L.Config.from_seq((2, 4, 1, 8, 4, 1, 1, 1))
    assert int(lib.qf_w8a16_workspace_bytes(M, N, K, L.LAYOUT_TILED, ctypes.byref(c))) > L.SCRATCH_BYTES
    x = torch.zeros(M, K, dtype=torch.bfloat16, device=DEV)
    img = torch.zeros(qf.tiled_numel(N, K), dtype=torch.int8, device=DEV)
    s = torch.ones(N, device=DEV)
    y = torch.zeros(M, N, dtype=torch.bfloat16, device=DEV)
    rc = lib.qf_w8a16_gemm_noalloc(x.data_ptr(), K, img.data_ptr(), K, L.LAYOUT_TILED, s.data_ptr(), y.data_ptr(), N,
                                   L.DTYPE_BF16, M, N, K, ctypes.byref(c), torch.cuda.current_stream().cuda_stream)
    assert rc == L.ERR_WORKSPACE
    torch.cuda.synchronize()
    assert int(y.view(torch.int16).abs().sum()) == 0
