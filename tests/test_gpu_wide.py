"""GPU parity of the wide-M kernel (QF_KERNEL_MFMA_WIDE: TILED weights, M > 16) against the oracle
(the tolerance rule of oracle.check_w8a16) and, bit for bit, against the decode kernel run over 16-row
slices with one k-slice and the same K split (partials summed by the same second-pass kernel).  Both
sum every output over each split's k-steps in the same order with the same MFMA instruction and apply
the scale the same way, so their results must be identical."""
import pytest
import torch

import qwen_fastpath as qf
from qwen_fastpath import _lib as L
from helpers import bf16_bits, dev_inputs

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def wide(nt, waves, depth, split=1):
    return (L.KERNEL_MFMA_WIDE, split, nt, waves, depth, 1, 1, 1)


def slices(x, wt, s, out=torch.bfloat16, split=1):
    """The decode kernel (x ring, 1 tile x 4 wavefronts, depth 4, non-temporal loads, one k-slice,
    second-pass split reduction) over 16-row slices."""
    cfg = (L.KERNEL_MFMA_XRING, split, 1, 4, 4, 1, 1, 1)
    return torch.cat([qf.w8a16_mm(x[i:i + 16], wt, s, cfg, out, qf.TILED) for i in range(0, x.shape[0], 16)])


def auto_split(M, N, K):
    c = qf.resolve_config(M, N, K, qf.TILED)
    assert c.kernel == L.KERNEL_MFMA_WIDE
    return c.split_k


def bits(t):
    return t.view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32)


def random_layer(N, K, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, device=DEV, generator=g)
    s = (torch.rand(N, device=DEV, generator=g) * 0.004 + 1e-4).float()
    return qf.to_tiled(w.t()), s, g


@pytest.mark.parametrize("M", [17, 33, 64, 65, 130, 200])
def test_wide_against_oracle(oracle, M):
    N, K = 1000, 2048
    inp = oracle.gen_inputs(M, N, K, seed=100 + M)
    x, w, s = dev_inputs(inp, DEV)
    wt = qf.to_tiled(w)
    split = auto_split(M, N, K)
    y = qf.w8a16_mm(x, wt, s, None, torch.bfloat16, qf.TILED)
    torch.cuda.synchronize()
    rep = oracle.check_w8a16(bf16_bits(y), inp.x, inp.w, inp.s)
    print(f"wide M={M} N={N} K={K}: {rep}", flush=True)
    assert rep.ok, rep
    assert torch.equal(bits(y), bits(slices(x, wt, s, split=split)))


WIDE_SHAPES = [(nt, waves, depth) for nt in (1, 2) for waves in (4, 8) for depth in (4, 8)] + [(4, 4, 2)]


@pytest.mark.parametrize("nt,waves,depth", WIDE_SHAPES)
def test_wide_configs_bitwise(nt, waves, depth):
    """Every instantiated (tiles, wavefronts, depth) at 1..4 token tiles and 1..3 groups, a ragged N
    and a chunk count that does not divide the k-steps, bf16 and fp32 outputs."""
    N, K = 1000, 1024
    wt, s, g = random_layer(N, K, 11 + nt + waves + depth)
    x = torch.randn(160, K, device=DEV, generator=g).to(torch.bfloat16)
    for M in (1, 16, 20, 32, 48, 64, 100, 129, 160):
        y = qf.w8a16_mm(x[:M], wt, s, wide(nt, waves, depth), torch.bfloat16, qf.TILED)
        ref = slices(x[:M], wt, s)
        torch.cuda.synchronize()
        assert torch.equal(bits(y), bits(ref)), (nt, waves, depth, M)
    y = qf.w8a16_mm(x[:48], wt, s, wide(nt, waves, depth), torch.float32, qf.TILED)
    assert torch.equal(bits(y), bits(slices(x[:48], wt, s, torch.float32)))
    for split in (2, 3, 5):  # K splits (16 k-steps: uneven ranges at 3 and 5)
        y = qf.w8a16_mm(x[:100], wt, s, wide(nt, waves, depth, split), torch.bfloat16, qf.TILED)
        assert torch.equal(bits(y), bits(slices(x[:100], wt, s, split=split))), (nt, waves, depth, split)


def test_wide_edges_bitwise():
    """One k-step, one output channel, a strided x (row stride > K), and a 16-row tail group."""
    for (N, K) in ((1, 64), (17, 64), (33, 192), (5120, 64)):
        wt, s, g = random_layer(N, K, N + K)
        xw = torch.randn(80, K + 64, device=DEV, generator=g).to(torch.bfloat16)
        x = xw[:, :K]
        for M in (17, 64, 80):
            y = qf.w8a16_mm(x[:M], wt, s, None, torch.bfloat16, qf.TILED)
            torch.cuda.synchronize()
            assert torch.equal(bits(y), bits(slices(x[:M], wt, s, split=auto_split(M, N, K)))), (N, K, M)


@pytest.mark.parametrize("name,N,K", [("gate_up", 34816, 5120), ("o_proj", 5120, 8192), ("down", 5120, 17408),
                                      ("qkv", 10240, 5120)])
def test_wide_layer_shapes_bitwise(name, N, K):
    """The dense 27B-class layer's shapes at prefill-chunk widths, with the automatic configuration."""
    wt, s, g = random_layer(N, K, N ^ K)
    x = torch.randn(256, K, device=DEV, generator=g).to(torch.bfloat16)
    for M in (24, 64, 96, 256):
        y = qf.w8a16_mm(x[:M], wt, s, None, torch.bfloat16, qf.TILED)
        ref = slices(x[:M], wt, s, split=auto_split(M, N, K))
        torch.cuda.synchronize()
        print(f"{name} M={M} cfg={tuple(qf.resolve_config(M, N, K, qf.TILED))}", flush=True)
        assert torch.equal(bits(y), bits(ref)), (name, M)


def test_wide_and_widened_paths_in_a_graph():
    """The wide-M kernel with a K split (workspace + second-pass sum), without one, the widened-weights
    path (widening, library GEMM, scale/cast) and the W8A8 route (quantiser + int8 GEMM, with and
    without a K split, and the LDS-tiled int8 kernel) captured in one graph: four replays with eager work
    and zeroed outputs between them, each bitwise equal to the eager results."""
    cases = []
    for (M, N, K, seed) in ((40, 1000, 2048, 1), (300, 2000, 1024, 2)):
        wt, s, g = random_layer(N, K, seed)
        x = torch.randn(M, K, device=DEV, generator=g).to(torch.bfloat16)
        cases.append((x, wt, s))
    assert qf.resolve_config(40, 1000, 2048, qf.TILED).split_k > 1
    assert qf.resolve_config(300, 2000, 1024, qf.TILED).split_k == 1

    from qwen_fastpath import _lib as L
    assert L.w8a8_pick_config(40, 1000, 2048).split_k > 1

    def work():
        outs = [qf.w8a16_mm(x, wt, s, None, torch.bfloat16, qf.TILED) for (x, wt, s) in cases]
        x, wt, s = cases[1]
        outs.append(qf.w8a16_mm_prefill(x, wt, s, torch.bfloat16, qf.TILED, chunk_rows=768))
        outs += [qf.w8a8_mm(x, wt, s, torch.bfloat16) for (x, wt, s) in cases]  # quantiser + int8 GEMM
        outs.append(qf.w8a8_mm(x, wt, s, torch.bfloat16, (L.KERNEL_MFMA_W8A8_TILE, 1, 8, 8, 4, 1, 1, 1)))
        outs.append(qf.w8a8_mm(x, wt, s, torch.bfloat16, (L.KERNEL_MFMA_W8A8_TILE, 3, 8, 8, 4, 1, 1, 1)))  # fused K split
        return outs

    eager = [o.clone() for o in work()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        work()  # warm-up off the default stream (allocates the split-K workspace)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = work()
    torch.cuda.synchronize()
    for rep in range(4):
        for o in outs:
            o.fill_(0)
        junk = torch.randn(1 << 20, device=DEV).sum()  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(bits(o), bits(e)), (rep, i)
        del junk
