"""GPU parity of the stream kernel (QF_KERNEL_MFMA_STREAM: one workgroup per CU over a contiguous run of
16-row tiles, every wavefront splitting K, the prefetch ring running across tile boundaries), explicit
configurations, against the oracle (oracle.check_w8a16: every output within 1 bf16 ulp of the exact product
plus the fp32 floor).  Shapes where the runs are ragged: N not a multiple of 16 (a zero-padded last tile),
fewer tiles than CUs (idle workgroups), runs of 1 to 5 tiles, K equal to the wavefront count, 8 and 16
wavefronts, each instantiated depth; bf16 and fp32 outputs, padded output rows and rows that break vector
alignment; bitwise repeatability; rows computed independently of M."""
import numpy as np
import pytest
import torch

import qwen_fastpath as qf
from qwen_fastpath import _lib as L
from helpers import bf16_bits, dev_inputs

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
STREAM = L.KERNEL_MFMA_STREAM


def cfg(waves, depth):
    return qf.W8A16Config(STREAM, 1, 1, waves, depth, 1, waves, 0)


def run(x, img, s, c, out_dtype=torch.bfloat16):
    return qf.w8a16_mm(x, img, s, c, out_dtype, qf.TILED)


@pytest.mark.parametrize("M,N,K", [(5, 1000, 1024), (3, 16, 512), (8, 4100, 2048), (2, 5120, 5120),
                                   (5, 24592, 512), (1, 1, 640), (7, 300, 8192)])
@pytest.mark.parametrize("waves,depth", [(8, 4), (8, 2), (8, 3), (8, 5), (8, 6), (8, 8), (8, 12), (8, 16),
                                         (16, 2), (16, 4), (16, 8)])
def test_stream_against_oracle(oracle, M, N, K, waves, depth):
    if K // 64 < waves:
        pytest.skip("K has fewer 64-k steps than wavefronts")
    inp = oracle.gen_inputs(M, N, K, seed=M * 131 + N + K)
    x, w, s = dev_inputs(inp, DEV)
    img = qf.to_tiled(w)
    c = cfg(waves, depth)
    print(f"stream M={M} N={N} K={K} cfg={tuple(c)}", flush=True)
    y = run(x, img, s, c)
    y2 = run(x, img, s, c)
    torch.cuda.synchronize()
    rep = oracle.check_w8a16(bf16_bits(y), inp.x, inp.w, inp.s)
    assert rep.ok, (M, N, K, waves, depth, rep)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))  # bitwise repeatable


def test_stream_outputs_and_row_independence(oracle):
    """fp32 output, a padded output row stride and one that breaks 8-byte alignment (scalar stores), each equal
    to the bf16-output bits where they should be; row m of an M-row call equals the same row computed alone."""
    M, N, K = 6, 2000, 2048
    inp = oracle.gen_inputs(M, N, K, seed=5)
    x, w, s = dev_inputs(inp, DEV)
    img = qf.to_tiled(w)
    c = cfg(8, 4)
    y = run(x, img, s, c)
    y32 = run(x, img, s, c, torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(y32.to(torch.bfloat16).view(torch.int16), y.view(torch.int16))
    assert oracle.check_w8a16(bf16_bits(y), inp.x, inp.w, inp.s).ok
    lib = L.load()
    import ctypes
    for ldy in (N + 8, N + 3):
        yp = torch.full((M, ldy), float("nan"), dtype=torch.bfloat16, device=DEV)
        cs = L.Config.from_seq(tuple(c))
        rc = lib.qf_w8a16_gemm(x.data_ptr(), K, img.data_ptr(), K, qf.TILED, s.data_ptr(), yp.data_ptr(), ldy,
                               L.DTYPE_BF16, M, N, K, ctypes.byref(cs), None, 0, torch.cuda.current_stream().cuda_stream)
        L.check(rc, "stream padded ldy")
        torch.cuda.synchronize()
        assert torch.equal(yp[:, :N].view(torch.int16), y.view(torch.int16)), ldy
        assert torch.isnan(yp[:, N:].float()).all(), ldy
    for m in range(M):
        ym = run(x[m:m + 1].contiguous(), img, s, c)
        torch.cuda.synchronize()
        assert torch.equal(ym.view(torch.int16), y[m:m + 1].view(torch.int16)), m


def test_stream_auto_gate_up_graph_replay(oracle):
    """The automatic choice at gate_up's shape and M = 4 is the stream kernel; inside a graph its replays equal
    the eager call bit for bit, and the eager call passes the oracle."""
    M, N, K = 4, 34816, 5120
    assert qf.resolve_config(M, N, K, qf.TILED).kernel == STREAM
    inp = oracle.gen_inputs(M, N, K, seed=9)
    x, w, s = dev_inputs(inp, DEV)
    img = qf.to_tiled(w)
    eager = qf.w8a16_mm(x, img, s, None, torch.bfloat16, qf.TILED)
    st = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        y = qf.w8a16_mm(x, img, s, None, torch.bfloat16, qf.TILED)
    for rep in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), eager.view(torch.int16)), rep
    assert oracle.check_w8a16(bf16_bits(eager), inp.x, inp.w, inp.s).ok


@pytest.mark.parametrize("M,N,K", [(5, 1000, 5120), (16, 4100, 5120), (1, 16, 5120), (9, 34816, 5120),
                                   (12, 3000, 8192), (3, 300, 4096), (16, 24592, 4096)])
@pytest.mark.parametrize("waves,depth", [(8, 4), (8, 9), (8, 3), (8, 7), (16, 4)])
def test_stream_xreg_against_oracle(oracle, M, N, K, waves, depth):
    """x fragments held in registers (reduce 1, K = 64 W S for the instantiated S): passes the oracle at every M
    up to 16, and equals the LDS-staged stream kernel at the same wavefront count bit for bit wherever the
    latter's x slice fits in LDS (the same steps summed in the same order)."""
    xreg = qf.W8A16Config(STREAM, 1, 1, waves, depth, 1, waves, 1)
    inp = oracle.gen_inputs(M, N, K, seed=M + 7 * N + K)
    x, w, s = dev_inputs(inp, DEV)
    img = qf.to_tiled(w)
    print(f"stream xreg M={M} N={N} K={K} cfg={tuple(xreg)}", flush=True)
    try:
        y = run(x, img, s, xreg)
    except L.QFError as e:  # refused before any launch: no instantiation for this (K, waves, depth)
        assert e.status == L.ERR_UNSUPPORTED, e
        pytest.skip("not instantiated for this K")
    torch.cuda.synchronize()
    rep = oracle.check_w8a16(bf16_bits(y), inp.x, inp.w, inp.s)
    assert rep.ok, (M, N, K, waves, depth, rep)
    for lds_depth in ((2, 4, 8) if waves == 16 else (4,)):
        lds = qf.W8A16Config(STREAM, 1, 1, waves, lds_depth, 1, waves, 0)
        try:
            y_lds = run(x, img, s, lds)
        except L.QFError:
            continue  # the x slice does not fit beside the partial tiles
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y_lds.view(torch.int16)), (M, N, K, waves, lds_depth)


@pytest.mark.parametrize("M,N,K", [(5, 4100, 5120), (3, 1000, 2048), (9, 20000, 5120), (2, 16, 512)])
def test_stream_grid_variants_bitwise(M, N, K):
    """Which workgroup sums a tile does not change how it is summed: the strided assignment (reduce bit 1) and
    runs of a fixed tile count (reduce bit 2, tiles_per_wave 1..3: several workgroups a CU) give the bits of the
    default grid (one contiguous run per CU), with x staged in LDS or held in registers."""
    g = torch.Generator(device=DEV)
    g.manual_seed(M + N + K)
    x = torch.randn(M, K, device=DEV, generator=g).to(torch.bfloat16)
    img = torch.randint(-127, 128, (qf.tiled_numel(N, K),), dtype=torch.int8, device=DEV, generator=g)
    s = (torch.rand(N, device=DEV, generator=g) * 0.002 + 1e-4).float()
    for xreg in (0, 1):
        base = None
        for bits in (0, 2, 4, 6):
            for tpw in ((1, 2, 3) if bits & 4 else (1,)):
                c = qf.W8A16Config(STREAM, 1, tpw, 8, 4, 1, 8, bits | xreg)
                print(f"stream grid M={M} N={N} K={K} cfg={tuple(c)}", flush=True)
                try:
                    y = run(x, img, s, c)
                except L.QFError as e:
                    assert e.status == L.ERR_UNSUPPORTED, e
                    continue  # no register-x build for this K, or LDS too small
                torch.cuda.synchronize()
                if base is None:
                    base = y
                assert torch.equal(y.view(torch.int16), base.view(torch.int16)), (M, N, K, tuple(c))
