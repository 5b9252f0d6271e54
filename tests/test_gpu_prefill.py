"""GPU tests of the M > 16 path on TILED weights: the exact int8 -> bf16 widening of weight rows from
either layout, and the chunked library bf16 GEMM with fp32 accumulation and the scale after the K
reduction, against the oracle's tolerance rule."""
import numpy as np
import pytest
import torch

import qwen_fastpath as qf
from helpers import bf16_bits, dev_inputs, to_dev_bf16

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.mark.parametrize("layout", [qf.ROWMAJOR, qf.TILED])
def test_dequant_rows_exact(layout):
    N, K = 1000, 2048
    g = torch.Generator(device=DEV)
    g.manual_seed(3)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, device=DEV, generator=g)
    src = w.t() if layout == qf.ROWMAJOR else qf.to_tiled(w.t())
    for n0, rows in ((0, N), (37, 100), (512, 488), (999, 1)):
        out = qf.dequant_bf16(src, N, K, layout, n0, rows)
        assert torch.equal(out, w[n0:n0 + rows].float().to(torch.bfloat16)), (layout, n0, rows)
    # into a wider buffer (row stride > K)
    buf = torch.zeros((64, K + 64), dtype=torch.bfloat16, device=DEV)
    qf.dequant_bf16(src, N, K, layout, 100, 64, buf)
    assert torch.equal(buf[:, :K], w[100:164].float().to(torch.bfloat16))
    assert torch.count_nonzero(buf[:, K:]) == 0


@pytest.mark.parametrize("M", [17, 64, 300])
def test_prefill_tiled_against_oracle(oracle, M):
    N, K = 1000, 2048
    inp = oracle.gen_inputs(M, N, K, seed=M)
    x, w, s = dev_inputs(inp, DEV)
    wt = qf.to_tiled(w)
    for chunk in (256, 8192):  # several chunks, then one
        y = qf.w8a16_mm_prefill(x, wt, s, torch.bfloat16, qf.TILED, chunk_rows=chunk)
        torch.cuda.synchronize()
        rep = oracle.check_w8a16(bf16_bits(y), inp.x, inp.w, inp.s)
        print(f"prefill M={M} chunk={chunk}: {rep}", flush=True)
        assert rep.ok, rep
    y32 = qf.w8a16_mm_prefill(x, w, s, torch.float32, qf.ROWMAJOR)
    ex = oracle.w8a16_exact(inp.x, inp.w, inp.s)[1]
    err = np.abs(y32.cpu().numpy().astype(np.float64) - ex).max() / np.sqrt(np.mean(ex ** 2))
    assert err <= 1e-5, err


@pytest.mark.parametrize("M", [40, 260])
def test_prefill_dispatcher_on_tiled_layer(oracle, M):
    """torch.ops.qwen_fastpath.qf_int8_linear with layout=TILED and M > 16: 16-row slices of the
    decode kernel up to 192 rows, the chunked bf16 GEMM above."""
    N, K = 512, 1024
    inp = oracle.gen_inputs(M, N, K, seed=M)
    x, w, s = dev_inputs(inp, DEV)
    y = torch.ops.qwen_fastpath.qf_int8_linear(x.view(2, M // 2, K), qf.to_tiled(w), s, None, qf.TILED)
    torch.cuda.synchronize()
    assert y.shape == (2, M // 2, N)
    assert oracle.check_w8a16(bf16_bits(y.view(M, N)), inp.x, inp.w, inp.s).ok
