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


@pytest.mark.parametrize("M", [40, 260, 1100])
@pytest.mark.parametrize("mode", ["w8a8", "w8a16"])
def test_prefill_dispatcher_on_tiled_layer(oracle, monkeypatch, M, mode):
    """torch.ops.qwen_fastpath.qf_int8_linear with layout=TILED and M > 16.  Default (w8a8): the
    reference's W8A8 arithmetic on the int8 MFMA, bitwise equal to the package's restatement of it.
    QWEN_FAST_LINEAR_PREFILL=w8a16: the wide-M kernel up to 1024 rows, the widened bf16 library GEMM
    above, within the W8A16 tolerance of the exact product."""
    from qwen_fastpath import patches as P
    if mode == "w8a16":
        monkeypatch.setenv("QWEN_FAST_LINEAR_PREFILL", "w8a16")
    else:
        monkeypatch.delenv("QWEN_FAST_LINEAR_PREFILL", raising=False)
    N, K = 512, 1024
    inp = oracle.gen_inputs(M, N, K, seed=M)
    x, w, s = dev_inputs(inp, DEV)
    y = torch.ops.qwen_fastpath.qf_int8_linear(x.view(2, M // 2, K), qf.to_tiled(w), s, None)
    torch.cuda.synchronize()
    assert y.shape == (2, M // 2, N)
    if mode == "w8a16":
        assert oracle.check_w8a16(bf16_bits(y.view(M, N)), inp.x, inp.w, inp.s).ok
    else:
        ref = P.w8a8_reference(x, w, s, None, torch.bfloat16)
        torch.cuda.synchronize()
        assert torch.equal(y.view(M, N).view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("M,N,offset", [(1, 8, 0), (7, 1000, 0), (64, 8192, 0), (33, 1001, 0), (5, 64, 1)])
def test_scale_cast_matches_torch(M, N, offset):
    """qf_scale_cast_bf16 against torch's (acc * s).to(bf16): random values over the whole fp32 range,
    ties and near-ties of bf16 rounding, zeros, denormals, infinities and NaN; the vector path and,
    with a ragged N or a misaligned view, the element path."""
    g = torch.Generator(device=DEV)
    g.manual_seed(M * N)
    acc = torch.randn(M, N + offset, device=DEV, generator=g) * torch.exp2(torch.randint(-60, 60, (M, N + offset), device=DEV, generator=g).float())
    acc = acc[:, offset:]
    flat = acc.reshape(-1) if acc.is_contiguous() else None
    if flat is not None and flat.numel() >= 16:
        bits = torch.tensor([0x3F808000, 0x3F818000, 0x3F808001, 0x00000001, 0x80000000, 0x7F800000, 0xFF800000,
                             0x7F7FFFFF, 0x7FC00000, 0x3F80FFFF, 0x007FFFFF, 0x3F7F8000], dtype=torch.int64)
        flat[:12] = bits.to(torch.int32).view(torch.float32).to(DEV)
    s = (torch.rand(N, device=DEV, generator=g) * 2 + 0.25).float()
    s[: min(N, 3)] = 1.0
    out = torch.full((M, N), 7.0, dtype=torch.bfloat16, device=DEV)
    qf.scale_cast_bf16(acc, s, out)
    ref = (acc * s).to(torch.bfloat16)
    torch.cuda.synchronize()
    nan = torch.isnan(ref)
    assert torch.equal(torch.isnan(out), nan)
    assert torch.equal(out.view(torch.int16)[~nan], ref.view(torch.int16)[~nan])


def test_prefill_chunks_bitwise_equal_to_torch_epilogue():
    """The fused epilogue leaves the chunked path's output unchanged: widening + torch.mm + the
    scale/cast pass against the same GEMM followed by torch's elementwise scale and cast."""
    M, N, K = 100, 3000, 1024
    g = torch.Generator(device=DEV)
    g.manual_seed(9)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, device=DEV, generator=g)
    s = (torch.rand(N, device=DEV, generator=g) * 0.004 + 1e-4).float()
    x = torch.randn(M, K, device=DEV, generator=g).to(torch.bfloat16)
    wt = qf.to_tiled(w.t())
    y = qf.w8a16_mm_prefill(x, wt, s, torch.bfloat16, qf.TILED, chunk_rows=1024)
    ref = torch.cat([(torch.mm(x, w[n0:n0 + 1024].to(torch.bfloat16).t(), out_dtype=torch.float32)
                      * s[n0:n0 + 1024]).to(torch.bfloat16) for n0 in range(0, N, 1024)], dim=1)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
