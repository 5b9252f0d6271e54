"""Soak tests of the fused last-arrival K-split reductions, which order their partial sums by device-scope stores
completed before an arrival counter rather than by a kernel boundary: over many back-to-back calls with varying
inputs, the fused result must equal the second-pass (or unsplit) result bit for bit, every call.  Each test is
bounded (a fixed number of calls, a few seconds) and stops at the first mismatching call, naming it."""
import pytest
import torch

import qwen_fastpath as qf
from qwen_fastpath import _lib as L

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
CHUNK = 50


def _bits(t):
    return t.view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32)


@pytest.mark.parametrize("M,N,K,split", [(5, 5120, 17408, 3), (16, 5120, 17408, 4), (5, 1024, 8192, 8)])
def test_soak_decode_fused_split_k(M, N, K, split):
    """The decode kernel's fused split-K (reduce 0: the last workgroup of each n-block sums the splits) against the
    second-pass kernel (reduce 1), 4000 calls each on TILED weights, a different x every call (down's shape at M = 5
    is the automatic configuration of the layer's down GEMM)."""
    g = torch.Generator(device=DEV)
    g.manual_seed(M + N + K + split)
    img = torch.randint(-127, 128, (qf.tiled_numel(N, K),), dtype=torch.int8, device=DEV, generator=g)
    s = (torch.randn(N, device=DEV, generator=g).abs() * 0.002 + 1e-4).float()
    xs = torch.randn(CHUNK, M, K, device=DEV, generator=g).to(torch.bfloat16)
    fused = qf.W8A16Config(L.KERNEL_MFMA, split, 1, 8, 4, 1, 2, 0)
    second = fused._replace(reduce=1)
    print(f"soak decode M={M} N={N} K={K} split={split}", flush=True)
    for chunk in range(4000 // CHUNK):
        xs.mul_(-1.0) if chunk % 2 else None  # vary the inputs between chunks
        a = [qf.w8a16_mm(xs[i], img, s, fused, torch.bfloat16, qf.TILED) for i in range(CHUNK)]
        b = [qf.w8a16_mm(xs[i], img, s, second, torch.bfloat16, qf.TILED) for i in range(CHUNK)]
        torch.cuda.synchronize()
        for i in range(CHUNK):
            assert torch.equal(_bits(a[i]), _bits(b[i])), f"call {chunk * CHUNK + i}: fused split-K differs"


@pytest.mark.parametrize("M,N,K,split", [(512, 5120, 17408, 4), (1024, 5120, 8192, 3)])
def test_soak_w8a8_tile_fused_split_k(M, N, K, split):
    """The W8A8 tile kernel's fused K split (the last of a tile's split copies adds the others' int32 partials)
    against the unsplit tile kernel, 1000 calls each with a different activation every call: exact integer sums,
    so the bits must agree."""
    g = torch.Generator(device=DEV)
    g.manual_seed(M + N + K)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, device=DEV, generator=g)
    img = qf.to_tiled(w.t())
    del w
    s = (torch.rand(N, device=DEV, generator=g) * 0.004 + 1e-4).float()
    xs = torch.randn(4, M, K, device=DEV, generator=g).to(torch.bfloat16)
    split_cfg = (L.KERNEL_MFMA_W8A8_TILE, split, 8, 8, 4, 1, 1, 0)
    one = (L.KERNEL_MFMA_W8A8_TILE, 1, 8, 8, 4, 1, 1, 1)
    print(f"soak w8a8 tile M={M} N={N} K={K} split={split}", flush=True)
    for chunk in range(1000 // 20):
        a = [qf.w8a8_mm(xs[i % 4] * (1 + chunk), img, s, torch.bfloat16, split_cfg) for i in range(20)]
        b = [qf.w8a8_mm(xs[i % 4] * (1 + chunk), img, s, torch.bfloat16, one) for i in range(20)]
        torch.cuda.synchronize()
        for i in range(20):
            assert torch.equal(_bits(a[i]), _bits(b[i])), f"call {chunk * 20 + i}: fused K split differs"
