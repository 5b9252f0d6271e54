"""GPU parity of the W8A8 path on TILED weights (qf_quantize_tokens_int8 + qf_w8a8_gemm), the arithmetic
of the reference's M > 16 fallback (scaled_int8_quant + cutlass_scaled_mm, plugin/qwen_fastpath/
patches.py:99-100).  Pinned bit for bit against the package's torch restatement of that arithmetic
(patches.w8a8_reference: per-token scale amax / 127, half-even rounding, exact integer sums,
(sum * s_a) * s_w), and against the reference's published W8A8 error statistic."""
import numpy as np
import pytest
import torch

import qwen_fastpath as qf
from qwen_fastpath import _lib as L
from qwen_fastpath import patches as P
from helpers import dev_inputs

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def bits(t):
    return t.view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32)


def random_case(M, N, K, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, device=DEV, generator=g)
    s = (torch.rand(N, device=DEV, generator=g) * 0.004 + 1e-4).float()
    x = (torch.randn(M, K, device=DEV, generator=g) * torch.exp2(torch.randint(-4, 5, (M, 1), device=DEV,
                                                                               generator=g).float()))
    return x.to(torch.bfloat16), w, s


def test_quantize_tokens_closed_form():
    """s_a = amax * fl(1/127); xq = clamp(rint(x / s_a)) with an IEEE division; a zero row gives 0 / 0;
    rows holding the extremes quantise them to +-127 (and -128 never, as |x| <= amax)."""
    M, K = 37, 5120
    x, _, _ = random_case(M, 8, K, 1)
    x[3] = 0
    x[5, 7] = -1e4
    xq, s_a = qf.quantize_tokens_int8(x)
    xf = x.float()
    amax = xf.abs().amax(dim=-1)
    s_ref = amax * torch.tensor(1.0 / 127.0, dtype=torch.float32, device=DEV)
    q_ref = torch.where(s_ref[:, None] > 0, torch.round(xf / torch.where(s_ref > 0, s_ref, 1.0)[:, None]),
                        torch.zeros_like(xf)).clamp(-128, 127).to(torch.int8)
    torch.cuda.synchronize()
    assert torch.equal(s_a, s_ref)
    assert torch.equal(xq, q_ref)
    assert s_a[3].item() == 0.0 and int(xq[3].abs().max()) == 0
    assert int(xq[5, 7]) == -127


@pytest.mark.parametrize("M", [17, 64, 100, 300])
def test_w8a8_matches_restatement(M):
    N, K = 1000, 2048
    x, w, s = random_case(M, N, K, M)
    y = qf.w8a8_mm(x, qf.to_tiled(w.t()), s, torch.bfloat16)
    ref = P.w8a8_reference(x, w.t(), s, None, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(bits(y), bits(ref)), M


W8A8_SHAPES = [(nt, waves, depth) for nt in (2, 4) for waves in (4, 8) for depth in (2, 4)]


@pytest.mark.parametrize("nt,waves,depth", W8A8_SHAPES)
def test_w8a8_configs_and_splits_bitwise(nt, waves, depth):
    """Every instantiated (tiles, wavefronts, depth) at 1..4 token tiles and several groups, K splits
    with uneven ranges, fp32 output; int32 sums make every split order exact."""
    N, K = 1000, 1024
    x, w, s = random_case(160, N, K, 7 + nt + waves + depth)
    wt = qf.to_tiled(w.t())
    for M in (1, 16, 20, 48, 64, 100, 160):
        for split in (1, 3):
            cfg = (L.KERNEL_MFMA_W8A8, split, nt, waves, depth, 1, 1, 1)
            y = qf.w8a8_mm(x[:M], wt, s, torch.bfloat16, cfg)
            ref = P.w8a8_reference(x[:M], w.t(), s, None, torch.bfloat16)
            torch.cuda.synchronize()
            assert torch.equal(bits(y), bits(ref)), (nt, waves, depth, M, split)
    cfg = (L.KERNEL_MFMA_W8A8, 2, nt, waves, depth, 1, 1, 1)
    y = qf.w8a8_mm(x[:48], wt, s, torch.float32, cfg)
    assert torch.equal(bits(y), bits(P.w8a8_reference(x[:48], w.t(), s, None, torch.float32)))


@pytest.mark.parametrize("name,N,K", [("gate_up", 34816, 5120), ("o_proj", 5120, 8192), ("down", 5120, 17408),
                                      ("qkv", 10240, 5120)])
def test_w8a8_layer_shapes(name, N, K):
    x, w, s = random_case(512, N, K, N ^ K)
    wt = qf.to_tiled(w.t())
    for M in (17, 96, 512):
        y = qf.w8a8_mm(x[:M], wt, s, torch.bfloat16)
        ref = P.w8a8_reference(x[:M], w.t(), s, None, torch.bfloat16)
        torch.cuda.synchronize()
        print(f"{name} M={M} cfg={L.w8a8_pick_config(M, N, K).to_tuple()}", flush=True)
        assert torch.equal(bits(y), bits(ref)), (name, M)


def w8a8_group_rows(cfg, M, N):
    """Token rows per group of the W8A8 launch (w8a8_groups in csrc/qf_w8a16.hip, restated)."""
    blocks = -(-((N + 15) // 16) // (cfg.waves * cfg.tiles_per_wave))
    max_rows = 128 if cfg.tiles_per_wave == 2 and blocks * -(-M // 128) >= 128 else 64
    g0 = -(-M // max_rows)
    return (-(-M // g0) + 15) // 16 * 16


@pytest.mark.parametrize("name,M,N,K,rows", [
    ("qkv", 128, 10240, 5120, 64), ("o_proj", 256, 5120, 8192, 64), ("split2", 2304, 3840, 17408, 128),
    # 4-wavefront workgroups with token groups of more than 64 rows (5 to 8 token tiles a fragment)
    ("qkv", 160, 10240, 5120, 80), ("qkv", 192, 10240, 5120, 96), ("n1280", 1600, 1280, 5120, 128)])
def test_w8a8_auto_exceptions(name, M, N, K, rows):
    """The automatic rule's exceptions (4-wavefront unsplit workgroups, also with 80- to 128-row token
    groups; a split in two for a long K whose last round of 128-row workgroups is nearly empty) against
    the restatement, on both layouts."""
    cfg = L.w8a8_pick_config(M, N, K)
    assert cfg.kernel == L.KERNEL_MFMA_W8A8, cfg.to_tuple()
    if name == "split2":
        assert cfg.split_k == 2, cfg.to_tuple()
    else:
        assert cfg.waves == 4 and cfg.split_k == 1, cfg.to_tuple()
    assert w8a8_group_rows(cfg, M, N) == rows, cfg.to_tuple()
    x, w, s = random_case(M, N, K, M + N)
    y = qf.w8a8_mm(x, qf.to_tiled(w.t()), s, torch.bfloat16)
    ref = P.w8a8_reference(x, w.t(), s, None, torch.bfloat16)
    y_r = qf.w8a8_mm(x, w.t(), s, torch.bfloat16, layout=qf.ROWMAJOR)
    torch.cuda.synchronize()
    print(f"{name} M={M} cfg={L.w8a8_pick_config(M, N, K).to_tuple()}", flush=True)
    assert torch.equal(bits(y), bits(ref)) and torch.equal(bits(y_r), bits(ref)), name


def test_w8a8_error_statistic(oracle):
    """Against the exact product, the W8A8 path's rel-L2 is the reference's published W8A8 statistic
    (0.0083-0.0094, data/measurements.json:420-427), as on its own fallback."""
    M, N, K = 17, 5120, 6144
    inp = oracle.gen_inputs(M, N, K, seed=4, dist="reftest")
    x, w, s = dev_inputs(inp, DEV)
    y = qf.w8a8_mm(x, qf.to_tiled(w), s, torch.bfloat16)
    torch.cuda.synchronize()
    ex = oracle.w8a16_f64(inp.x, inp.w, inp.s)
    yf = y.float().cpu().numpy().astype(np.float64)
    rel = np.linalg.norm(yf - ex) / np.linalg.norm(ex)
    assert 0.006 <= rel <= 0.012, rel


@pytest.mark.parametrize("nt,waves,depth", [(2, 8, 4), (2, 8, 2), (2, 4, 4), (2, 4, 2)])
def test_w8a8_128_row_groups_bitwise(nt, waves, depth):
    """5..8 token tiles a weight fragment: N wide enough that the 128-row groups are taken (128 or more
    workgroups), M over one and two groups with ragged tails, with and without a K split."""
    N, K = 34816, 256
    x, w, s = random_case(256, N, K, 31 + waves + depth)
    wt = qf.to_tiled(w.t())
    for M in (65, 80, 100, 128, 200, 256):
        for split in (1, 2):
            cfg = (L.KERNEL_MFMA_W8A8, split, nt, waves, depth, 1, 1, 1)
            y = qf.w8a8_mm(x[:M], wt, s, torch.bfloat16, cfg)
            ref = P.w8a8_reference(x[:M], w.t(), s, None, torch.bfloat16)
            torch.cuda.synchronize()
            assert torch.equal(bits(y), bits(ref)), (nt, waves, depth, M, split)


@pytest.mark.parametrize("M,N,K", [(17, 1000, 2048), (100, 513, 1024), (300, 64, 5120), (1, 16, 64)])
def test_w8a8_against_oracle(oracle, M, N, K):
    """The quantiser and the GEMM bit for bit against the oracle's numpy restatement (oracle.w8a8_linear),
    bf16 and fp32 outputs."""
    from helpers import bf16_bits
    inp = oracle.gen_inputs(M, N, K, seed=M + N)
    x, w, s = dev_inputs(inp, DEV)
    xq, s_a = qf.quantize_tokens_int8(x)
    y = qf.w8a8_mm(x, qf.to_tiled(w), s, torch.bfloat16)
    y32 = qf.w8a8_mm(x, qf.to_tiled(w), s, torch.float32)
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.quantize_tokens(inp.x)
    assert np.array_equal(xq.cpu().numpy(), q_ref) and np.array_equal(s_a.cpu().numpy(), s_ref)
    assert np.array_equal(bf16_bits(y), oracle.w8a8_linear(inp.x, inp.w, inp.s))
    assert np.array_equal(y32.cpu().numpy(), oracle.w8a8_linear(inp.x, inp.w, inp.s, out_f32=True))


@pytest.mark.parametrize("K", [64, 5120, 8192, 8256, 17408, 24576, 24640, 30720])
def test_quantize_tokens_all_row_lengths(oracle, K):
    """The three quantiser variants (row kept in registers up to 4 or 12 pieces a thread, read twice
    beyond) against the oracle, at the row lengths on either side of each switch."""
    M = 9
    inp = oracle.gen_inputs(M, 16, K, seed=K)
    x, _, _ = dev_inputs(inp, DEV)
    xq, s_a = qf.quantize_tokens_int8(x)
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.quantize_tokens(inp.x)
    assert np.array_equal(s_a.cpu().numpy(), s_ref)
    assert np.array_equal(xq.cpu().numpy(), q_ref)


@pytest.mark.parametrize("name,N,K", [("small", 1000, 2048), ("o_proj", 5120, 8192), ("gate_up", 34816, 5120)])
def test_w8a8_rowmajor_weights(oracle, name, N, K):
    """Row-major weights (the checkpoint's [N, K], seen as the [K, N] stride-(1, K) view, and a strided copy
    with rows 64 bytes apart more than K) give the TILED image's results bit for bit: each lane loads
    the same 16 bytes either way."""
    x, w, s = random_case(300, N, K, N + 3)
    wt = qf.to_tiled(w.t())
    wide = torch.zeros((N, K + 64), dtype=torch.int8, device=DEV)
    wide[:, :K] = w
    for M in (17, 64, 300):
        y_t = qf.w8a8_mm(x[:M], wt, s, torch.bfloat16)
        y_r = qf.w8a8_mm(x[:M], w.t(), s, torch.bfloat16, layout=qf.ROWMAJOR)
        y_s = qf.w8a8_mm(x[:M], wide[:, :K].t(), s, torch.bfloat16, layout=qf.ROWMAJOR)
        torch.cuda.synchronize()
        assert torch.equal(bits(y_r), bits(y_t)) and torch.equal(bits(y_s), bits(y_t)), (name, M)
    if name == "small":
        inp = oracle.gen_inputs(40, N, K, seed=3)
        xd, wd, sd = dev_inputs(inp, DEV)
        from helpers import bf16_bits
        assert np.array_equal(bf16_bits(qf.w8a8_mm(xd, wd, sd, torch.bfloat16, layout=qf.ROWMAJOR)),
                              oracle.w8a8_linear(inp.x, inp.w, inp.s))


def test_rowmajor_m17_dispatch_uses_the_int8_kernel(oracle, monkeypatch):
    """Without vLLM, a row-major layer's M > 16 call runs the W8A8 arithmetic on the int8 MFMA: the
    dispatcher op's output equals the oracle's W8A8 restatement bit for bit."""
    P._fallback_impl = None
    monkeypatch.setattr(P, "_vllm_w8a8", lambda: None)
    try:
        inp = oracle.gen_inputs(17, 5120, 6144, seed=4)
        x, w, s = dev_inputs(inp, DEV)
        y = torch.ops.qwen_fastpath.qf_int8_linear(x, w, s, None)
        torch.cuda.synchronize()
        from helpers import bf16_bits
        assert np.array_equal(bf16_bits(y), oracle.w8a8_linear(inp.x, inp.w, inp.s))
    finally:
        P._fallback_impl = None


TILE_CFG = (L.KERNEL_MFMA_W8A8_TILE, 1, 8, 8, 4, 1, 1, 1)


def w8a8_into(x, w, s, layout, ldw, y, out_dtype, cfg, x_tiled=False):
    """qf_w8a8_gemm (x_tiled: qf_quantize_tokens_int8_tiled + qf_w8a8_gemm_xt) into a caller's output
    y [M, ldy] (row stride ldy >= N), through the C ABI."""
    import ctypes
    lib = L.load()
    M, K = x.shape
    N = s.numel()
    xq, s_a = qf.quantize_tokens_int8(x, tiled=x_tiled)
    c = L.Config.from_seq(cfg)
    dt = L.DTYPE_BF16 if out_dtype == torch.bfloat16 else L.DTYPE_F32
    need = int(lib.qf_w8a8_workspace_bytes(M, N, K, layout, ctypes.byref(c)))
    ws = torch.zeros((max(need, 16),), dtype=torch.uint8, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    if x_tiled:
        rc = lib.qf_w8a8_gemm_xt(xq.data_ptr(), s_a.data_ptr(), w.data_ptr(), ldw, layout, s.data_ptr(), y.data_ptr(),
                                 y.stride(0), dt, M, N, K, ctypes.byref(c), ws.data_ptr(), need, stream)
    else:
        rc = lib.qf_w8a8_gemm(xq.data_ptr(), K, s_a.data_ptr(), w.data_ptr(), ldw, layout, s.data_ptr(), y.data_ptr(),
                              y.stride(0), dt, M, N, K, ctypes.byref(c), ws.data_ptr(), need, stream)
    L.check(rc, "qf_w8a8_gemm_xt" if x_tiled else "qf_w8a8_gemm")
    return ws


def tile_tokens(xq):
    """The token-tiled image of a row-major int8 [M, K] (rows padded with zeros to a multiple of 16): block
    (b, s) at (b * K/64 + s) KiB, token 16 b + r at k 64 s + 16 g .. +15 at byte 16 (16 g + r) of it."""
    M, K = xq.shape
    Mp = (M + 15) // 16 * 16
    pad = torch.zeros((Mp, K), dtype=torch.int8, device=xq.device)
    pad[:M] = xq
    return pad.view(Mp // 16, 16, K // 64, 4, 16).permute(0, 2, 3, 1, 4).reshape(-1)


@pytest.mark.parametrize("x_tiled", [False, True])
@pytest.mark.parametrize("M,N,K", [(256, 512, 1024), (300, 1000, 640), (520, 1004, 1024), (17, 4112, 5120),
                                   (64, 2056, 512), (1000, 5120, 8192), (513, 16, 64)])
def test_w8a8_tile_kernel_bitwise(M, N, K, x_tiled):
    """The LDS-tiled kernel (explicit configuration) bit for bit against the restatement: token blocks and
    channel blocks cut by M and N (N not a multiple of 8 or 16), TILED and row-major weights (also rows
    64 bytes apart more than K), bf16 output staged through LDS (rows 16-byte aligned), bf16 rows not so
    aligned (ldy % 8 == 4) and fp32 output stored from the registers, a padded output (ldy > N); row-major
    and token-tiled activations."""
    x, w, s = random_case(M, N, K, M * 7 + N)
    ref = P.w8a8_reference(x, w.t(), s, None, torch.bfloat16)
    ref32 = P.w8a8_reference(x, w.t(), s, None, torch.float32)
    wt = qf.to_tiled(w.t())
    wide = torch.zeros((N, K + 64), dtype=torch.int8, device=DEV)
    wide[:, :K] = w
    for layout, wp, ldw in ((qf.TILED, wt, 0), (qf.ROWMAJOR, w, K), (qf.ROWMAJOR, wide, K + 64)):
        for ldy in (N, N + 8, N + 4):
            y = torch.full((M, ldy), float("nan"), dtype=torch.bfloat16, device=DEV)
            w8a8_into(x, wp, s, layout, ldw, y, torch.bfloat16, TILE_CFG, x_tiled)
            torch.cuda.synchronize()
            assert torch.equal(bits(y[:, :N]), bits(ref)), (M, N, K, layout, ldw, ldy)
            if ldy > N:
                assert torch.isnan(y[:, N:].float()).all(), (M, N, K, layout, ldy)  # nothing past N written
        y32 = torch.empty((M, N), dtype=torch.float32, device=DEV)
        w8a8_into(x, wp, s, layout, ldw, y32, torch.float32, TILE_CFG, x_tiled)
        torch.cuda.synchronize()
        assert torch.equal(bits(y32), bits(ref32)), (M, N, K, layout, ldw, "fp32")


def test_w8a8_tile_kernel_against_oracle(oracle):
    """The LDS-tiled kernel against the oracle's numpy restatement (oracle.w8a8_linear), bf16 and fp32."""
    from helpers import bf16_bits
    M, N, K = 300, 513, 1024
    inp = oracle.gen_inputs(M, N, K, seed=11)
    x, w, s = dev_inputs(inp, DEV)
    y = qf.w8a8_mm(x, qf.to_tiled(w), s, torch.bfloat16, TILE_CFG)
    y32 = qf.w8a8_mm(x, qf.to_tiled(w), s, torch.float32, TILE_CFG)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(y), oracle.w8a8_linear(inp.x, inp.w, inp.s))
    assert np.array_equal(y32.cpu().numpy(), oracle.w8a8_linear(inp.x, inp.w, inp.s, out_f32=True))


@pytest.mark.parametrize("name,M,N,K", [("gate_up", 2048, 34816, 5120), ("down", 2048, 5120, 17408),
                                        ("qkv", 1024, 10240, 5120), ("o_proj", 2048, 5120, 8192),
                                        ("gate_up", 768, 34816, 5120), ("down", 512, 5120, 17408),
                                        ("down", 1024, 5120, 17408), ("down", 1536, 5120, 17408),
                                        ("o_proj", 768, 5120, 8192), ("qkv", 640, 10240, 5120),
                                        ("gate_up", 129, 34816, 5120), ("gate_up", 200, 34816, 5120),
                                        ("gate_up", 320, 34816, 5120), ("gate_up", 384, 34816, 5120),
                                        ("down", 544, 5120, 17408)])
def test_w8a8_tile_kernel_auto_layer_shapes(name, M, N, K):
    """Where the automatic rule picks the LDS-tiled kernel (the layer shapes at prefill widths, and with a
    K split and the fused reduction where the tile grid is under a round), the result equals the
    restatement bit for bit on both layouts."""
    cfg = L.w8a8_pick_config(M, N, K)
    assert cfg.kernel == L.KERNEL_MFMA_W8A8_TILE, cfg.to_tuple()
    tiles = -(-N // 256) * -(-M // 256)
    assert (cfg.split_k > 1) == (tiles <= 128), cfg.to_tuple()
    x, w, s = random_case(M, N, K, M + 3 * N)
    ref = P.w8a8_reference(x, w.t(), s, None, torch.bfloat16)
    y = qf.w8a8_mm(x, qf.to_tiled(w.t()), s, torch.bfloat16)
    y_r = qf.w8a8_mm(x, w.t(), s, torch.bfloat16, layout=qf.ROWMAJOR)
    torch.cuda.synchronize()
    print(f"{name} M={M} cfg={cfg.to_tuple()}", flush=True)
    assert torch.equal(bits(y), bits(ref)) and torch.equal(bits(y_r), bits(ref)), name


@pytest.mark.parametrize("M,N,K", [(4096, 4352, 256), (4096, 4344, 256), (4096, 4700, 128), (4000, 4616, 192)])
def test_w8a8_tile_kernel_tail_split(M, N, K):
    """The tile kernel's second launch past whole rounds of 256 workgroups (M = 4096: 16 token blocks).
    N = 4352 / 4344: 17 channel blocks, 272 workgroups; the last block's channels (ragged or not) run on
    the wide kernel (reduce 0 and 2: too few for 128 x 128 workgroups).  N = 4700 / 4616: 19 blocks, 304
    workgroups; the 604 / 520 channels past the first 16 blocks run on 128 x 128 workgroups of the tile
    kernel (reduce 0, 160 of them; N = 4700 ends in a partial chunk of 8 channels) or on the wide kernel
    (reduce 2).
    Each writes the same output at a column offset.  M = 4000 leaves the last token blocks of both shapes
    partial.  Bit for bit equal to the single launch (reduce 1) and to the restatement, on both layouts,
    row-major and token-tiled activations, bf16 rows staged (ldy % 8 == 0) or not, and fp32 outputs."""
    x, w, s = random_case(M, N, K, N + K)
    wt = qf.to_tiled(w.t())
    cfgs = [(L.KERNEL_MFMA_W8A8_TILE, 1, 8, 8, 4, 1, 1, red) for red in (0, 2)] + [TILE_CFG]
    for out_dtype in (torch.bfloat16, torch.float32):
        ref = P.w8a8_reference(x, w.t(), s, None, out_dtype)
        for layout, wp, ldw in ((qf.TILED, wt, 0), (qf.ROWMAJOR, w, K)):
            for cfg in cfgs:
                for x_tiled in (False, True):
                    for pad in ((8, 4) if out_dtype == torch.bfloat16 else (8,)):
                        y = torch.full((M, N + pad), float("nan"), dtype=out_dtype, device=DEV)
                        w8a8_into(x, wp, s, layout, ldw, y, out_dtype, cfg, x_tiled)
                        torch.cuda.synchronize()
                        case = (M, N, K, out_dtype, layout, cfg, x_tiled, pad)
                        assert torch.equal(bits(y[:, :N]), bits(ref)), case
                        assert torch.isnan(y[:, N:].float()).all(), case


@pytest.mark.parametrize("M,N,K", [(2048, 8192, 128), (2048, 8000, 128)])
def test_w8a8_tile_kernel_whole_rounds(M, N, K):
    """Tile grids that are whole rounds of 256 workgroups (rest 0: 32 channel blocks x 8 token blocks) run in
    one launch: N = 8192, and N = 8000, whose blocks hold 8192 channel slots.  Bit for bit against the
    restatement with reduce 0, 2 and 1 and the automatic configuration, on both layouts, with nothing written
    past N."""
    x, w, s = random_case(M, N, K, N + 5 * K)
    wt = qf.to_tiled(w.t())
    ref = P.w8a8_reference(x, w.t(), s, None, torch.bfloat16)
    cfgs = [(L.KERNEL_MFMA_W8A8_TILE, 1, 8, 8, 4, 1, 1, red) for red in (0, 2, 1)]
    for layout, wp, ldw in ((qf.TILED, wt, 0), (qf.ROWMAJOR, w, K)):
        auto = L.w8a8_pick_config(M, N, K, layout).to_tuple()
        for cfg in cfgs + [auto]:
            print(f"whole rounds M={M} N={N} K={K} layout={layout} cfg={cfg}", flush=True)
            y = torch.full((M, N + 8), float("nan"), dtype=torch.bfloat16, device=DEV)
            w8a8_into(x, wp, s, layout, ldw, y, torch.bfloat16, cfg)
            torch.cuda.synchronize()
            assert torch.equal(bits(y[:, :N]), bits(ref)), (M, N, K, layout, cfg)
            assert torch.isnan(y[:, N:].float()).all(), (M, N, K, layout, cfg)


@pytest.mark.parametrize("M,N,K,split", [(300, 1000, 640, 2), (300, 1000, 640, 3), (1000, 5120, 8192, 3),
                                         (520, 1004, 1024, 4), (256, 512, 128, 2), (17, 4112, 5120, 8),
                                         (513, 16, 192, 3), (2048, 1280, 17408, 5)])
def test_w8a8_tile_kernel_split_k(M, N, K, split):
    """The tile kernel with K split across workgroups and the fused reduction (the last split of a tile to
    arrive adds the others' int32 slots): bit for bit equal to the restatement on both layouts, row-major and
    token-tiled activations, staged and unstaged bf16 rows and fp32; every arrival counter back at zero.
    Uneven split ranges (K / 64 not a multiple of the split) and a single split per step (K = 128, 2 splits)."""
    x, w, s = random_case(M, N, K, M * 3 + N + split)
    ref = P.w8a8_reference(x, w.t(), s, None, torch.bfloat16)
    ref32 = P.w8a8_reference(x, w.t(), s, None, torch.float32)
    wt = qf.to_tiled(w.t())
    cfg = (L.KERNEL_MFMA_W8A8_TILE, split, 8, 8, 4, 1, 1, 1)
    for layout, wp, ldw in ((qf.TILED, wt, 0), (qf.ROWMAJOR, w, K)):
        for x_tiled in (False, True):
            for out_dtype, pad in ((torch.bfloat16, 8), (torch.bfloat16, 4), (torch.float32, 4)):
                y = torch.full((M, N + pad), float("nan"), dtype=out_dtype, device=DEV)
                ws = w8a8_into(x, wp, s, layout, ldw, y, out_dtype, cfg, x_tiled)
                torch.cuda.synchronize()
                case = (M, N, K, split, layout, x_tiled, out_dtype, pad)
                assert torch.equal(bits(y[:, :N]), bits(ref if out_dtype == torch.bfloat16 else ref32)), case
                assert torch.isnan(y[:, N:].float()).all(), case
                assert int(ws[:L.COUNTER_BYTES].view(torch.int32).abs().sum()) == 0, case


@pytest.mark.parametrize("M,N,K", [(300, 1000, 640), (17, 4112, 1024), (129, 520, 192), (384, 2064, 5120),
                                   (1000, 16, 128), (257, 34816, 1024)])
def test_w8a8_tile_kernel_128_token_workgroups(M, N, K):
    """The tile kernel's 256-channel x 128-token workgroups (reduce 3; a stage's 24 fragments, weights first,
    3 to a wavefront, so wavefront 5 copies one weight and two activation fragments): bit for bit equal to
    the restatement on both layouts, row-major and token-tiled activations, staged and unstaged bf16 rows
    and fp32; ragged M and N, one channel tile, one k-step pair."""
    x, w, s = random_case(M, N, K, M * 7 + N + K)
    ref = P.w8a8_reference(x, w.t(), s, None, torch.bfloat16)
    ref32 = P.w8a8_reference(x, w.t(), s, None, torch.float32)
    wt = qf.to_tiled(w.t())
    cfg = (L.KERNEL_MFMA_W8A8_TILE, 1, 8, 8, 4, 1, 1, 3)
    for layout, wp, ldw in ((qf.TILED, wt, 0), (qf.ROWMAJOR, w, K)):
        for x_tiled in (False, True):
            for out_dtype, pad in ((torch.bfloat16, 8), (torch.bfloat16, 4), (torch.float32, 4)):
                y = torch.full((M, N + pad), float("nan"), dtype=out_dtype, device=DEV)
                w8a8_into(x, wp, s, layout, ldw, y, out_dtype, cfg, x_tiled)
                torch.cuda.synchronize()
                case = (M, N, K, layout, x_tiled, out_dtype, pad)
                assert torch.equal(bits(y[:, :N]), bits(ref if out_dtype == torch.bfloat16 else ref32)), case
                assert torch.isnan(y[:, N:].float()).all(), case


@pytest.mark.parametrize("M,K", [(1, 64), (15, 128), (16, 1024), (17, 5120), (300, 8192), (2048, 5120),
                                 (33, 17408)])
def test_quantize_tokens_tiled_image(M, K):
    """qf_quantize_tokens_int8_tiled writes the same scales as the row-major quantiser and, byte for byte,
    the token-tiled image of its xq (rows past M zero), over a buffer that starts filled with garbage."""
    x, _, _ = random_case(M, 8, K, M + K)
    x[M // 2] = 0
    xq, s_a = qf.quantize_tokens_int8(x)
    import ctypes
    lib = L.load()
    nbytes = int(lib.qf_tokens_tiled_bytes(M, K))
    assert nbytes == (M + 15) // 16 * 16 * K
    xt = torch.full((nbytes,), 85, dtype=torch.int8, device=DEV)
    s_t = torch.full((M,), float("nan"), dtype=torch.float32, device=DEV)
    L.check(lib.qf_quantize_tokens_int8_tiled(x.data_ptr(), K, M, K, xt.data_ptr(), s_t.data_ptr(),
                                              torch.cuda.current_stream().cuda_stream), "tiled")
    xt2, s_t2 = qf.quantize_tokens_int8(x, tiled=True)
    torch.cuda.synchronize()
    assert torch.equal(s_t, s_a) and torch.equal(s_t2, s_a)
    assert torch.equal(xt, tile_tokens(xq)) and torch.equal(xt2, xt)
    assert int(lib.qf_tokens_tiled_bytes(M, K + 1)) == 0 and int(lib.qf_tokens_tiled_bytes(0, K)) == 0


@pytest.mark.parametrize("nt,waves,depth", W8A8_SHAPES)
def test_w8a8_xt_wide_kernel_configs(nt, waves, depth):
    """The wide kernel reads the token-tiled image as the row-major activations: every instantiated
    shape, 1..8 token tiles, several groups, K splits, both weight layouts where served, bit for bit."""
    N, K = 1000, 1024
    x, w, s = random_case(300, N, K, 29 + nt + waves + depth)
    wt = qf.to_tiled(w.t())
    for M in (1, 16, 20, 100, 160, 300):
        ref = P.w8a8_reference(x[:M], w.t(), s, None, torch.bfloat16)
        for split in (1, 3):
            cfg = (L.KERNEL_MFMA_W8A8, split, nt, waves, depth, 1, 1, 1)
            y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
            w8a8_into(x[:M], wt, s, qf.TILED, 0, y, torch.bfloat16, cfg, True)
            torch.cuda.synchronize()
            assert torch.equal(bits(y), bits(ref)), (nt, waves, depth, M, split)
    for M in (17, 128, 300):  # row-major weights: the automatic shape
        ref = P.w8a8_reference(x[:M], w.t(), s, None, torch.float32)
        y = torch.empty((M, N), dtype=torch.float32, device=DEV)
        w8a8_into(x[:M], w, s, qf.ROWMAJOR, K, y, torch.float32, (0, 0, 0, 0, 0, 0, 0, 0), True)
        torch.cuda.synchronize()
        assert torch.equal(bits(y), bits(ref)), ("rowmajor", M)


@pytest.mark.parametrize("M,N,K", [(2048, 34816, 5120), (17, 1000, 2048), (768, 34816, 5120), (333, 5120, 17408)])
def test_w8a8_mm_activation_layouts_agree(M, N, K):
    """w8a8_mm with the activations in either layout, and with the automatic choice, gives the same bits."""
    x, w, s = random_case(M, N, K, M ^ N)
    wt = qf.to_tiled(w.t())
    ys = [qf.w8a8_mm(x, wt, s, torch.bfloat16, x_tiled=t) for t in (None, False, True)]
    torch.cuda.synchronize()
    assert all(torch.equal(bits(ys[0]), bits(y)) for y in ys[1:]), (M, N, K)
