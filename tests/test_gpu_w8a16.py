"""GPU parity of the HIP W8A16 kernels against the oracle (tolerance rule in oracle.check_w8a16:
max|err|/RMS <= 1e-2, <= 1 bf16 ulp + fp32 floor from the exact product, <= 2 ulp + floor from the
reference-kernel arithmetic, <= 2% of outputs off the correctly rounded value), plus the invariants
that hold at any size: determinism, row independence, one-hot closed form, layout equivalence and
graph replay."""
import numpy as np
import pytest
import torch

import qwen_fastpath as qf
from qwen_fastpath import _lib as L
from helpers import bf16_bits, dev_inputs, to_dev_bf16

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")

# (N, K) at M = 5 for the dense 27B-class layer, and the other benchmark shapes
LAYER = {"qkv": (10240, 5120), "o_proj": (5120, 8192), "gate_up": (34816, 5120), "down": (5120, 17408)}


def run(x, w_t, s, cfg=None, layout=qf.ROWMAJOR, out=torch.bfloat16):
    y = qf.w8a16_mm(x, w_t, s, cfg, out, layout)
    torch.cuda.synchronize()
    return y


def check(oracle, inp, y_bits, ref=True, label=""):
    ex = oracle.w8a16_exact(inp.x, inp.w, inp.s)
    rb = None
    if ref:
        M, N, K = inp.shape
        c = oracle.ref_pick_config(N, K)
        if c is not None:
            rb = oracle.w8a16_refkernel(inp.x, inp.w, inp.s, c[2], c[3])[0]
    rep = oracle.check_w8a16(y_bits, inp.x, inp.w, inp.s, exact=ex, ref_bits=rb)
    print(f"{label}: {rep}", flush=True)
    assert rep.ok, f"{label}: {rep}"
    return rep


@pytest.mark.parametrize("M", list(range(1, 17)))
def test_small_shapes_every_m(oracle, M):
    for (N, K) in ((16, 64), (48, 320), (200, 1024), (1000, 2048)):
        inp = oracle.gen_inputs(M, N, K, seed=M * 7 + N)
        x, w, s = dev_inputs(inp, DEV)
        check(oracle, inp, bf16_bits(run(x, w, s)), label=f"auto M={M} N={N} K={K}")


WNWK = [(4, 1), (8, 1), (2, 2), (4, 2), (8, 2), (1, 4), (2, 4), (4, 4), (1, 8), (2, 8)]
MFMA_CFGS = [(nt, wn, wk, d, h) for nt in (1, 2) for (wn, wk) in WNWK for d in (4, 8) for h in (0, 1)]


@pytest.mark.parametrize("nt,wn,wk,depth,hint", MFMA_CFGS)
def test_mfma_configs(oracle, nt, wn, wk, depth, hint):
    M, N, K = 5, 1040, 5120
    inp = oracle.gen_inputs(M, N, K, seed=nt * 1000 + wn * 100 + wk * 10 + depth + hint)
    x, w, s = dev_inputs(inp, DEV)
    wt = qf.to_tiled(w)
    outs = {}
    for sk in (1, 3, 8):
        cfg = qf.W8A16Config(L.KERNEL_MFMA, sk, nt, wn * wk, depth, hint, wk)
        for layout, ww in ((qf.ROWMAJOR, w), (qf.TILED, wt)):
            y = bf16_bits(run(x, ww, s, cfg, layout))
            outs[(sk, layout)] = y
        # the two layouts hold the same values in the same per-lane order: identical results
        assert np.array_equal(outs[(sk, qf.ROWMAJOR)], outs[(sk, qf.TILED)])
        check(oracle, inp, outs[(sk, qf.ROWMAJOR)], label=f"mfma nt={nt} wn={wn} wk={wk} d={depth} h={hint} sk={sk}")


XRING_CFGS = [(nt, wn, d, h) for nt in (1, 2) for wn in (4, 8) for d in (4, 8) for h in (0, 1)]


@pytest.mark.parametrize("nt,wn,depth,hint", XRING_CFGS)
def test_mfma_xring_configs(oracle, nt, wn, depth, hint):
    """x staged through the two-slot LDS ring: the oracle's tolerance, and bit for bit the result of the
    whole-slice kernel with the same shape (same products, same order), at M = 1, 5 and 16."""
    for M in (1, 5, 16):
        N, K = 1040, 5120
        inp = oracle.gen_inputs(M, N, K, seed=M * 100 + nt * 10 + wn + depth + hint)
        x, w, s = dev_inputs(inp, DEV)
        wt = qf.to_tiled(w)
        for sk in (1, 3):
            ring = qf.W8A16Config(L.KERNEL_MFMA_XRING, sk, nt, wn, depth, hint, 1)
            staged = qf.W8A16Config(L.KERNEL_MFMA, sk, nt, wn, depth, hint, 1)
            for layout, ww in ((qf.ROWMAJOR, w), (qf.TILED, wt)):
                y = bf16_bits(run(x, ww, s, ring, layout))
                check(oracle, inp, y, label=f"xring M={M} nt={nt} wn={wn} d={depth} h={hint} sk={sk} layout={layout}")
                try:
                    y2 = bf16_bits(run(x, ww, s, staged, layout))
                except L.QFError:  # the whole slice does not fit in LDS
                    continue
                assert np.array_equal(y, y2), (M, sk, layout)


def test_xring_unsplit_where_the_whole_slice_does_not_fit(oracle):
    """M = 16 over K = 17408 unsplit: the whole x slice (557 KiB) exceeds LDS, the ring needs 20 KiB."""
    M, N, K = 16, 512, 17408
    inp = oracle.gen_inputs(M, N, K, seed=99)
    x, w, s = dev_inputs(inp, DEV)
    with pytest.raises(L.QFError):
        run(x, w, s, qf.W8A16Config(L.KERNEL_MFMA, 1, 2, 8, 4, 1, 1), qf.ROWMAJOR)
    y = bf16_bits(run(x, qf.to_tiled(w), s, qf.W8A16Config(L.KERNEL_MFMA_XRING, 1, 2, 8, 4, 1, 1), qf.TILED))
    check(oracle, inp, y, label="xring M=16 K=17408 unsplit")


def test_fused_split_k_counters_return_to_zero(oracle):
    """Every split-K call leaves the arrival counters at the front of the workspace at zero, so the
    persistent workspace serves the next call: repeated calls give identical, correct results."""
    from qwen_fastpath import w8a16 as W
    M, N, K = 5, 5120, 8192
    inp = oracle.gen_inputs(M, N, K, seed=77)
    x, w, s = dev_inputs(inp, DEV)
    ys = []
    for sk, wk in ((2, 4), (4, 4), (7, 2), (16, 1), (3, 8)):
        cfg = qf.W8A16Config(L.KERNEL_MFMA, sk, 1, 16 if wk > 1 else 4, 8, 1, wk)
        for _ in range(3):
            ys.append(bf16_bits(run(x, w, s, cfg)))
            ws = W._workspaces[(0, torch.cuda.current_stream().cuda_stream)]
            assert int(ws[:65536].view(torch.int32).abs().sum()) == 0
        assert np.array_equal(ys[-1], ys[-2]) and np.array_equal(ys[-1], ys[-3])
        check(oracle, inp, ys[-1], label=f"fused split-K sk={sk} wk={wk}")
        # the second-pass kernel sums the same partials in the same order: identical bits
        cfg2 = cfg._replace(reduce=1)
        assert np.array_equal(bf16_bits(run(x, w, s, cfg2)), ys[-1])


@pytest.mark.parametrize("name", ["o_proj", "qkv"])
def test_large_lds_without_split(oracle, name):
    """x slices above 64 KiB of LDS (gfx950 allows 160 KiB per workgroup), no K split."""
    N, K = LAYER[name]
    inp = oracle.gen_inputs(5, N, K, seed=3)
    x, w, s = dev_inputs(inp, DEV)
    wt = qf.to_tiled(w)
    for (wn, wk) in ((2, 8), (1, 8), (4, 4)):
        cfg = qf.W8A16Config(L.KERNEL_MFMA, 1, 1, wn * wk, 8, 1, wk, 0)
        y = bf16_bits(run(x, wt, s, cfg, qf.TILED))
        check(oracle, inp, y, label=f"{name} lds>64K wn={wn} wk={wk}")


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_gemv_configs(oracle, M):
    for (N, K) in ((37, 64), (1000, 5120), (4096, 8192)):
        inp = oracle.gen_inputs(M, N, K, seed=M + N)
        x, w, s = dev_inputs(inp, DEV)
        for rpw in (2, 4):
            for hint in (0, 1):
                for sk in (1, 2, 5):
                    if sk > K // 64 or M * -(-(K // 64) // sk) * 64 * 2 > 160 * 1024 - 256:
                        continue  # more k-steps than splits, or the x slice exceeds the LDS budget
                    cfg = qf.W8A16Config(L.KERNEL_GEMV, sk, rpw, 4, 0, hint, 1)
                    check(oracle, inp, bf16_bits(run(x, w, s, cfg)),
                          label=f"gemv M={M} N={N} K={K} rpw={rpw} h={hint} sk={sk}")


@pytest.mark.parametrize("name", list(LAYER))
def test_layer_shapes_m5_full_size(oracle, name):
    N, K = LAYER[name]
    inp = oracle.gen_inputs(5, N, K, seed=0)
    x, w, s = dev_inputs(inp, DEV)
    check(oracle, inp, bf16_bits(run(x, w, s)), label=f"{name} M=5")
    # the same kernel with an fp32 output against the exact product: the 1e-2 bound at fp32 precision
    rel = oracle.check_w8a16_f32(run(x, w, s, out=torch.float32).cpu().numpy(), inp.x, inp.w, inp.s)
    print(f"{name} M=5 fp32 out: max|err|/RMS = {rel:.2e}", flush=True)
    assert rel <= oracle.REL_MAX_TOL and rel <= 1e-5


# One tensor-parallel rank's shards at TP = 8: qkv and gate_up split N, o_proj and down split K.
TP8 = {"qkv": (1280, 5120), "o_proj": (5120, 1024), "gate_up": (4352, 5120), "down": (5120, 2176)}


@pytest.mark.parametrize("name", list(TP8))
def test_tp8_rank_shapes_tiled(oracle, name):
    """The auto shapes for few workgroups (4-wavefront workgroups, DEPTH 8 on longer k ranges) on TILED weights."""
    N, K = TP8[name]
    inp = oracle.gen_inputs(5, N, K, seed=8)
    x, w, s = dev_inputs(inp, DEV)
    cfg = qf.resolve_config(5, N, K, qf.TILED)
    y = run(x, qf.to_tiled(w), s, layout=qf.TILED)
    check(oracle, inp, bf16_bits(y), label=f"tp8 {name} M=5 tiled cfg={tuple(cfg)}")


def test_single_linear_m1(oracle):
    inp = oracle.gen_inputs(1, 5120, 5120, seed=0)
    x, w, s = dev_inputs(inp, DEV)
    check(oracle, inp, bf16_bits(run(x, w, s)), label="5120x5120 M=1")


@pytest.mark.parametrize("M", [1, 2, 3, 5, 8, 12, 16])
def test_gate_up_m_sweep(oracle, M):
    inp = oracle.gen_inputs(M, 34816, 5120, seed=M)
    x, w, s = dev_inputs(inp, DEV)
    check(oracle, inp, bf16_bits(run(x, w, s)), label=f"gate_up M={M}")
    if M <= 4:
        cfg = qf.W8A16Config(L.KERNEL_GEMV, 1, 4, 4, 0, 0, 1)
        check(oracle, inp, bf16_bits(run(x, w, s, cfg)), label=f"gate_up gemv M={M}")


def test_determinism_and_row_independence(oracle):
    N, K = 5120, 17408
    inp = oracle.gen_inputs(16, N, K, seed=21)
    x, w, s = dev_inputs(inp, DEV)
    cfg = qf.W8A16Config(L.KERNEL_MFMA, 16, 2, 8, 4, 0, 2)
    ys = [bf16_bits(run(x, w, s, cfg)) for _ in range(3)]
    assert all(np.array_equal(ys[0], y) for y in ys[1:])
    for M in (1, 5, 9):
        ym = bf16_bits(run(x[:M].contiguous(), w, s, cfg))
        assert np.array_equal(ym, ys[0][:M])


def test_one_hot_closed_form(oracle):
    N, K = 512, 1024
    inp = oracle.gen_inputs(1, N, K, seed=5)
    ks = [0, 1, 15, 16, 63, 64, 511, 1023]
    xb = np.zeros((len(ks), K), dtype=np.uint16)
    for m, k in enumerate(ks):
        xb[m, k] = 0x3F80
    x = to_dev_bf16(xb, DEV)
    w = torch.from_numpy(inp.w).to(DEV)
    s = torch.from_numpy(inp.s).to(DEV)
    for cfg in (None, qf.W8A16Config(L.KERNEL_MFMA, 4, 1, 8, 4, 1, 2)):
        y = bf16_bits(run(x, w.t(), s, cfg))
        want = oracle.bf16_from_f64(inp.w[:, ks].T.astype(np.float64) * inp.s.astype(np.float64))
        assert np.array_equal(y, want)


def test_extreme_weights_and_zero_rows(oracle):
    M, N, K = 6, 96, 4096
    inp = oracle.gen_inputs(M, N, K, seed=9)
    inp.w[:32] = 127
    inp.w[32:64] = -128
    inp.w[64:, ::2] = -127
    inp.x[2] = 0
    x, w, s = dev_inputs(inp, DEV)
    y = bf16_bits(run(x, w, s))
    check(oracle, inp, y, ref=False, label="extremes")
    assert np.all(oracle.bf16_to_f32(y[2]) == 0)


def test_strided_activations_and_fp32_output(oracle):
    M, N, K = 7, 640, 2048
    inp = oracle.gen_inputs(M, N, K, seed=13)
    x, w, s = dev_inputs(inp, DEV)
    wide = torch.zeros((M, K + 256), dtype=torch.bfloat16, device=DEV)
    wide[:, 128:128 + K] = x
    xs = wide[:, 128:128 + K]            # row stride K + 256, 256-byte offset
    assert xs.stride(0) == K + 256
    y = bf16_bits(run(xs, w, s))
    check(oracle, inp, y, label="strided x")
    y32 = run(xs, w, s, out=torch.float32).cpu().numpy()
    ex = oracle.w8a16_exact(inp.x, inp.w, inp.s)[1]
    assert np.max(np.abs(y32 - ex)) <= 1e-5 * np.max(np.abs(ex))
    assert np.array_equal(oracle.bf16_from_f64(y32.astype(np.float64)), y)


def test_tiled_round_trip(oracle):
    for (N, K) in ((100, 64), (34816, 5120), (5120, 17408)):
        inp = oracle.gen_inputs(1, N, K, seed=1)
        w = torch.from_numpy(inp.w).to(DEV)
        wt = qf.to_tiled(w.t())
        back = qf.from_tiled(wt, N, K)
        torch.cuda.synchronize()
        assert torch.equal(back, w.t())
        # the image is the documented permutation
        if N == 100:
            img = wt.cpu().numpy().reshape(-1, K // 64, 64, 16)
            wp = np.zeros((112, K), dtype=np.int8)
            wp[:N] = inp.w
            for t in range(img.shape[0]):
                for st in range(K // 64):
                    for l in range(64):
                        row, col = t * 16 + l % 16, st * 64 + 16 * (l // 16)
                        assert np.array_equal(img[t, st, l], wp[row, col:col + 16])


def test_graph_capture_replay(oracle):
    shapes = [(5, 10240, 5120), (5, 5120, 8192), (5, 5120, 17408)]
    bufs = []
    for i, (M, N, K) in enumerate(shapes):
        inp = oracle.gen_inputs(M, N, K, seed=40 + i)
        bufs.append((inp, *dev_inputs(inp, DEV)))
    eager = [bf16_bits(run(x, w, s)) for (_, x, w, s) in bufs]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for (_, x, w, s) in bufs:  # warm-up off the default stream
            qf.w8a16_mm(x, w, s, None, torch.bfloat16)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [qf.w8a16_mm(x, w, s, None, torch.bfloat16) for (_, x, w, s) in bufs]
    torch.cuda.synchronize()
    for rep in range(4):
        for o in outs:
            o.fill_(0)
        junk = torch.randn(1 << 20, device=DEV).sum()  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        for i, o in enumerate(outs):
            assert np.array_equal(bf16_bits(o), eager[i]), (rep, i)
        del junk
