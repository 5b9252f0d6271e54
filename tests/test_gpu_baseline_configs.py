"""GPU parity at the benchmark's own sizes, on the configuration the library picks for each layout:

* the four GEMMs of the dense 27B-class layer at M = 5 (qkv 10240x5120, o_proj 5120x8192, gate_up 34816x5120,
  down 5120x17408; down's automatic shape on TILED weights is the fused last-arrival K split) and the
  single 5120x5120 linear at M = 1, on both weight layouts, seed 0;
* the gate_up M sweep (M = 1, 2, 3, 5, 8, 12, 16) on TILED weights;
* the 64-layer decode-step stack at M = 5 (distinct seeded weights per layer, o_proj reading the first
  8192 qkv outputs, down the first 17408 gate_up outputs, each layer's output re-normalised to unit RMS
  as the next input inside the next qkv GEMM's staging, qf_w8a16_gemm_rmsnorm, the same bits as
  qf_rms_norm_rows_bf16 and then the GEMM) captured as one graph: replays equal the eager step bit for bit, and for sampled
  layers every GEMM is checked against the oracle on the input it actually received.

Each check applies oracle.check_w8a16 (every output within 1 bf16 ulp plus the fp32 floor of the exact
product, max(|err| - ulp) / RMS <= 1e-2) and compares the kernel with the reference kernel's own arithmetic
on the same inputs (oracle.w8a16_refkernel, the Triton tile order and split of plugin/qwen_fastpath/w8a16.py):
the outputs that are not the correctly rounded product may be at most 2x + 8 as many as the reference's.
The stated bound read against the correctly rounded product, rel_max = max|y - bf16(exact)| / RMS(exact)
<= 1e-2, is recorded for both but not asserted: one rounding flip of an output above 1.3 x RMS exceeds it,
and the reference arithmetic itself gives 1.15e-2 on gate_up at M = 5, seed 0.  With
QF_PARITY_TABLE=<path> set, every checked configuration appends a row to that markdown file."""
import os

import pytest
import torch

import qwen_fastpath as qf
from helpers import bf16_bits, dev_inputs

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
LAYER = {"qkv": (10240, 5120), "o_proj": (5120, 8192), "gate_up": (34816, 5120), "down": (5120, 17408)}
LAYOUTS = {"tiled": qf.TILED, "rowmajor": qf.ROWMAJOR}

_table_path = os.environ.get("QF_PARITY_TABLE")


def _record(label, cfg, rep, ref):
    if not _table_path:
        return
    new = not os.path.exists(_table_path)
    with open(_table_path, "a") as f:
        if new:
            f.write("| configuration | kernel config | rel_max | reference arithmetic rel_max | rel_excess | rel_l2 | "
                    "outputs != RNE(exact) (reference arithmetic) | max ulp |\n|---|---|---|---|---|---|---|---|\n")
        f.write(f"| {label} | {list(cfg) if cfg is not None else '-'} | {rep.rel_max:.2e} | {ref.rel_max:.2e} | "
                f"{rep.rel_excess:.2e} | {rep.rel_l2:.3e} | {rep.n_diff_exact} ({ref.n_diff_exact}) | "
                f"{rep.max_ulp_exact:.2f} |\n")


def _check(oracle, x_bits, w, s, y_bits, label, cfg):
    exact = oracle.w8a16_exact(x_bits, w, s)
    N, K = w.shape
    c = oracle.ref_pick_config(N, K)
    rb = oracle.w8a16_refkernel(x_bits, w, s, c[2], c[3])[0]
    ref = oracle.check_w8a16(rb, x_bits, w, s, exact=exact)
    rep = oracle.check_w8a16(y_bits, x_bits, w, s, exact=exact, ref_bits=rb)
    print(f"{label} cfg={cfg}: {rep} | reference arithmetic: rel_max={ref.rel_max:.2e} diff={ref.n_diff_exact}",
          flush=True)
    _record(label, cfg, rep, ref)
    assert rep.ok, f"{label}: {rep}"
    assert rep.n_diff_exact <= 2 * ref.n_diff_exact + 8, (
        f"{label}: {rep.n_diff_exact} outputs off the correctly rounded product, reference arithmetic "
        f"{ref.n_diff_exact}")
    return rep


def _run(inp, layout):
    x, w, s = dev_inputs(inp, DEV)
    M, N, K = inp.shape
    wl = qf.to_tiled(w) if layout == qf.TILED else w
    cfg = qf.resolve_config(M, N, K, layout)
    y = qf.w8a16_mm(x, wl, s, None, torch.bfloat16, layout)
    torch.cuda.synchronize()
    return bf16_bits(y), cfg


@pytest.mark.parametrize("lname", list(LAYOUTS))
@pytest.mark.parametrize("name", list(LAYER))
def test_layer_gemm_m5_full_size(oracle, name, lname):
    N, K = LAYER[name]
    inp = oracle.gen_inputs(5, N, K, seed=0)
    y, cfg = _run(inp, LAYOUTS[lname])
    _check(oracle, inp.x, inp.w, inp.s, y, f"{name} M=5 {lname}", cfg)


@pytest.mark.parametrize("lname", list(LAYOUTS))
def test_single_linear_m1_full_size(oracle, lname):
    inp = oracle.gen_inputs(1, 5120, 5120, seed=0)
    y, cfg = _run(inp, LAYOUTS[lname])
    _check(oracle, inp.x, inp.w, inp.s, y, f"5120x5120 M=1 {lname}", cfg)


@pytest.mark.parametrize("M", [1, 2, 3, 5, 8, 12, 16])
def test_gate_up_m_sweep_tiled(oracle, M):
    inp = oracle.gen_inputs(M, 34816, 5120, seed=M)
    y, cfg = _run(inp, qf.TILED)
    _check(oracle, inp.x, inp.w, inp.s, y, f"gate_up M={M} tiled", cfg)


# ------------------------------------------------------------------------------------------------
# 64-layer decode step
# ------------------------------------------------------------------------------------------------

NL = 64
M5 = 5
SAMPLED = (0, 37, 63)


class _StackLayer:
    """One layer's four TILED weights (random int8 in [-127, 127] written straight into the image, which
    is a permutation of the row-major weight) and per-channel scales |N(0,1)|*0.002 + 1e-4."""

    def __init__(self, i):
        g = torch.Generator(device=DEV)
        g.manual_seed(10_000 + i)
        self.w, self.s = {}, {}
        for name, (N, K) in LAYER.items():
            self.w[name] = torch.randint(-127, 128, (qf.tiled_numel(N, K),), dtype=torch.int8, device=DEV, generator=g)
            self.s[name] = torch.randn(N, device=DEV, generator=g).abs_().mul_(0.002).add_(1e-4)


def _step(layers, x0, record=None, fused=True):
    """One decode step.  fused: layers 1..63 take the previous layer's output through the normalising qkv GEMM
    (qf_w8a16_gemm_rmsnorm); otherwise through qf_rms_norm_rows_bf16 and then the GEMM (the same bits)."""
    h = x0
    d = None
    for i, L_ in enumerate(layers):
        mm = lambda a, n: qf.w8a16_mm(a, L_.w[n], L_.s[n], None, torch.bfloat16, qf.TILED)  # noqa: E731
        if d is not None:
            h = qf.rms_norm_rows(d) if (not fused or record is not None) else None
        ins = {"qkv": h}
        if d is not None and fused:
            qkv = qf.w8a16_mm_rmsnorm(d, L_.w["qkv"], L_.s["qkv"], None, torch.bfloat16, qf.TILED)
        else:
            qkv = mm(h, "qkv")
        ins["o_proj"] = qkv[:, :8192]
        o = mm(ins["o_proj"], "o_proj")
        ins["gate_up"] = o
        gu = mm(o, "gate_up")
        ins["down"] = gu[:, :17408]
        d = mm(ins["down"], "down")
        if record is not None and i in record:
            record[i] = ({n: t.clone() for n, t in ins.items()}, {"qkv": qkv, "o_proj": o, "gate_up": gu, "down": d})
    return qf.rms_norm_rows(d)  # unit RMS, torch's default eps for bf16 (2^-23)


def test_stack64_graph_replay_and_sampled_layers(oracle):
    torch.manual_seed(0)
    layers = [_StackLayer(i) for i in range(NL)]
    x0 = torch.randn(M5, 5120, device=DEV).to(torch.bfloat16)
    record = {i: None for i in SAMPLED}
    eager = _step(layers, x0, record).clone()
    torch.cuda.synchronize()
    assert torch.isfinite(eager.float()).all()
    again = _step(layers, x0)
    assert torch.equal(eager, again), "eager step is not bitwise reproducible"
    unfused = _step(layers, x0, fused=False)
    assert torch.equal(eager, unfused), "the normalising qkv GEMM differs from the norm launch + GEMM"

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _step(layers, x0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = _step(layers, x0)
    for r in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"graph replay {r} differs from the eager step"
        torch.randn(1 << 20, device=DEV).sum().item()  # eager work between replays
    print(f"stack64: {NL} layers, 3 replays equal to the eager step", flush=True)

    for i in SAMPLED:
        ins, outs = record[i]
        for name, (N, K) in LAYER.items():
            x_bits = bf16_bits(ins[name].contiguous())
            w_rm = qf.from_tiled(layers[i].w[name], N, K).t().contiguous().cpu().numpy()  # [N, K]
            s = layers[i].s[name].cpu().numpy()
            _check(oracle, x_bits, w_rm, s, bf16_bits(outs[name]), f"stack64 layer {i} {name} M=5 tiled",
                   qf.resolve_config(M5, N, K, qf.TILED))


@pytest.mark.parametrize("M,N", [(5, 5120), (1, 8), (7, 8192), (16, 4096), (3, 17408 // 8 * 8 // 4), (5, 17408),
                                 (2, 34816), (64, 5120), (200, 1024)])
def test_rms_norm_rows(M, N):
    """The stack's glue (qf_rms_norm_rows_bf16) against torch's fp32 restatement and torch's rms_norm (eps 2^-23,
    torch's default for bf16 inputs), also with eps 2^-7: at most one bf16 ulp apart; reproducible; in place equal
    to out of place."""
    g = torch.Generator(device=DEV)
    g.manual_seed(M * 131 + N)
    scale = torch.exp2(torch.randint(-6, 7, (M, 1), device=DEV, generator=g).float())
    x = (torch.randn(M, N, device=DEV, generator=g) * scale).to(torch.bfloat16)
    y = qf.rms_norm_rows(x)
    xf = x.float()
    ref = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 2.0 ** -23)).to(torch.bfloat16)
    tref = torch.nn.functional.rms_norm(x, (N,))
    y7 = qf.rms_norm_rows(x, eps=2.0 ** -7)
    ref7 = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 2.0 ** -7)).to(torch.bfloat16)
    again = qf.rms_norm_rows(x)
    inplace = x.clone()
    qf.rms_norm_rows(inplace, out=inplace)
    torch.cuda.synchronize()
    yi = y.view(torch.int16).int()
    assert (yi - ref.view(torch.int16).int()).abs().max().item() <= 1
    assert (yi - tref.view(torch.int16).int()).abs().max().item() <= 1
    assert (y7.view(torch.int16).int() - ref7.view(torch.int16).int()).abs().max().item() <= 1
    assert torch.equal(y, again) and torch.equal(y, inplace)


@pytest.mark.parametrize("M,N,K,cfg", [
    (5, 10240, 5120, None),                       # qkv's automatic shape: MFMA kernel, 4 tile groups x 2 k-slices
    (5, 34816, 5120, None),                       # gate_up's: the stream kernel, x staged in LDS
    (3, 5120, 8192, None),                        # o_proj's: 2 x 4
    (1, 5120, 5120, None),                        # the single linear at M = 1: 1 x 4, 4 wavefronts
    (16, 4096, 2048, (2, 1, 1, 8, 4, 1, 1, 0)),   # 8 x 1
    (7, 1000, 4096, (2, 1, 1, 8, 4, 1, 4, 0)),    # 2 x 4, ragged N
    (5, 2000, 17408, None),                       # a K split: the two calls instead
    (16, 100, 64, (2, 1, 1, 8, 4, 1, 1, 0)),      # 8 x 1, one k-step: a thread's scaled pieces span several rows
    (9, 300, 256, (2, 1, 1, 4, 4, 1, 4, 0)),      # 1 x 4: 9 rows' sums on 4 wavefronts
    (8, 34816, 5120, None),                       # the stream kernel at its widest x-in-LDS row count
])
def test_gemm_rmsnorm_bitwise(M, N, K, cfg):
    """qf_w8a16_gemm_rmsnorm (the staged rows normalised inside the GEMM) equals qf_rms_norm_rows_bf16 followed by
    the GEMM bit for bit, bf16 and fp32 outputs, rows at scales 2^-6 .. 2^6 and a zero row, eps 2^-23 and 2^-7;
    a configuration that splits K is refused by the library (QF_ERR_UNSUPPORTED) and the package makes the two
    calls."""
    import ctypes
    from qwen_fastpath import _lib as L
    g = torch.Generator(device=DEV)
    g.manual_seed(M * 7 + N + K)
    scale = torch.exp2(torch.randint(-6, 7, (M, 1), device=DEV, generator=g).float())
    x = (torch.randn(M, K, device=DEV, generator=g) * scale).to(torch.bfloat16)
    if M > 2:
        x[1].zero_()
    img = torch.randint(-127, 128, (qf.tiled_numel(N, K),), dtype=torch.int8, device=DEV, generator=g)
    s = (torch.randn(N, device=DEV, generator=g).abs() * 0.002 + 1e-4).float()
    c = None if cfg is None else qf.W8A16Config(*cfg)
    print(f"gemm_rmsnorm M={M} N={N} K={K} cfg={cfg}", flush=True)
    for eps in (2.0 ** -23, 2.0 ** -7):
        for dt in (torch.bfloat16, torch.float32):
            want = qf.w8a16_mm(qf.rms_norm_rows(x, eps), img, s, c, dt, qf.TILED)
            got = qf.w8a16_mm_rmsnorm(x, img, s, c, dt, qf.TILED, eps)
            torch.cuda.synchronize()
            bits = torch.int16 if dt == torch.bfloat16 else torch.int32
            assert torch.equal(got.view(bits), want.view(bits)), (M, N, K, cfg, eps, dt)
    lib = L.load()
    rc_cfg = L.Config.from_seq(tuple(c) if c is not None else (0,) * 8)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    need = int(lib.qf_w8a16_workspace_bytes(M, N, K, qf.TILED, ctypes.byref(rc_cfg)))
    ws = torch.zeros(max(need, 16), dtype=torch.uint8, device=DEV)
    rc = lib.qf_w8a16_gemm_rmsnorm(x.data_ptr(), K, 2.0 ** -23, img.data_ptr(), K, qf.TILED, s.data_ptr(), y.data_ptr(),
                                   N, L.DTYPE_BF16, M, N, K, ctypes.byref(rc_cfg), ws.data_ptr(), ws.numel(),
                                   torch.cuda.current_stream().cuda_stream)
    split = qf.resolve_config(M, N, K, qf.TILED).split_k > 1 if cfg is None else cfg[1] > 1
    assert rc == (L.ERR_UNSUPPORTED if split else L.OK), rc
