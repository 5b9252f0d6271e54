"""Benchmark of the W8A16 decode GEMM on one MI355X.

Default workload (one "step"): the four per-layer GEMMs of a dense GQA 27B-class transformer at M = 5
tokens (1 verified + 4 draft): qkv K=5120 N=10240, o_proj K=8192 N=5120, gate_up K=5120 N=34816,
down K=17408 N=5120; int8 [N, K] weights with fp32 per-channel scales |N(0,1)|*0.002+1e-4, bf16
N(0,1) activations, synthetic and seeded.  Each step runs one layer's GEMMs; the weights rotate over
several distinct layers (more bytes than the 256 MB MALL), so every step streams
its weights from HBM.  Steps are captured 32 to a graph, as a decode forward pass is.  Output: one JSON
line on stdout.

  value        algorithmic bytes of all timed steps / wall time of the timed steps (GB/s)
  roofline     the dominant kernel (gate_up): algorithmic bytes per launch / its mean duration from
               HIP events on the launch stream; peak 8 TB/s; traffic from the committed rocprofv3
               FETCH_SIZE / WRITE_SIZE summary when one exists for this workload
  cpu_baseline the oracle's fp32-dequant restatement of the reference CPU path
               (F.linear(x.float(), W.float() * s[:, None])) on a bounded sample, host cores

Other modes, one JSON line each: --workload stack64 (64 distinct layers, one hipGraph per decode
step, the layer output re-normalised to unit RMS as the next layer's input); --workload msweep (gate_up at M = 1..16);
--workload lm_head (int8 draft head 151936x5120 + pad-masked argmax at M = 1, 4);
--workload prefill (gate_up at M = 64 .. 2048 through the three M > 16 routes, the W8A8 GEMM alone at
M = 2048 beside the vendor int8 GEMM, and the layer's four GEMMs through the W8A8 route at M = 512, 1024, 2048);
--workload spec_attn (split-KV verification attention of one full-attention layer, H=24, H_kv=4,
D=256, 800-position pages, at the reference's contexts and batch shapes);
--profile-gemm NAME --iters N (only that GEMM, for rocprofv3); --profile-w8a8 M [--w8a8-gemm NAME] --iters N
(only the W8A8 GEMM on gate_up or NAME at M rows, activations quantised beforehand); --copy-probe (a plain device copy
of known size, for counter calibration).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "qwen-a100-fastpath_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "W8A16 GEMM HBM GB/s (% of 8 TB/s) + µs/layer at M=5, 27B shapes"
PEAK_GBS = 8000.0
M_TOKENS = 5
GEMMS = {  # name: (N, K)
    "qkv": (10240, 5120),
    "o_proj": (5120, 8192),
    "gate_up": (34816, 5120),
    "down": (5120, 17408),
}
DOMINANT = "gate_up"
GRAPH_STEPS = 32  # decode steps captured per graph (a multiple of the rotated layer count)
PROFILE_SUMMARY = os.path.join(ROOT, "profiles", "w8a16_layer_m5_pmc.md")
W8A8_PROFILE = os.path.join(ROOT, "profiles", "w8a8_gate_up_m2048_pmc.txt")


def algo_bytes(M: int, N: int, K: int) -> int:
    """Compulsory bytes: int8 weights + fp32 scales + bf16 activations + bf16 outputs."""
    return N * K + 4 * N + 2 * M * K + 2 * M * N


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Layer:
    """One layer's four weight sets plus fixed activations.  With layout TILED the weights are
    converted once at set-up (the load-time repack) and only the tiled image is kept."""

    def __init__(self, torch, qf, dev, seed: int, M: int, layout: int):
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.layout = layout
        self.w, self.s, self.x = {}, {}, {}
        for name, (N, K) in GEMMS.items():
            w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
            w_t = w.t()  # [K, N] view with stride (1, K), as vLLM holds it
            self.w[name] = qf.to_tiled(w_t) if layout == qf.TILED else w_t
            del w, w_t
            self.s[name] = (torch.randn(N, device=dev, generator=g).abs() * 0.002 + 1e-4).float()
            self.x[name] = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)

    def gemm(self, qf, torch, name, cfg=None):
        return qf.w8a16_mm(self.x[name], self.w[name], self.s[name], cfg, torch.bfloat16, self.layout)


def release_cache(torch):
    """Return the caching allocator's free blocks to the driver.  Measured on MI355X: with large freed blocks
    held in torch's cache (set-up temporaries, earlier weight sets), the streaming GEMMs run 4-5% slower
    (gate_up M = 5: 31.5 against 29.8 us, whether the blocks were freed before or after the weights were
    allocated; the same bytes kept allocated cost nothing), so every timed section starts with none."""
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def capture(torch, fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    return g, out


def read_traffic(path=PROFILE_SUMMARY):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 summary, if any."""
    try:
        text = open(path).read()
    except OSError:
        return None
    f = re.search(r"^fetch_bytes_per_launch:\s*([0-9.eE+]+)", text, re.M)
    w = re.search(r"^write_bytes_per_launch:\s*([0-9.eE+]+)", text, re.M)
    if not (f and w):
        return None
    return float(f.group(1)) + float(w.group(1))


def host_threads() -> int:
    """Threads for the CPU baseline: the box's OMP_NUM_THREADS when set (its CPU share), else every core
    this process may run on."""
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, int(env)) if env.isdigit() else cores


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_baseline(M: int, seed: int = 0):
    """The oracle's fp32-dequant restatement of the reference CPU path (bench/test_w8a16.py:15,
    F.linear(x.float(), W.float() * s[:, None])) per GEMM: the single 5120x5120 linear at M = 1 and each of
    the layer's four GEMMs at M, one warm-up then the best of five.  value = the layer's four GEMMs'
    algorithmic bytes / the sum of their best times."""
    from oracle import oracle as O
    cores = host_threads()
    try:
        from threadpoolctl import threadpool_limits
        limiter = threadpool_limits(limits=cores)
    except Exception:  # noqa: BLE001 - threadpoolctl optional
        limiter = None
    shapes = [("single_linear_m1", 1, 5120, 5120)] + [(n, M, N, K) for n, (N, K) in GEMMS.items()]
    per = {}
    for i, (name, m, N, K) in enumerate(shapes):
        inp = O.gen_inputs(m, N, K, seed=seed + i)
        O.fp32_dequant_linear(inp.x, inp.w, inp.s)
        best = float("inf")
        for _ in range(5):
            t0 = time.perf_counter()
            O.fp32_dequant_linear(inp.x, inp.w, inp.s)
            best = min(best, time.perf_counter() - t0)
        per[name] = {"M": m, "N": N, "K": K, "ms": round(best * 1e3, 2),
                     "GB_s": round(algo_bytes(m, N, K) / best / 1e9, 3)}
    if limiter is not None and hasattr(limiter, "unregister"):
        limiter.unregister()
    layer_s = sum(per[n]["ms"] for n in GEMMS) / 1e3
    total_bytes = sum(algo_bytes(M, N, K) for (N, K) in GEMMS.values())
    model = cpu_model()
    return {
        "value": round(total_bytes / layer_s / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"per GEMM, 1 warm-up + best of 5, numpy fp32 BLAS over {cores} threads: the layer's 4 GEMMs at M={M} "
                   f"({total_bytes / 1e6:.1f} MB) take {layer_s * 1e3:.1f} ms; 5120x5120 at M=1 "
                   f"{per['single_linear_m1']['ms']} ms" + (f"; {model}" if model else "")),
        "per_gemm": per,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", choices=["layer", "stack64", "msweep", "lm_head", "prefill", "spec_attn", "tp8"],
                    default="layer")
    ap.add_argument("--layers", type=int, default=20,
                    help="distinct layers allocated at start and rotated through (layer workload; 20 x 363 MB)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--profile-gemm", choices=list(GEMMS) + ["single"], default=None,
                    help="only that GEMM at M=5 (single: the 5120x5120 linear at M=1), --iters launches, weights "
                         "rotating past the MALL (for rocprofv3)")
    ap.add_argument("--profile-w8a8", type=int, default=None, metavar="M",
                    help="only the W8A8 GEMM on --w8a8-gemm at M rows, --iters launches (for rocprofv3)")
    ap.add_argument("--w8a8-gemm", choices=list(GEMMS), default="gate_up",
                    help="the layer GEMM of --profile-w8a8 (default gate_up)")
    ap.add_argument("--iters", type=int, default=200)
    ap.add_argument("--copy-probe", action="store_true")
    ap.add_argument("--read-probe", action="store_true", help="only the library's read probe over the dominant GEMM's bytes")
    ap.add_argument("--layout", choices=["tiled", "rowmajor"], default="tiled",
                    help="weight layout: tiled = pre-permuted at load (default), rowmajor = checkpoint layout")
    ap.add_argument("--cfg", default=None, help="explicit config kernel,split_k,tiles,waves,depth,hint (profile mode)")
    ap.add_argument("--attn-case", default=None,
                    help="spec_attn profile mode: CTX,Q,B -- only that case, --iters calls, no JSON line")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        log("bench.py: this build measures one GPU only (the W8A16 op runs on a single GPU); "
            "run with --gpus 1")
        sys.exit(2)

    import torch
    import qwen_fastpath as qf

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    layout = qf.TILED if args.layout == "tiled" else qf.ROWMAJOR

    if args.copy_probe:
        n = 1 << 30
        a = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        b = torch.empty_like(a)
        for _ in range(args.iters):
            b.copy_(a)
        torch.cuda.synchronize()
        log(f"copy probe: {args.iters} copies of {n} bytes")
        return

    if args.read_probe:
        ceiling = read_ceiling(torch, qf, dev, algo_bytes(M_TOKENS, *GEMMS[DOMINANT]))
        log(f"read probe: {ceiling:.0f} GB/s")
        return

    if args.profile_w8a8:
        M = args.profile_w8a8
        g = torch.Generator(device=dev)
        g.manual_seed(13)
        name = args.w8a8_gemm
        sets = prefill_weight_sets(torch, qf, dev, g, name=name)
        gemm, cfg = w8a8_gate_up_gemm(torch, qf, dev, g, M, sets, name)
        for i in range(args.iters):
            gemm(i % 2)
        torch.cuda.synchronize()
        log(f"profile: {args.iters} launches of the W8A8 GEMM on {name} M={M} cfg={cfg.to_tuple()}")
        return

    if args.profile_gemm == "single":
        N1 = K1 = 5120
        g1 = torch.Generator(device=dev)
        g1.manual_seed(99)
        sets1 = []
        for i in range(16):  # 16 x 26 MB rotate past the 256 MB MALL
            w1 = torch.randint(-127, 128, (N1, K1), dtype=torch.int8, device=dev, generator=g1).t()
            sets1.append((qf.to_tiled(w1) if layout == qf.TILED else w1,
                          (torch.randn(N1, device=dev, generator=g1).abs() * 0.002 + 1e-4).float(),
                          torch.randn(1, K1, device=dev, generator=g1).to(torch.bfloat16)))
        for i in range(args.iters):
            w1, s1, x1 = sets1[i % len(sets1)]
            qf.w8a16_mm(x1, w1, s1, None, torch.bfloat16, layout)
        torch.cuda.synchronize()
        log(f"profile: {args.iters} launches of the single linear M=1 N=K=5120 layout={args.layout} "
            f"cfg={tuple(qf.resolve_config(1, N1, K1, layout))}")
        return

    if args.profile_gemm:
        N, K = GEMMS[args.profile_gemm]
        cfg = qf.W8A16Config(*[int(v) for v in args.cfg.split(",")]) if args.cfg else None
        sets = [Layer(torch, qf, dev, 1000 + i, M_TOKENS, layout) for i in range(args.layers)]
        for i in range(args.iters):
            sets[i % len(sets)].gemm(qf, torch, args.profile_gemm, cfg)
        torch.cuda.synchronize()
        log(f"profile: {args.iters} launches of {args.profile_gemm} M={M_TOKENS} N={N} K={K} layout={args.layout} "
            f"cfg={tuple(cfg) if cfg else tuple(qf.resolve_config(M_TOKENS, N, K, layout))}")
        return

    if args.workload == "stack64":
        run_stack64(torch, qf, dev, args)
        return
    if args.workload == "msweep":
        run_msweep(torch, qf, dev, args)
        return
    if args.workload == "lm_head":
        run_lm_head(torch, qf, dev, args)
        return
    if args.workload == "prefill":
        run_prefill(torch, qf, dev, args)
        return
    if args.workload == "spec_attn":
        run_spec_attn(torch, qf, dev, args)
        return
    if args.workload == "tp8":
        run_tp8(torch, qf, dev, args)
        return

    M = M_TOKENS
    R = max(1, args.layers)
    log(f"bench: allocating {R} layers ({R * sum(N * K for N, K in GEMMS.values()) / 1e9:.2f} GB of int8 weights)")
    layers = [Layer(torch, qf, dev, 1000 + i, M, layout) for i in range(R)]
    release_cache(torch)
    bytes_per_step = sum(algo_bytes(M, N, K) for (N, K) in GEMMS.values())

    # Steps are captured GRAPH_STEPS at a time (step i runs layer i % R), as a decode forward pass
    # captures all of its layers in one graph; K steps = K // GRAPH_STEPS replays of that graph plus
    # one graph holding the remaining K % GRAPH_STEPS steps.
    def steps_fn(first, count):
        return lambda: [layers[(first + i) % R].gemm(qf, torch, n) for i in range(count) for n in GEMMS]

    gsteps = GRAPH_STEPS - GRAPH_STEPS % R if GRAPH_STEPS >= R else R
    block = capture(torch, steps_fn(0, gsteps))[0]

    def run_steps(k):
        for _ in range(k // gsteps):
            block.replay()
        return k % gsteps

    rest_w = run_steps(args.warmup)
    torch.cuda.synchronize()
    tail = capture(torch, steps_fn(0, args.steps % gsteps))[0] if args.steps % gsteps else None
    if rest_w:
        capture(torch, steps_fn(0, rest_w))[0].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run_steps(args.steps)
    if tail is not None:
        tail.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    value = args.steps * bytes_per_step / elapsed / 1e9
    ms_per_step = elapsed / args.steps * 1e3
    log(f"bench: {args.steps} steps in {elapsed * 1e3:.1f} ms: {ms_per_step * 1e3:.2f} us/layer, {value:.0f} GB/s "
        f"({100 * value / PEAK_GBS:.1f}% of 8 TB/s)")

    # per-GEMM times: a graph of launches of one GEMM, its weights rotating over every layer's copy (all
    # allocated at start, as a model's weights are; 20 layers put even o_proj's copies past 768 MB, three times
    # the 256 MB MALL); HIP events on the current stream around each replay
    per_gemm = {}
    dominant_us = None
    for name, (N, K) in GEMMS.items():
        sets = [(L_.w[name], L_.s[name], L_.x[name]) for L_ in layers]
        reps = max(1, 40 // len(sets))
        g, _ = capture(torch, lambda: [qf.w8a16_mm(x_, w_, s_, None, torch.bfloat16, layout)
                                       for _ in range(reps) for (w_, s_, x_) in sets])
        launches = reps * len(sets)
        g.replay()
        torch.cuda.synchronize()
        times = []
        for _ in range(10):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            g.replay()
            e1.record()
            e1.synchronize()
            times.append(e0.elapsed_time(e1) * 1e3 / launches)
        us = sorted(times)[len(times) // 2]
        b = algo_bytes(M, N, K)
        cfg = qf.resolve_config(M, N, K, layout)
        per_gemm[name] = {"N": N, "K": K, "us": round(us, 2), "best_us": round(min(times), 2),
                          "weight_sets_rotated": len(sets), "rotated_MB": round(len(sets) * N * K / 1e6, 1),
                          "GB_s": round(b / us / 1e3, 1), "weight_GB_s": round(N * K / us / 1e3, 1),
                          "pct_peak": round(100 * b / us / 1e3 / PEAK_GBS, 1), "config": list(cfg)}
        log(f"  {name:8s} N={N:6d} K={K:6d}: {us:7.2f} us  {b / us / 1e3:7.0f} GB/s  "
            f"{100 * b / us / 1e3 / PEAK_GBS:5.1f}%  cfg={tuple(cfg)}")
        if name == DOMINANT:
            dominant_us = us
        del g, sets

    # The reference's single-linear case at one token: N = K = 5120, M = 1 (reported beside the step).
    single = {}
    N1, K1 = 5120, 5120
    g1 = torch.Generator(device=dev)
    g1.manual_seed(99)
    sets1 = []
    for i in range(16):  # 16 x 26 MB rotate past the 256 MB MALL
        w1 = torch.randint(-127, 128, (N1, K1), dtype=torch.int8, device=dev, generator=g1).t()
        sets1.append((qf.to_tiled(w1) if layout == qf.TILED else w1,
                      (torch.randn(N1, device=dev, generator=g1).abs() * 0.002 + 1e-4).float(),
                      torch.randn(1, K1, device=dev, generator=g1).to(torch.bfloat16)))
    release_cache(torch)
    best1 = []
    us1 = time_graph(torch, lambda: [qf.w8a16_mm(x1, w1, s1, None, torch.bfloat16, layout)
                                     for _ in range(8) for (w1, s1, x1) in sets1], 8 * len(sets1), best=best1)
    b1 = algo_bytes(1, N1, K1)
    single = {"N": N1, "K": K1, "M": 1, "us": round(us1, 2), "best_us": round(best1[0], 2),
              "GB_s": round(b1 / us1 / 1e3, 1), "weight_GB_s": round(N1 * K1 / us1 / 1e3, 1),
              "pct_peak": round(100 * b1 / us1 / 1e3 / PEAK_GBS, 1), "config": list(qf.resolve_config(1, N1, K1, layout))}
    log(f"  single linear M=1 N=K=5120: {us1:7.2f} us  {b1 / us1 / 1e3:7.0f} GB/s  {100 * b1 / us1 / 1e3 / PEAK_GBS:5.1f}%")
    del sets1
    release_cache(torch)

    dom_bytes = algo_bytes(M, *GEMMS[DOMINANT])
    achieved = dom_bytes / dominant_us / 1e3
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_GBS, 4), "traffic": read_traffic(),
                "kernel": f"{DOMINANT} M={M} N={GEMMS[DOMINANT][0]} K={GEMMS[DOMINANT][1]}",
                "algorithmic_bytes_per_launch": dom_bytes, "mean_launch_us": round(dominant_us, 2)}

    # the practical ceiling at each GEMM's size: the fastest of the library's read probes over the same bytes
    # (no math), each probe's time kept beside it
    for name, (N, K) in GEMMS.items():
        b = algo_bytes(M, N, K)
        detail = {}
        gbs = read_ceiling(torch, qf, dev, b, detail)
        per_gemm[name]["read_probe_us"] = round(b / gbs / 1e3, 2)
        per_gemm[name]["read_probes_us"] = detail
        per_gemm[name]["pct_of_read_probe"] = round(100 * per_gemm[name]["read_probe_us"] / per_gemm[name]["us"], 1)
        log(f"  read probe {name:8s} ({b / 1e6:6.1f} MB): {b / gbs / 1e3:7.2f} us  {gbs:6.0f} GB/s  {detail}")
        if name == DOMINANT:
            roofline["read_probe_GB_s"] = round(gbs, 1)
    b1 = algo_bytes(1, N1, K1)
    detail1 = {}
    gbs1 = read_ceiling(torch, qf, dev, b1, detail1)
    single["read_probe_us"] = round(b1 / gbs1 / 1e3, 2)
    single["read_probes_us"] = detail1
    single["pct_of_read_probe"] = round(100 * single["read_probe_us"] / single["us"], 1)

    # the launch floor: the period of back-to-back graph launches of a one-workgroup kernel that touches no
    # memory -- what every GEMM launch pays before it moves its bytes; a GEMM of B bytes cannot take less than
    # floor + B / 8 TB/s in this timing.  The same with a 16 KiB read adds one HBM round trip.
    floor = launch_floor(torch, qf, dev)
    floor_read = launch_floor(torch, qf, dev, 16384)
    log(f"  launch floor (graph of empty kernels): {floor:.2f} us per launch; with a 16 KiB read {floor_read:.2f} us")
    for name, (N, K) in list(GEMMS.items()) + [("single_linear_m1", (N1, K1))]:
        d = per_gemm[name] if name in per_gemm else single
        b = algo_bytes(1 if name == "single_linear_m1" else M, N, K)
        d["us_at_peak_with_floor"] = round(floor + b / PEAK_GBS / 1e3, 2)
        d["pct_peak_after_floor"] = round(100 * b / max(d["us"] - floor, 1e-3) / 1e3 / PEAK_GBS, 1)

    msweep = msweep_rows(torch, qf, dev, layout, layers)
    del layers
    release_cache(torch)
    lm_head = lm_head_rows(torch, qf, dev)
    vendor = vendor_decode(torch, qf, dev)
    stack = stack64(torch, qf, dev, layout, steps=10, warmup=2)

    cpu = None if args.no_cpu else cpu_baseline(M)

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded int8 weights, fp32 scales, bf16 N(0,1) activations)",
        "config": {"workload": "dense GQA 27B-class layer GEMMs at M=5: qkv 10240x5120, o_proj 5120x8192, "
                               "gate_up 34816x5120, down 5120x17408 (N x K int8)",
                   "M": M, "layers_rotated": R, "bytes_per_step": bytes_per_step, "weight_layout": args.layout,
                   "timing": f"hipGraphs of {gsteps} steps replayed; step i runs layer i % {R}"},
        "us_per_layer": round(ms_per_step * 1e3, 2),
        "pct_of_peak": round(100 * value / PEAK_GBS, 2),
        "per_gemm": per_gemm,
        "single_linear_m1": single,
        "launch_floor_us": round(floor, 2),
        "launch_floor_read16k_us": round(floor_read, 2),
        "msweep": msweep,
        "lm_head": lm_head,
        "vendor_decode": vendor,
        "stack64": stack,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def read_ceiling(torch, qf, dev, window: int, detail=None) -> float:
    """GB/s of the fastest read of `window` bytes this library has: its read probes over rotating windows of
    that size (at least 768 MB in all, past the 256 MB MALL), timed like the GEMMs.  Probes: the stream-shaped
    probe (one workgroup per CU over a contiguous share, 8 wavefronts at depth 4 or 8, 16 at depth 4) and the
    grid-stride probe (512 and 2048 workgroups); the best is the practical HBM read ceiling at that size, a
    launch included.  With a dict as `detail`, each probe's µs per window is recorded in it."""
    from qwen_fastpath import _lib as L
    window = window // 4096 * 4096
    nwin = max(8, -(-(768 << 20) // window))
    buf = torch.empty(nwin * window, dtype=torch.uint8, device=dev)
    buf.fill_(1)
    lib = L.load()
    sink = torch.empty(max(2048, int(lib.qf_device_cus())), dtype=torch.int32, device=dev)
    probes = [("grid_stride_%d" % b, lambda i, st, b=b: lib.qf_read_probe(buf.data_ptr() + i * window, window,
                                                                          sink.data_ptr(), b, st))
              for b in (512, 2048)]
    probes += [("stream_w%d_d%d" % (w, d), lambda i, st, w=w, d=d: lib.qf_read_probe_stream(
                   buf.data_ptr() + i * window, window, sink.data_ptr(), w, d, st)) for (w, d) in ((8, 4), (8, 8), (16, 4))]
    # at least 40 launches a graph, as the GEMM timings have: a graph's own start is then a small share
    reps = -(-40 // nwin)
    best = 0.0
    for name, call in probes:
        def fn(call=call):
            st = torch.cuda.current_stream().cuda_stream
            for _ in range(reps):
                for i in range(nwin):
                    L.check(call(i, st), "probe")

        us = time_graph(torch, fn, nwin * reps)
        if detail is not None:
            detail[name] = round(us, 2)
        best = max(best, window / us / 1e3)
    del buf
    return best


def launch_floor(torch, qf, dev, read_bytes: int = 0) -> float:
    """µs per launch of a graph of 64 back-to-back launches of one workgroup: a kernel that touches no memory
    (read_bytes = 0: the dispatch cost of a dependent launch on this device), or the library's read probe
    over read_bytes (dispatch plus one HBM round trip)."""
    from qwen_fastpath import _lib as L
    lib = L.load()
    if read_bytes:
        buf = torch.ones(read_bytes, dtype=torch.uint8, device=dev)
        sink = torch.empty(1, dtype=torch.int32, device=dev)

        def fn():
            st = torch.cuda.current_stream().cuda_stream
            for _ in range(64):
                L.check(lib.qf_read_probe(buf.data_ptr(), buf.numel(), sink.data_ptr(), 1, st), "probe")
    else:
        def fn():
            st = torch.cuda.current_stream().cuda_stream
            for _ in range(64):
                L.check(lib.qf_empty_kernel(st), "empty kernel")

    return time_graph(torch, fn, 64)


def time_graph(torch, fn, launches, reps=10, best=None):
    """Median µs per launch of a captured fn() that issues `launches` launches; with a list as `best`,
    the fastest replay's µs per launch is appended to it."""
    g, _ = capture(torch, fn)
    g.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1) * 1e3 / launches)
    del g
    if best is not None:
        best.append(min(times))
    return sorted(times)[len(times) // 2]


def msweep_rows(torch, qf, dev, layout, layers=None) -> dict:
    """gate_up (N=34816, K=5120) at M = 1, 2, 3, 5, 8, 12, 16 over rotating weight sets past the 256 MB MALL (the
    given layers' gate_up weights, else 5 sets of its own, 891 MB), each M a graph of 40 launches timed with HIP
    events: {M: µs, GB/s, % of 8 TB/s, config}."""
    N, K = GEMMS["gate_up"]
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    if layers is not None:
        sets = [(L_.w["gate_up"], L_.s["gate_up"]) for L_ in layers[:8]]
    else:
        sets = []
        for i in range(5):
            w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g).t()
            sets.append((qf.to_tiled(w) if layout == qf.TILED else w,
                         (torch.randn(N, device=dev, generator=g).abs() * 0.002 + 1e-4).float()))
            del w
        release_cache(torch)
    R = len(sets)
    rows = {}
    for M in (1, 2, 3, 5, 8, 12, 16):
        xs = [torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16) for _ in range(R)]
        reps = max(1, 40 // R)
        us = time_graph(torch, lambda: [qf.w8a16_mm(xs[i], w, s, None, torch.bfloat16, layout)
                                        for _ in range(reps) for i, (w, s) in enumerate(sets)], reps * R)
        b = algo_bytes(M, N, K)
        rows[M] = {"us": round(us, 2), "GB_s": round(b / us / 1e3, 1), "pct_peak": round(100 * b / us / 1e3 / PEAK_GBS, 1),
                   "config": list(qf.resolve_config(M, N, K, layout))}
        log(f"  gate_up M={M:2d}: {us:7.2f} us  {b / us / 1e3:7.0f} GB/s  {100 * b / us / 1e3 / PEAK_GBS:5.1f}%")
    del sets
    torch.cuda.empty_cache()
    return rows


def run_msweep(torch, qf, dev, args):
    """gate_up (N=34816, K=5120) at M = 1, 2, 3, 5, 8, 12, 16 (msweep_rows) as its own line."""
    layout = qf.TILED if args.layout == "tiled" else qf.ROWMAJOR
    rows = msweep_rows(torch, qf, dev, layout)
    worst = min(r["GB_s"] for r in rows.values())
    line = {"metric": METRIC, "value": worst, "unit": "GB/s", "n_gpus": 1, "steps": 10, "warmup": 2,
            "ms_per_step": round(rows[5]["us"] / 1e3, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded int8 weights, fp32 scales, bf16 activations)",
            "config": {"workload": "gate_up 34816x5120 M sweep (value = the slowest M's GB/s)", "weight_layout": args.layout},
            "per_m": rows}
    print(json.dumps(line), flush=True)


def vendor_decode(torch, qf, dev, M: int = 5) -> dict:
    """The platform's own GEMMs at the decode width, beside the kernel (context, as the reference times CUTLASS
    next to its kernel, data/measurements.json:371-378): per layer GEMM, (a) F.linear on bf16 weights widened
    ahead of time (hipBLASLt; twice the weight bytes), (b) torch._int_mm on int8 activations padded to 32 rows
    and the row-major int8 weights (int32 out; the W8A8 arithmetic without its quantiser and epilogue).  Weights
    rotate over sets past the MALL; µs per call from HIP events around a graph, and each route's GB/s of the
    layer GEMM's algorithmic W8A16 bytes (what the kernel moves) for comparison."""
    import torch.nn.functional as F
    out = {}
    g = torch.Generator(device=dev)
    g.manual_seed(23)
    for name, (N, K) in GEMMS.items():
        row = {}
        b = algo_bytes(M, N, K)
        nset = max(3, -(-(768 << 20) // (2 * N * K)))
        try:
            ws = [(torch.randint(-127, 128, (N, K), device=dev, generator=g, dtype=torch.int8).to(torch.bfloat16)
                   * 0.01) for _ in range(nset)]
            x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
            us = time_graph(torch, lambda: [F.linear(x, w) for _ in range(4) for w in ws], 4 * nset)
            row["bf16_linear_us"] = round(us, 2)
            row["bf16_linear_pct_of_w8a16_bytes"] = round(100 * b / us / 1e3 / PEAK_GBS, 1)
            del ws
        except Exception as e:  # noqa: BLE001 - context figure only
            row["bf16_linear_error"] = str(e)[:120]
        try:
            nset8 = max(3, -(-(768 << 20) // (N * K)))
            ws8 = [torch.randint(-127, 128, (N, K), device=dev, generator=g, dtype=torch.int8) for _ in range(nset8)]
            xq = torch.randint(-127, 128, (32, K), device=dev, generator=g, dtype=torch.int8)
            us = time_graph(torch, lambda: [torch._int_mm(xq, w.t()) for _ in range(4) for w in ws8], 4 * nset8)
            row["int8_int_mm_m32_us"] = round(us, 2)
            row["int8_int_mm_pct_of_w8a16_bytes"] = round(100 * b / us / 1e3 / PEAK_GBS, 1)
            del ws8
        except Exception as e:  # noqa: BLE001 - context figure only
            row["int8_int_mm_error"] = str(e)[:120]
        torch.cuda.empty_cache()
        out[name] = row
        log(f"  vendor {name:8s} M={M}: {row}")
    return out


def w8a8_gate_up_gemm(torch, qf, dev, g, M, sets, name="gate_up"):
    """The W8A8 GEMM alone on a layer GEMM (gate_up by default) at M rows (activations quantised once,
    beforehand, in the layout w8a8_mm gives that kernel; a K split gets its own workspace): returns a callable
    that runs it on weight set i, and its configuration."""
    import ctypes
    from qwen_fastpath import _lib as QL
    N, K = GEMMS[name]
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    lib = QL.load()
    cfg = QL.w8a8_pick_config(M, N, K)
    x_tiled = cfg.kernel == QL.KERNEL_MFMA_W8A8_TILE
    xq, s_a = qf.quantize_tokens_int8(x, tiled=x_tiled)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    need = int(lib.qf_w8a8_workspace_bytes(M, N, K, qf.TILED, ctypes.byref(cfg)))
    ws = torch.zeros(max(need, 16), dtype=torch.uint8, device=dev)  # arrival counters start at zero
    ws_ptr = ws.data_ptr() if need else None

    def gemm(i):
        st = torch.cuda.current_stream().cuda_stream
        if x_tiled:
            QL.check(lib.qf_w8a8_gemm_xt(xq.data_ptr(), s_a.data_ptr(), sets[i][0].data_ptr(), 0, qf.TILED,
                                         sets[i][1].data_ptr(), y.data_ptr(), N, QL.DTYPE_BF16, M, N, K,
                                         ctypes.byref(cfg), ws_ptr, need, st), "qf_w8a8_gemm_xt")
        else:
            QL.check(lib.qf_w8a8_gemm(xq.data_ptr(), K, s_a.data_ptr(), sets[i][0].data_ptr(), 0, qf.TILED,
                                      sets[i][1].data_ptr(), y.data_ptr(), N, QL.DTYPE_BF16, M, N, K, ctypes.byref(cfg),
                                      ws_ptr, need, st), "qf_w8a8_gemm")
    return gemm, cfg


def prefill_weight_sets(torch, qf, dev, g, count=2, name="gate_up"):
    """A layer GEMM's (gate_up by default) int8 weights in the TILED layout with fp32 scales, `count`
    distinct sets."""
    N, K = GEMMS[name]
    sets = []
    for _ in range(count):
        w = qf.to_tiled(torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g).t())
        sets.append((w, (torch.randn(N, device=dev, generator=g).abs() * 0.002 + 1e-4).float()))
    return sets


def prefill_layer_rows(torch, qf, dev, g, widths=(512, 1024, 2048)):
    """The layer's four GEMMs through the W8A8 route the dispatcher takes for M > 16 on TILED weights
    (quantiser + int8 GEMM, as w8a8_mm runs them), two weight sets per shape rotated: µs, int8 TOPS and the
    configuration the automatic rule picks (a K split on the narrow-N shapes at the smaller widths)."""
    from qwen_fastpath import _lib as QL
    out = {}
    for name in ("qkv", "o_proj", "gate_up", "down"):
        N, K = GEMMS[name]
        sets = []
        for _ in range(2):
            w = qf.to_tiled(torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g).t())
            sets.append((w, (torch.randn(N, device=dev, generator=g).abs() * 0.002 + 1e-4).float()))
        for M in widths:
            x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
            f = lambda i: qf.w8a8_mm(x, sets[i][0], sets[i][1], torch.bfloat16)  # noqa: E731
            us = min(time_graph(torch, lambda: [f(i) for _ in range(2) for i in range(2)], 4, reps=5)
                     for _ in range(2))
            tops = 2.0 * M * N * K / us / 1e6
            cfg = QL.w8a8_pick_config(M, N, K)
            out[f"{name} M={M}"] = {"N": N, "K": K, "M": M, "us": round(us, 1), "TOPS": round(tops, 1),
                                    "pct_int8_mfma_peak": round(100 * tops / 5000.0, 1), "config": cfg.to_tuple()}
            log(f"  prefill {name:7s} M={M:5d}: w8a8 {us:8.1f} us {tops:7.1f} TOPS cfg {cfg.to_tuple()}")
        del sets
    return out


def run_prefill(torch, qf, dev, args):
    """gate_up (N=34816, K=5120) at prefill widths M = 64 ... 2048 on TILED weights, two weight sets
    rotated (356 MB, past the 256 MB last-level cache), three routes timed interleaved (best of 2
    medians):
    * w8a8: the reference's M > 16 arithmetic (per-token int8 activations, exact int32 sums on the int8
      MFMA), the dispatcher's default (QWEN_FAST_LINEAR_PREFILL=w8a8);
    * wide: the W8A16 wide-M kernel (the w8a16 setting up to TILED_WIDE_MAX_M rows);
    * widened: exact bf16 widening + hipBLASLt bf16 GEMM + one scale/cast pass (w8a16 above that)."""
    from qwen_fastpath import _lib as QL
    from qwen_fastpath.patches import TILED_WIDE_MAX_M
    N, K = GEMMS["gate_up"]
    g = torch.Generator(device=dev)
    g.manual_seed(13)
    sets = prefill_weight_sets(torch, qf, dev, g)
    rows = {}
    for M in (64, 256, 512, 1024, 2048):
        x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
        paths = {"w8a8": lambda i: qf.w8a8_mm(x, sets[i][0], sets[i][1], torch.bfloat16),
                 "wide": lambda i: qf.w8a16_mm(x, sets[i][0], sets[i][1], None, torch.bfloat16, qf.TILED),
                 "widened": lambda i: qf.w8a16_mm_prefill(x, sets[i][0], sets[i][1], torch.bfloat16, qf.TILED)}
        t = {}
        for _ in range(2):
            for k, f in paths.items():
                us = time_graph(torch, lambda: [f(i) for _ in range(2) for i in range(2)], 4, reps=5)
                t[k] = min(t.get(k, float("inf")), us)
        us = t["w8a8"]
        w8a16 = "wide" if M <= TILED_WIDE_MAX_M else "widened"
        tflops = 2.0 * M * N * K / us / 1e6
        rows[M] = {"us": round(us, 1), "TOPS": round(tflops, 1), "pct_int8_mfma_peak": round(100 * tflops / 5000.0, 1),
                   "path": "w8a8", "us_w8a16": round(t[w8a16], 1), "w8a16_path": w8a16,
                   "us_w8a16_wide_kernel": round(t["wide"], 1), "us_w8a16_widened_gemm": round(t["widened"], 1)}
        log(f"  prefill gate_up M={M:5d}: w8a8 {us:8.1f} us {tflops:7.1f} TOPS | w8a16: wide kernel {t['wide']:.1f} us, "
            f"widened + library GEMM {t['widened']:.1f} us")
    # Roofline of the dominant kernel at M = 2048: the W8A8 GEMM alone (activations quantised beforehand),
    # HIP events around graph replays on the stream it is launched on.  MFMA-bound: 2MNK int8 ops.
    M = 2048
    gemm, cfg = w8a8_gate_up_gemm(torch, qf, dev, g, M, sets)
    us_k = min(time_graph(torch, lambda: [gemm(i) for _ in range(2) for i in range(2)], 4, reps=5) for _ in range(2))
    tops_k = 2.0 * M * N * K / us_k / 1e6
    log(f"  prefill gate_up M= 2048 W8A8 GEMM alone: {us_k:.1f} us {tops_k:.1f} TOPS ({100 * tops_k / 5000:.1f}% of 5 POP/s)")
    # The same int8 product through the vendor GEMM (torch._int_mm, hipBLASLt) on a row-major copy of the
    # weights, int32 output: what the platform's own int8 GEMM reaches at this shape.
    xq = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev, generator=g)
    wrm = [qf.from_tiled(w, N, K) for w, _ in sets]  # [K, N] views of [N, K] row-major int8
    us_v = min(time_graph(torch, lambda: [torch._int_mm(xq, wrm[i]) for _ in range(2) for i in range(2)], 4, reps=5)
               for _ in range(2))
    tops_v = 2.0 * M * N * K / us_v / 1e6
    log(f"  prefill gate_up M= 2048 vendor int8 GEMM (torch._int_mm): {us_v:.1f} us {tops_v:.1f} TOPS")
    del wrm
    # The tile kernel's call is two launches when its workgroups pass whole rounds of 256 by at most 64
    # (reduce 0): the whole rounds' channel blocks, then the rest on 128 x 128 tile workgroups when they
    # make one round of 128 to 256, else on the wide kernel.
    mb = -(-M // 256)
    tile_wgs = -(-N // 256) * mb
    whole = tile_wgs // 256 * 256
    tail = cfg.reduce == 0 and whole > 0 and 0 < tile_wgs - whole <= 64 and whole % mb == 0
    tile_name = "w8a8_tile_kernel"
    if tail:
        n_tail = N - whole // mb * 256
        small = -(-(-(-n_tail // 16)) // 8) * -(-M // 128)
        tile_name += (f" + {small} 128x128 tile workgroups on the last {n_tail} channels" if 128 <= small <= 256
                      else f" + w8a8_wide_kernel on the last {n_tail} channels")
    tile_name += ", token-tiled activations"
    roofline = {"bound": "mfma", "achieved": round(tops_k, 1), "peak": 5000.0, "unit": "TOPS",
                "frac": round(tops_k / 5000.0, 4), "traffic": read_traffic(W8A8_PROFILE),
                "kernel": (f"{tile_name if cfg.kernel == QL.KERNEL_MFMA_W8A8_TILE else 'w8a8_wide_kernel'} "
                           f"gate_up M=2048 N={N} K={K} (int8 MFMA, cfg {cfg.to_tuple()})"),
                "vendor_int8_gemm": {"us": round(us_v, 1), "TOPS": round(tops_v, 1),
                                     "what": "torch._int_mm (hipBLASLt) on row-major int8 weights, int32 output"}}
    line = {"metric": METRIC, "value": rows[2048]["TOPS"], "unit": "TOPS", "n_gpus": 1, "steps": 4, "warmup": 1,
            "ms_per_step": round(rows[2048]["us"] / 1e3, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "int8", "data": "synthetic (seeded int8 weights, fp32 scales, bf16 activations)",
            "config": {"workload": "gate_up 34816x5120 prefill widths on TILED weights, W8A8 (value = M=2048 TOPS)"},
            "per_m": rows, "roofline": roofline}
    del sets
    line["layer_w8a8"] = prefill_layer_rows(torch, qf, dev, g)
    if not args.no_cpu:
        line["cpu_baseline"] = prefill_cpu_baseline()
    print(json.dumps(line), flush=True)


def prefill_cpu_baseline(M: int = 2048, N: int = 2048, K: int = 5120):
    """The oracle's fp32-dequant restatement of the reference CPU path (bench/test_w8a16.py:15) at a
    prefill width, on an N-channel slice of gate_up, best of 3, in TFLOP/s."""
    from oracle import oracle as O
    cores = max(1, min(len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1), 16))
    try:
        from threadpoolctl import threadpool_limits
        threadpool_limits(limits=cores)
    except Exception:  # noqa: BLE001 - threadpoolctl optional
        pass
    inp = O.gen_inputs(M, N, K, seed=6)
    best = float("inf")
    for _ in range(3):
        t0 = time.perf_counter()
        O.fp32_dequant_linear(inp.x, inp.w, inp.s)
        best = min(best, time.perf_counter() - t0)
    return {"value": round(2.0 * M * N * K / best / 1e12, 4), "unit": "TOPS", "cores": cores, "kind": "port",
            "sample": f"M={M} over a {N}-channel slice of gate_up (K={K}), fp32 dequant linear, best of 3 over "
                      f"{cores} threads: {best * 1e3:.1f} ms"}


# One tensor-parallel rank's share of the layer at TP = 8: qkv and gate_up split N (column-parallel), o_proj
# and down split K (row-parallel; the all-reduce that would follow them is not part of this measurement).
TP8_GEMMS = {"qkv": (1280, 5120), "o_proj": (5120, 1024), "gate_up": (4352, 5120), "down": (5120, 2176)}


def run_tp8(torch, qf, dev, args):
    """The layer's four GEMMs at M=5 on one TP=8 rank's shapes, TILED weights, 16 layers rotated (726 MB)."""
    layout = qf.TILED if args.layout == "tiled" else qf.ROWMAJOR
    M, R = M_TOKENS, 16
    g = torch.Generator(device=dev)
    g.manual_seed(17)
    layers = []
    for _ in range(R):
        sets = {}
        for name, (N, K) in TP8_GEMMS.items():
            w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g).t()
            sets[name] = (qf.to_tiled(w) if layout == qf.TILED else w,
                          (torch.randn(N, device=dev, generator=g).abs() * 0.002 + 1e-4).float(),
                          torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16))
            del w
        layers.append(sets)

    def gemm(sets, name):
        w, s_, x = sets[name]
        return qf.w8a16_mm(x, w, s_, None, torch.bfloat16, layout)

    rows = {}
    for name, (N, K) in TP8_GEMMS.items():
        us = time_graph(torch, lambda n=name: [gemm(L_, n) for _ in range(8) for L_ in layers], 8 * R)
        b = algo_bytes(M, N, K)
        rows[name] = {"N": N, "K": K, "us": round(us, 2), "GB_s": round(b / us / 1e3, 1),
                      "pct_peak": round(100 * b / us / 1e3 / PEAK_GBS, 1),
                      "config": list(qf.resolve_config(M, N, K, layout))}
        log(f"  tp8 {name:8s} N={N:5d} K={K:5d}: {us:6.2f} us  {b / us / 1e3:6.0f} GB/s  {100 * b / us / 1e3 / PEAK_GBS:5.1f}%")
    us_layer = time_graph(torch, lambda: [gemm(L_, n) for _ in range(4) for L_ in layers for n in TP8_GEMMS], 4 * R)
    b_layer = sum(algo_bytes(M, N, K) for N, K in TP8_GEMMS.values())
    log(f"  tp8 layer step (4 GEMMs): {us_layer:6.2f} us  {b_layer / us_layer / 1e3:6.0f} GB/s  "
        f"{100 * b_layer / us_layer / 1e3 / PEAK_GBS:5.1f}%")
    line = {"metric": METRIC, "value": round(b_layer / us_layer / 1e3, 1), "unit": "GB/s", "n_gpus": 1, "steps": 10,
            "warmup": 2, "ms_per_step": round(us_layer / 1e3, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded int8 weights, fp32 scales, bf16 activations)",
            "config": {"workload": "one TP=8 rank's layer GEMMs at M=5 (qkv 1280x5120, o_proj 5120x1024, "
                                   "gate_up 4352x5120, down 5120x2176), 16 layers rotated; no all-reduce",
                       "weight_layout": args.layout},
            "per_gemm": rows}
    print(json.dumps(line), flush=True)


def lm_head_cpu_baseline(M: int = 1, rows: int = 16384, H: int = 5120):
    """The reference's draft-head path on the host (patches.py:160-166,178-185 in the oracle's fp32-dequant
    form): logits = x . (w * s)^T in fp32, rounded to bf16, the pad columns masked, argmax.  Timed on a
    vocabulary slice of `rows` rows, best of 3, as GB/s of the slice's compulsory bytes."""
    import numpy as np
    from oracle import oracle as O
    cores = max(1, min(len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1), 16))
    try:
        from threadpoolctl import threadpool_limits
        threadpool_limits(limits=cores)
    except Exception:  # noqa: BLE001 - threadpoolctl optional
        pass
    inp = O.gen_inputs(M, rows, H, seed=5)
    best = float("inf")
    for _ in range(3):
        t0 = time.perf_counter()
        logits = O.fp32_dequant_linear(inp.x, inp.w, inp.s)
        O.argmax_rows(O.bf16_from_f64(logits.astype(np.float64)), rows - 64, 0)
        best = min(best, time.perf_counter() - t0)
    b = rows * H + 4 * rows + 2 * M * H + 8 * M
    return {"value": round(b / best / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"M={M}, a {rows}-row slice of the 151936x5120 head ({b / 1e6:.1f} MB), fp32 dequant linear + "
                      f"bf16 rounding + pad mask + argmax, best of 3 over {cores} threads: {best * 1e3:.1f} ms"}


def lm_head_rows(torch, qf, dev) -> dict:
    """Int8 MTP draft head: V=151936, H=5120, at M = 1 and 4, with the draft-head configuration's inputs: int8
    weights uniform in [-127, 127] and per-row scales |N(0,1)| * 0.002 + 1e-4 (the head's TILED copy), bf16
    N(0,1) hidden rows.  One step = W8A16 logits for M hidden rows plus the pad-masked argmax (64 pad columns,
    vocab offset 0), fused into the GEMM epilogue (the default) and as logits then argmax; weights rotate over
    2 copies (1.56 GB)."""
    V, H, num_pad = 151936, 5120, 64
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    heads = []
    for i in range(2):
        w = torch.randint(-127, 128, (V, H), dtype=torch.int8, device=dev, generator=g)
        sc = (torch.randn(V, device=dev, generator=g).abs() * 0.002 + 1e-4).float()
        heads.append(qf.Int8Head(qf.to_tiled(w.t()), sc, num_pad, qf.pick_config(V, H, qf.TILED), qf.TILED))
        del w
    release_cache(torch)
    rows = {}
    for M in (1, 4):
        hs = [torch.randn(M, H, device=dev, generator=g).to(torch.bfloat16) for _ in heads]

        def step(i):  # W8A16 logits, then the pad-masked argmax over them
            return qf.int8_top_tokens(heads[i], hs[i], 0, fused=False)

        def step_fused(i):  # argmax folded into the GEMM epilogue (logits neither written nor re-read)
            return qf.int8_top_tokens(heads[i], hs[i], 0, fused=True)

        def logits(i):  # the GEMM alone
            return qf.int8_logits(heads[i], hs[i])
        reps = 8
        launches = reps * len(heads)
        us, us2, us3 = float("inf"), float("inf"), float("inf")
        for _ in range(3):  # interleaved, the best of three each: the first graph timed after set-up runs slower
            us = min(us, time_graph(torch, lambda: [step(i) for _ in range(reps) for i in range(len(heads))], launches))
            us2 = min(us2, time_graph(torch, lambda: [step_fused(i) for _ in range(reps) for i in range(len(heads))],
                                      launches))
            us3 = min(us3, time_graph(torch, lambda: [logits(i) for _ in range(reps) for i in range(len(heads))],
                                      launches))
        b = algo_bytes(M, V, H) - 2 * M * V + 8 * M  # compulsory: weights, scales and x read, M ids written
        bg = algo_bytes(M, V, H)
        best = us2  # int8_top_tokens' default: the fused epilogue
        rows[M] = {"us_per_draft_step": round(best, 2), "GB_s": round(b / best / 1e3, 1),
                   "pct_peak": round(100 * b / best / 1e3 / PEAK_GBS, 1), "algorithmic_bytes": b,
                   "us_logits_then_argmax": round(us, 2), "us_fused_epilogue": round(us2, 2),
                   "us_gemm_alone": round(us3, 2), "gemm_alone_pct_peak": round(100 * bg / us3 / 1e3 / PEAK_GBS, 1)}
        log(f"  lm_head M={M}: logits + argmax {us:7.2f} us, argmax fused into the epilogue {us2:7.2f} us, GEMM alone "
            f"{us3:7.2f} us;  fused {b / best / 1e3:6.0f} GB/s  {100 * b / best / 1e3 / PEAK_GBS:5.1f}%")
    del heads
    torch.cuda.empty_cache()
    return rows


def run_lm_head(torch, qf, dev, args):
    """The int8 draft head (lm_head_rows) as its own line, with its CPU baseline."""
    rows = lm_head_rows(torch, qf, dev)
    line = {"metric": METRIC, "value": rows[1]["GB_s"], "unit": "GB/s", "n_gpus": 1, "steps": 10, "warmup": 2,
            "ms_per_step": round(rows[1]["us_per_draft_step"] / 1e3, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (int8 uniform [-127, 127] weights, per-row fp32 scales |N(0,1)|*0.002+1e-4)",
            "config": {"workload": "int8 draft lm_head 151936x5120 plus the pad-masked argmax, ids out "
                                   "(value = M=1 GB/s of compulsory bytes)",
                       "weight_layout": "tiled"},
            "per_m": rows}
    if not args.no_cpu:
        line["cpu_baseline"] = lm_head_cpu_baseline(1)
    print(json.dumps(line), flush=True)


# The reference kernel's published latency per full-attention layer on an A100 (µs), by (Q, requests)
# and cached context: data/measurements.json "attention_kernel" (ours_Q3, ours_Q4, ours_Q3_B2).
ATTN_REF_A100_US = {
    (3, 1): {1000: 23.9, 8000: 41.6, 38000: 126.2, 100000: 294.1},
    (4, 1): {1000: 24.4, 8000: 43.8, 38000: 129.1, 100000: 294.7},
    (3, 2): {1000: 26.5, 8000: 70.2, 38000: 236.1, 100000: 565.5},
}
ATTN_METRIC = ("split-KV verification attention: KV-cache GB/s (% of 8 TB/s) and µs per full-attention layer, "
               "38K context, Q=3, 1 request")
ATTN_PROFILE = os.path.join(ROOT, "profiles", "spec_attn_kernel_trace.md")


def attn_kv_bytes(lens, HKV=4, D=256) -> int:
    """Compulsory bytes of one call: every cached position's K and V rows of every kv head, once."""
    return sum(int(n) for n in lens) * HKV * 2 * D * 2


def attn_cpu_baseline(ctx=38000, Q=3):
    """The oracle's fp64 restatement of the reference gold (bench/test_spec_attn.py:23-31) on one layer."""
    import numpy as np
    from oracle import attn as A
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    cores = max(1, min(cores, 16))
    try:
        from threadpoolctl import threadpool_limits
        threadpool_limits(limits=cores)
    except Exception:  # noqa: BLE001 - threadpoolctl optional
        pass
    inp = A.gen_spec_inputs(ctx, Q, 1, seed=0)
    q, kc, vc = inp.query(), inp.key_cache(), inp.value_cache()
    best = float("inf")
    for _ in range(2):
        t0 = time.perf_counter()
        A.spec_attention(q, kc, vc, inp.seq_lens, inp.block_table, 1, Q, 4, 256 ** -0.5)
        best = min(best, time.perf_counter() - t0)
    b = attn_kv_bytes(inp.seq_lens)
    return {"value": round(b / best / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"one layer at ctx={ctx}, Q={Q}, 1 request ({b / 1e6:.1f} MB of KV), fp64 numpy over "
                      f"{cores} threads, best of 2: {best * 1e3:.0f} ms/layer"}


def run_spec_attn(torch, qf, dev, args):
    """One full-attention layer of the 27B model (H=24, H_kv=4, D=256, 800-position pages, K and V
    interleaved per row as [page][H_kv][PAGE][2D]) at the reference's contexts and batch shapes
    (bench/test_spec_attn.py:7-19).  Each layer's pages come from a shared 1.7 GB pool through its own
    shuffled block table, and the calls rotate over enough layers (>= 2, > 512 MB) that every call
    streams its KV from HBM; calls are captured in a graph."""
    H, HKV, D, PAGE = 24, 4, 256, 800
    npages = 520
    g = torch.Generator(device=dev)
    g.manual_seed(21)
    kv = torch.randn(npages, HKV, PAGE, 2 * D, device=dev, generator=g).to(torch.bfloat16)
    key_cache, value_cache = kv.transpose(1, 2).split(D, dim=-1)
    rows = {}
    cases = [(Q, B, ctx) for (Q, B) in ATTN_REF_A100_US for ctx in (1000, 8000, 38000, 100000)]
    if args.attn_case:
        ctx, Q, B = (int(v) for v in args.attn_case.split(","))
        cases = [(Q, B, ctx)]
    for Q, B, ctx in cases:
        ref = ATTN_REF_A100_US.get((Q, B), {})
        if True:
            L = ctx + Q
            lens = [max(L - 7 * b, 1) for b in range(B)]
            nblk = (L + PAGE - 1) // PAGE + 1
            per_layer = B * nblk
            # enough layers that one pass reads > 640 MB of KV (2.5x the MALL), within the pool
            n_layers = max(2, min(128, npages // per_layer, -(-(640 << 20) // attn_kv_bytes(lens, HKV, D))))
            assert n_layers * per_layer <= npages
            perm = torch.randperm(npages, device=dev, generator=g).to(torch.int32)
            tables = [perm[i * per_layer:(i + 1) * per_layer].view(B, nblk).contiguous() for i in range(n_layers)]
            seq_lens = torch.tensor(lens, dtype=torch.int32, device=dev)
            q = torch.randn(B * Q, H, D, device=dev, generator=g).to(torch.bfloat16)
            out = torch.empty_like(q)
            scale = D ** -0.5

            def call(i):
                qf.gqa_packed_spec_attention(q, key_cache, value_cache, out, seq_lens, tables[i], B, Q, HKV, scale)
            if args.attn_case:
                for it in range(args.iters):
                    call(it % n_layers)
                torch.cuda.synchronize()
                log(f"spec_attn profile: {args.iters} calls at ctx={ctx} Q={Q} B={B}, {n_layers} layers rotated")
                return
            reps = max(1, 32 // n_layers)
            us = time_graph(torch, lambda: [call(i) for _ in range(reps) for i in range(n_layers)], reps * n_layers)
            b = attn_kv_bytes(lens, HKV, D)
            key = f"Q{Q}_B{B}_ctx{ctx}"
            rows[key] = {"us": round(us, 2), "GB_s": round(b / us / 1e3, 1), "pct_peak": round(100 * b / us / 1e3 / PEAK_GBS, 1),
                         "kv_bytes": b, "reference_a100_us": ref.get(ctx),
                         "speedup_vs_reference_a100": round(ref[ctx] / us, 2) if ctx in ref else None,
                         "layers_rotated": n_layers}
            log(f"  spec_attn Q={Q} B={B} ctx={ctx:6d}: {us:8.2f} us  {b / us / 1e3:7.0f} GB/s  "
                f"{100 * b / us / 1e3 / PEAK_GBS:5.1f}%  (reference on A100: {ref.get(ctx)} us)")
    head = rows["Q3_B1_ctx38000"]
    line = {"metric": ATTN_METRIC, "value": head["GB_s"], "unit": "GB/s", "n_gpus": 1, "steps": 10, "warmup": 2,
            "ms_per_step": round(head["us"] / 1e3, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic (N(0,1) bf16 queries and KV cache, shuffled pages)",
            "config": {"workload": "one full-attention layer, H=24 H_kv=4 D=256, 800-position pages; value = "
                                   "ctx 38000, Q=3, 1 request", "num_splits": "auto: CUs / (requests x kv heads) (64 at 1 request)", "min_chunk": 64},
            # achieved: KV bytes / duration of the whole layer call (prefix + combine kernels, HIP events
            # on the launch stream); traffic: the prefix kernel's FETCH_SIZE + WRITE_SIZE bytes per launch
            "roofline": {"bound": "hbm", "achieved": head["GB_s"], "peak": PEAK_GBS, "unit": "GB/s",
                         "frac": round(head["GB_s"] / PEAK_GBS, 4), "traffic": read_traffic(ATTN_PROFILE)},
            "per_case": rows}
    if not args.no_cpu:
        line["cpu_baseline"] = attn_cpu_baseline()
    print(json.dumps(line), flush=True)


class StackLayer:
    """One layer of the 64-layer stack: its four weights drawn straight into the layout the GEMMs read
    (random int8 in [-127, 127]; the TILED image is a permutation of the row-major weight, so random bytes
    in it are a random weight) and scales |N(0,1)|*0.002 + 1e-4."""

    def __init__(self, torch, qf, dev, seed: int, layout: int):
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.w, self.s = {}, {}
        for name, (N, K) in GEMMS.items():
            if layout == qf.TILED:
                self.w[name] = torch.randint(-127, 128, (qf.tiled_numel(N, K),), dtype=torch.int8, device=dev,
                                             generator=g)
            else:
                self.w[name] = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g).t()
            self.s[name] = torch.randn(N, device=dev, generator=g).abs_().mul_(0.002).add_(1e-4)


def stack64(torch, qf, dev, layout: int, steps: int, warmup: int) -> dict:
    """64 layers x 4 GEMMs at M=5 with distinct weights (23.2 GB), one hipGraph per decode step.  Glue
    between GEMMs (the workload leaves it open): o_proj reads the first 8192 qkv outputs and down the
    first 17408 gate_up outputs, both as strided views (no copy); the next layer's input is the layer
    output re-normalised to unit RMS per row, done by the next qkv GEMM as it stages its input
    (qf_w8a16_gemm_rmsnorm: the bits of qf_rms_norm_rows_bf16 then the GEMM).  Timed by wall clock around
    `steps` replays after `warmup`."""
    M = M_TOKENS
    nl = 64
    log(f"stack64: allocating {nl} layers ({nl * sum(N * K for N, K in GEMMS.values()) / 1e9:.1f} GB)")
    layers = [StackLayer(torch, qf, dev, 5000 + i, layout) for i in range(nl)]
    release_cache(torch)
    x0 = torch.randn(M, 5120, device=dev).to(torch.bfloat16)

    def step():
        d = None
        for L_ in layers:
            mm = lambda a, n: qf.w8a16_mm(a, L_.w[n], L_.s[n], None, torch.bfloat16, layout)  # noqa: E731
            # the layer input: x0, then the previous layer's output scaled to unit RMS per row (torch rms_norm's
            # default eps for bf16), normalised inside the qkv GEMM's staging (the same bits as
            # qf_rms_norm_rows_bf16 followed by the GEMM, without a launch of its own)
            qkv = mm(x0, "qkv") if d is None else qf.w8a16_mm_rmsnorm(d, L_.w["qkv"], L_.s["qkv"], None,
                                                                      torch.bfloat16, layout)
            o = mm(qkv[:, :8192], "o_proj")
            gu = mm(o, "gate_up")
            d = mm(gu[:, :17408], "down")
        return qf.rms_norm_rows(d)  # the step's output: the last layer's, normalised

    g, _ = capture(torch, step)
    bytes_per_step = nl * sum(algo_bytes(M, N, K) for (N, K) in GEMMS.values())
    for _ in range(max(1, warmup)):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g.replay()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    value = steps * bytes_per_step / el / 1e9
    log(f"stack64: {steps} steps, {el / steps * 1e3:.3f} ms/step, {value:.0f} GB/s "
        f"({100 * value / PEAK_GBS:.1f}% of 8 TB/s)")
    del g, layers
    return {"layers": nl, "M": M, "steps": steps, "warmup": max(1, warmup), "bytes_per_step": bytes_per_step,
            "ms_per_step": round(el / steps * 1e3, 4), "us_per_layer": round(el / steps / nl * 1e6, 2),
            "GB_s": round(value, 1), "pct_peak": round(100 * value / PEAK_GBS, 2),
            "timing": "wall clock around graph replays, one graph per decode step (256 GEMMs, 63 of them normalising "
                      "their input rows in their staging, + 1 row normalisation)"}


def run_stack64(torch, qf, dev, args):
    layout = qf.TILED if args.layout == "tiled" else qf.ROWMAJOR
    st = stack64(torch, qf, dev, layout, max(1, args.steps // 50), max(1, args.warmup // 10))
    line = {
        "metric": METRIC, "value": st["GB_s"], "unit": "GB/s", "n_gpus": 1, "steps": st["steps"],
        "warmup": st["warmup"], "ms_per_step": st["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded int8 weights, fp32 scales, bf16 activations)",
        "config": {"workload": "64-layer decode-step linear stack at M=5 (4 GEMMs/layer, distinct weights, "
                               "each layer's input normalised to unit RMS inside its qkv GEMM), one hipGraph per step",
                   "M": st["M"], "layers": st["layers"],
                   "bytes_per_step": st["bytes_per_step"]},
        "us_per_layer": st["us_per_layer"],
        "pct_of_peak": st["pct_peak"],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
