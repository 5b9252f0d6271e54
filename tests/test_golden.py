"""Known-answer fixtures (tests/golden/, written by tests/golden/make_golden.py from exact rational
arithmetic and IEEE fp32 numpy, independently of the oracle's code): the oracle must reproduce them
bit for bit (CPU), and the HIP kernels must meet the tolerance rule against them (GPU)."""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name))


def w8a16_cases():
    d = load("w8a16_cases.npz")
    return [(str(n), d[f"{n}__x"], d[f"{n}__w"], d[f"{n}__s"], d[f"{n}__y"], d[f"{n}__y64"]) for n in d["names"]]


def test_oracle_reproduces_w8a16_fixtures(oracle):
    for name, x, w, s, y, y64 in w8a16_cases():
        bits, ex = oracle.w8a16_exact(x, w, s)
        assert np.array_equal(bits, y), name
        assert np.array_equal(ex, y64), name


def test_oracle_reproduces_quantizer_and_argmax_fixtures(oracle):
    d = load("quantize_rows.npz")
    q, s = oracle.quantize_rows(d["w"])
    assert np.array_equal(q, d["q"]) and np.array_equal(s, d["s"])
    a = load("argmax_rows.npz")
    ids = oracle.argmax_rows(a["logits"], int(a["n_valid"]), int(a["offset"]))
    assert np.array_equal(ids, a["ids"])


@pytest.mark.gpu
def test_kernels_against_w8a16_fixtures(oracle):
    import torch
    import qwen_fastpath as qf
    from helpers import bf16_bits, to_dev_bf16
    dev = torch.device("cuda:0")
    for name, x, w, s, y, y64 in w8a16_cases():
        M, K = x.shape
        N = w.shape[0]
        xd = to_dev_bf16(x, dev)
        wt = torch.from_numpy(w).to(dev).t()
        sd = torch.from_numpy(s).to(dev)
        outs = [qf.w8a16_mm(xd, wt, sd, None, torch.bfloat16, qf.ROWMAJOR),
                qf.w8a16_mm(xd, qf.to_tiled(wt), sd, None, torch.bfloat16, qf.TILED)]
        torch.cuda.synchronize()
        for layout, out in zip(("rowmajor", "tiled"), outs):
            rep = oracle.check_w8a16(bf16_bits(out), x, w, s, exact=(y, y64))
            print(f"golden {name} {layout}: {rep}", flush=True)
            assert rep.ok, (name, layout, rep)
        y32 = qf.w8a16_mm(xd, wt, sd, None, torch.float32, qf.ROWMAJOR)
        torch.cuda.synchronize()
        err = np.abs(y32.cpu().numpy().astype(np.float64) - y64).max() / max(np.sqrt(np.mean(y64 ** 2)), 1e-30)
        assert err <= 1e-5, (name, err)


@pytest.mark.gpu
def test_kernels_against_quantizer_and_argmax_fixtures():
    import torch
    import qwen_fastpath as qf
    dev = torch.device("cuda:0")
    d = load("quantize_rows.npz")
    wd = torch.from_numpy(d["w"].view(np.int16)).to(dev).view(torch.bfloat16)
    q, s = qf.quantize_lm_head(wd)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), d["q"]) and np.array_equal(s.cpu().numpy(), d["s"])
    a = load("argmax_rows.npz")
    logits = torch.from_numpy(a["logits"].view(np.int16)).to(dev).view(torch.bfloat16)
    n_pad = logits.shape[1] - int(a["n_valid"])
    ids = qf.top_tokens(logits, n_pad, int(a["offset"]))
    assert np.array_equal(ids.cpu().numpy(), a["ids"])
