"""Writes the known-answer fixtures in this directory (run: python tests/golden/make_golden.py).

The reference repository ships no golden vectors for its W8A16 path (its only pins are published
error statistics), so these fixtures are computed here, independently of the oracle's C code:

* w8a16_cases.npz -- inputs and expected outputs of y = bf16_rne(s[n] * sum_k x[m,k] w[n,k])
  (plugin/qwen_fastpath/w8a16.py:34-42 with the exact product of bench/test_w8a16.py:15).  The
  expected values are computed with exact rational arithmetic (fractions.Fraction) and rounded to
  bf16 half-to-even by hand; they include a ragged N, every M class, one-hot rows, zero rows and
  the int8 extremes.
* quantize_rows.npz -- the draft-head per-row quantiser (plugin/qwen_fastpath/patches.py:144-146):
  s = max(amax, 1e-8) * fl32(1/127), q = clamp(rint(w / s), -127, 127), with IEEE fp32 numpy
  arithmetic.
* argmax_rows.npz -- the pad-masked draft argmax (patches.py:182-185): columns >= n_valid excluded,
  NaN is the maximum, the first index wins ties, the vocab offset is added.

Inputs are seeded (numpy PCG64) and bf16 values are produced by torch's CPU fp32 -> bf16 cast.
"""
from fractions import Fraction
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def to_bf16_bits(a: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def bf16_bits_to_f64(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def rne_bf16_bits(v: Fraction) -> int:
    """bf16 bit pattern of the rational v rounded to nearest, ties to even (finite range only)."""
    if v == 0:
        return 0
    sign = 0x8000 if v < 0 else 0
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    q_exp = max(e, -126) - 7              # 8 significant bits; subnormals below 2^-126
    q = round(a / Fraction(2) ** q_exp)   # Fraction.__round__: half to even
    if q == 256:                          # rounding carried into the next binade
        q, q_exp = 128, q_exp + 1
    assert q_exp + 7 <= 127, "fixture values stay finite"
    if q < 128:                           # subnormal
        return sign | q
    return sign | ((q_exp + 7 + 127) << 7) | (q - 128)


def w8a16_case(name, M, N, K, rng, special=None):
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    s = (np.abs(rng.standard_normal(N)) * 0.002 + 1e-4).astype(np.float32)
    if special == "edges":
        x[0, :] = 0.0                          # a zero row
        if M > 1:
            x[1, :] = 0.0
            x[1, K // 3] = 1.0                 # one-hot: y = bf16(s * w[:, K/3])
        w[0, :] = 127
        w[1, :] = -128                         # int8 minimum (not produced by the quantiser)
        w[2, ::2] = -127
        s[3] = np.float32(7.5)
        s[4] = np.float32(2.0 ** -20)
    xb = to_bf16_bits(x)
    xf = [[Fraction(float(v)) for v in row] for row in bf16_bits_to_f64(xb)]
    y = np.empty((M, N), dtype=np.uint16)
    y64 = np.empty((M, N), dtype=np.float64)
    for m in range(M):
        for n in range(N):
            acc = sum(xf[m][k] * int(w[n, k]) for k in range(K) if xf[m][k])
            v = acc * Fraction(float(s[n]))
            y[m, n] = rne_bf16_bits(v)
            y64[m, n] = float(v)
    return {f"{name}__x": xb, f"{name}__w": w, f"{name}__s": s, f"{name}__y": y, f"{name}__y64": y64}


def main():
    rng = np.random.default_rng(20260501)
    cases = {}
    specs = [("m1_n16_k64", 1, 16, 64, None), ("m3_n37_k128", 3, 37, 128, None),
             ("m5_n48_k320", 5, 48, 320, "edges"), ("m8_n64_k256", 8, 64, 256, None),
             ("m16_n32_k192", 16, 32, 192, "edges"), ("m5_n100_k512", 5, 100, 512, None)]
    for name, M, N, K, special in specs:
        cases.update(w8a16_case(name, M, N, K, rng, special))
    cases["names"] = np.array([s[0] for s in specs])
    np.savez_compressed(os.path.join(HERE, "w8a16_cases.npz"), **cases)

    # draft-head quantiser
    V, H = 40, 320
    wf = (rng.standard_normal((V, H)) * np.exp2(rng.integers(-8, 4, (V, 1)))).astype(np.float32)
    wf[0] = 0.0                                # amax floor
    wf[1] = 0.25
    wf[1, 5] = -3.0                            # clamps to -127 exactly
    wb = to_bf16_bits(wf)
    vals = bf16_bits_to_f64(wb).astype(np.float32)
    inv = np.float32(1.0) / np.float32(127.0)
    amax = np.maximum(np.abs(vals).max(axis=1), np.float32(1e-8)).astype(np.float32)
    s = (amax * inv).astype(np.float32)
    q = np.clip(np.rint(vals / s[:, None]), -127, 127).astype(np.int8)
    np.savez_compressed(os.path.join(HERE, "quantize_rows.npz"), w=wb, q=q, s=s)

    # pad-masked argmax
    L = rng.standard_normal((6, 300)).astype(np.float32)
    L[0, 10] = L[0, 20] = 50.0                 # tie -> first index
    L[1, 299] = 99.0                           # inside the pad: ignored
    L[2, 7] = np.nan                           # NaN is the maximum
    L[3, :] = -np.inf                          # all -inf -> index 0
    L[4, 295] = 80.0                           # last pad column region
    lb = to_bf16_bits(L)
    n_valid, offset = 296, 1000
    lv = bf16_bits_to_f64(lb)[:, :n_valid]
    ids = []
    for row in lv:
        nan = np.flatnonzero(np.isnan(row))
        ids.append(int(nan[0]) if nan.size else int(np.argmax(row)))
    np.savez_compressed(os.path.join(HERE, "argmax_rows.npz"), logits=lb, n_valid=np.int64(n_valid),
                        offset=np.int64(offset), ids=np.array(ids, dtype=np.int64) + offset)


if __name__ == "__main__":
    main()
