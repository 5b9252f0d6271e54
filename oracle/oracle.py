"""CPU oracle for the W8A16 decode GEMM path.

TEST INFRASTRUCTURE ONLY.  This module is imported by tests/, by ``__graft_entry__.smoke()`` (as the
checker) and by ``bench.py``'s cpu_baseline leg (as the timed CPU reference).  The product package
never imports it and never falls back to it.

What is restated here (reference paths relative to the reference repository):

* ``gen_inputs``             seeded synthetic inputs drawn in the reference's order W -> scales -> x
                             (bench/test_w8a16.py:10-13), with the distributions of the benchmark
                             configurations (int8 uniform in [-127, 127], scales |N(0,1)|*0.002+1e-4,
                             x ~ N(0,1) in bf16) or of the reference's own test (rand*0.01+0.001).
* ``w8a16_exact``            bf16_rne(s[n] * sum_k x[m,k] w[n,k]) with no intermediate rounding
                             (C, 128-bit integers): the closed form of the op
                             (plugin/qwen_fastpath/w8a16.py:34-42, bench/test_w8a16.py:15).
* ``w8a16_f64``              the same product through fp64 BLAS (exact for these inputs, see
                             tests/test_oracle.py), used where the C loop would be slow.
* ``fp32_dequant_linear``    the reference's CPU oracle form F.linear(x.float(), W.float()*ws[:,None])
                             chunked by 8192 rows (bench/test_w8a16.py:15); also the CPU baseline.
* ``w8a16_refkernel``        the reference Triton kernel's fp32 arithmetic for a given
                             (BLOCK_K, SPLIT_K) (plugin/qwen_fastpath/w8a16.py:19-44,83).
* ``ref_pick_config``        the reference's tile table and heuristic (w8a16.py:47-68).
* ``quantize_rows``          the draft-head per-row quantiser (plugin/qwen_fastpath/patches.py:139-147).
* ``argmax_rows``            pad mask + argmax of draft logits (plugin/qwen_fastpath/patches.py:182-185).
* ``check_w8a16``            the tolerance rule for bf16 outputs: elementwise <= 1 bf16 ulp + an
                             fp32-accumulation floor from the exact product, <= 2 bf16 ulp (+ floor)
                             from the reference-kernel arithmetic, at most 2% of outputs off the
                             correctly rounded value, and max|err|/RMS <= 1e-2 beyond the output's
                             own bf16 quantum.
* ``check_w8a16_f32``        max|err|/RMS for fp32 outputs (the 1e-2 bound at fp32 precision).
* ``quantize_tokens``        dynamic symmetric per-token int8 quantisation, the arithmetic of vLLM's
                             scaled_int8_quant(x, symmetric=True) called at plugin/qwen_fastpath/patches.py:99.
* ``w8a8_linear``            that quantisation, exact integer sums with the int8 weights, and the
                             (sum * s_a) * s_w epilogue of cutlass_scaled_mm (patches.py:100): the
                             reference's M > 16 arithmetic.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libqf_oracle.so")
_lib = None


def build() -> str:
    """Compile the C restatement (gcc) into oracle/_build/."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        i32 = ctypes.c_int
        L.qf_oracle_bf16_from_f64.argtypes = [ctypes.c_double]
        L.qf_oracle_bf16_from_f64.restype = ctypes.c_uint16
        L.qf_oracle_bf16_from_f64_array.argtypes = [p, p, i64]
        L.qf_oracle_bf16_from_f64_array.restype = None
        L.qf_oracle_w8a16_exact.argtypes = [p, i64, p, i64, p, p, p, i32, i32, i32]
        L.qf_oracle_w8a16_exact.restype = i32
        L.qf_oracle_w8a16_refkernel.argtypes = [p, i64, p, i64, p, p, p, i32, i32, i32, i32, i32]
        L.qf_oracle_w8a16_refkernel.restype = i32
        L.qf_oracle_quantize_rows.argtypes = [p, i64, p, p, i32, i32]
        L.qf_oracle_quantize_rows.restype = None
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ----------------------------------------------------------------------------------------------
# bf16 helpers
# ----------------------------------------------------------------------------------------------

def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 values (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_from_f64(v: np.ndarray) -> np.ndarray:
    """Round float64 (or float32) values to bf16 bit patterns, nearest-even, in one rounding."""
    v = np.ascontiguousarray(v, dtype=np.float64)
    out = np.empty(v.shape, dtype=np.uint16)
    lib().qf_oracle_bf16_from_f64_array(_ptr(v), _ptr(out), v.size)
    return out


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |v| (2^(floor(log2|v|) - 7), floored at the subnormal quantum)."""
    a = np.abs(np.asarray(v, dtype=np.float64))
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    e = np.maximum(e, -126.0)
    return np.exp2(e - 7.0)


# ----------------------------------------------------------------------------------------------
# inputs
# ----------------------------------------------------------------------------------------------

@dataclass
class Inputs:
    x: np.ndarray      # uint16 bf16 bits [M, K]
    w: np.ndarray      # int8 [N, K] row-major
    s: np.ndarray      # float32 [N]

    @property
    def shape(self):
        return self.x.shape[0], self.w.shape[0], self.w.shape[1]


def gen_inputs(M: int, N: int, K: int, seed: int = 0, dist: str = "baseline") -> Inputs:
    """Seeded inputs, drawn W -> scales -> x (bench/test_w8a16.py:10-13 order).

    dist="baseline":  W int8 uniform in [-127, 127]; s = |N(0,1)| * 0.002 + 1e-4; x bf16 ~ N(0,1).
    dist="reftest":   the reference test's scales s = U[0,1) * 0.01 + 0.001 (bench/test_w8a16.py:11).
    """
    rng = np.random.Generator(np.random.PCG64(seed))
    w = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    if dist == "baseline":
        s = (np.abs(rng.standard_normal(N, dtype=np.float32)) * np.float32(0.002) + np.float32(1e-4)).astype(np.float32)
    elif dist == "reftest":
        s = (rng.random(N, dtype=np.float32) * np.float32(0.01) + np.float32(0.001)).astype(np.float32)
    else:
        raise ValueError(dist)
    x = bf16_from_f64(rng.standard_normal((M, K), dtype=np.float32))
    return Inputs(x=x, w=w, s=s)


# ----------------------------------------------------------------------------------------------
# the product
# ----------------------------------------------------------------------------------------------

def w8a16_exact(x: np.ndarray, w: np.ndarray, s: np.ndarray, with_f64: bool = True):
    """Exact, correctly rounded product.  Returns (bf16 bits [M,N], fp64 [M,N] or None).

    Raises ValueError when a row's exponent range exceeds the 128-bit accumulator (or holds
    inf/nan): such inputs are outside what this oracle pins.
    """
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.int8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    M, K = x.shape
    N = w.shape[0]
    assert w.shape[1] == K and s.shape == (N,)
    y = np.empty((M, N), dtype=np.uint16)
    y64 = np.empty((M, N), dtype=np.float64) if with_f64 else None
    rc = lib().qf_oracle_w8a16_exact(_ptr(x), K, _ptr(w), K, _ptr(s), _ptr(y),
                                     _ptr(y64) if with_f64 else None, M, N, K)
    if rc != 0:
        raise ValueError(f"row {rc - 1}: exponent range outside the exact oracle's accumulator")
    return y, y64


def w8a16_f64(x: np.ndarray, w: np.ndarray, s: np.ndarray, chunk: int = 8192) -> np.ndarray:
    """s[n] * sum_k x w in fp64 through BLAS (chunked over N).  Exact before the final multiply for
    inputs whose per-row exponent range keeps partial sums within 53 bits."""
    xf = bf16_to_f32(x).astype(np.float64)
    N = w.shape[0]
    out = np.empty((x.shape[0], N), dtype=np.float64)
    for i in range(0, N, chunk):
        out[:, i:i + chunk] = (xf @ w[i:i + chunk].astype(np.float64).T) * s[i:i + chunk].astype(np.float64)
    return out


def fp32_dequant_linear(x: np.ndarray, w: np.ndarray, s: np.ndarray, chunk: int = 8192) -> np.ndarray:
    """The reference's oracle form (bench/test_w8a16.py:15): F.linear(x.float(), W.float()*ws[:,None]),
    fp32, chunked over N by 8192 rows.  Returns float32 [M, N]."""
    xf = bf16_to_f32(x)
    N = w.shape[0]
    out = np.empty((x.shape[0], N), dtype=np.float32)
    for i in range(0, N, chunk):
        wd = w[i:i + chunk].astype(np.float32) * s[i:i + chunk, None]
        out[:, i:i + chunk] = xf @ wd.T
    return out


def w8a16_refkernel(x: np.ndarray, w: np.ndarray, s: np.ndarray, block_k: int, split_k: int):
    """Reference Triton kernel arithmetic (w8a16.py:19-44,83).  Returns (bf16 bits, fp32)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.int8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), dtype=np.uint16)
    y32 = np.empty((M, N), dtype=np.float32)
    rc = lib().qf_oracle_w8a16_refkernel(_ptr(x), K, _ptr(w), K, _ptr(s), _ptr(y), _ptr(y32), M, N, K,
                                         block_k, split_k)
    if rc != 0:
        raise ValueError("K must be a multiple of BLOCK_K * SPLIT_K (the reference kernel has no K mask)")
    return y, y32


# The reference's per-shape table and heuristic (plugin/qwen_fastpath/w8a16.py:47-68).
# (BLOCK_M, BLOCK_N, BLOCK_K, SPLIT_K, num_warps, num_stages), keyed by (N, K).
REF_TUNED = {
    (34816, 5120): (16, 32, 256, 1, 4, 3),
    (5120, 17408): (16, 32, 256, 2, 4, 3),
    (16384, 5120): (16, 32, 128, 1, 4, 4),
    (5120, 6144): (16, 64, 128, 4, 4, 3),
    (14336, 5120): (16, 32, 128, 4, 4, 4),
    (248320, 5120): (16, 64, 256, 1, 8, 3),
}


def ref_pick_config(N: int, K: int):
    cfg = REF_TUNED.get((N, K))
    if cfg is not None:
        return cfg
    sk = 1 if N >= 8192 else (4 if N >= 1024 else 8)
    for bk in (256, 128, 64):
        while sk > 1 and K % (bk * sk):
            sk //= 2
        if K % (bk * sk) == 0:
            return (16, 32, bk, sk, 4, 3)
    return None


# ----------------------------------------------------------------------------------------------
# W8A8: the reference's M > 16 fallback (scaled_int8_quant + cutlass_scaled_mm)
# ----------------------------------------------------------------------------------------------

def quantize_tokens(x_bits: np.ndarray):
    """Per-token symmetric int8 quantisation of bf16 bits [M, K] (vLLM scaled_int8_quant, symmetric,
    patches.py:99): s_a = amax_k |x| * fl32(1/127) in fp32 (how `amax / 127.0` evaluates on the device;
    vLLM's own kernel divides, at most one ulp apart), q = clamp(round_half_even(x / s_a), -128, 127)
    with an IEEE fp32 division; a row of zeros gets s_a = 0 and q = 0.  Returns (q int8, s_a fp32)."""
    xf = bf16_to_f32(np.ascontiguousarray(x_bits, dtype=np.uint16))
    amax = np.abs(xf).max(axis=1).astype(np.float32)
    r = np.float32(1.0) / np.float32(127.0)
    s_a = (amax * r).astype(np.float32)
    safe = np.where(s_a > 0, s_a, np.float32(1.0)).astype(np.float32)
    q = np.rint(xf / safe[:, None])
    q = np.where(s_a[:, None] > 0, q, np.float32(0.0))
    return np.clip(q, -128, 127).astype(np.int8), s_a


def w8a8_linear(x_bits: np.ndarray, w: np.ndarray, s_w: np.ndarray, out_f32: bool = False):
    """y[m, n] = ((fp32(sum_k q[m,k] w[n,k]) * s_a[m]) * s_w[n]) in fp32, rounded to bf16 bits unless
    out_f32: the reference's M > 16 arithmetic (scaled_int8_quant + cutlass_scaled_mm,
    patches.py:99-100).  The integer sums are exact (fp64 sums of |terms| <= 2^14, far below 2^53) and
    are rounded once to fp32."""
    q, s_a = quantize_tokens(x_bits)
    acc = (q.astype(np.float64) @ np.asarray(w, dtype=np.int8).astype(np.float64).T).astype(np.float32)
    y = (acc * s_a[:, None]) * np.asarray(s_w, dtype=np.float32)[None, :]
    return y if out_f32 else bf16_from_f64(y.astype(np.float64))


# ----------------------------------------------------------------------------------------------
# draft head
# ----------------------------------------------------------------------------------------------

def quantize_rows(wbf: np.ndarray):
    """Per-row int8 quantisation of bf16 bits [V, H] (patches.py:139-147).  Returns (q int8, s fp32)."""
    wbf = np.ascontiguousarray(wbf, dtype=np.uint16)
    V, H = wbf.shape
    q = np.empty((V, H), dtype=np.int8)
    s = np.empty((V,), dtype=np.float32)
    lib().qf_oracle_quantize_rows(_ptr(wbf), H, _ptr(q), _ptr(s), V, H)
    return q, s


def argmax_rows(logits_bits: np.ndarray, n_valid: int, index_offset: int = 0) -> np.ndarray:
    """Columns >= n_valid set to -inf, then torch.argmax semantics (NaN is the max, first index wins).
    (plugin/qwen_fastpath/patches.py:182-185)"""
    v = bf16_to_f32(logits_bits).astype(np.float64).copy()
    v[:, n_valid:] = -np.inf
    out = np.empty(v.shape[0], dtype=np.int64)
    for m in range(v.shape[0]):
        row = v[m]
        nan = np.isnan(row)
        out[m] = int(np.argmax(nan)) if nan.any() else int(np.argmax(row))
    return out + index_offset


# ----------------------------------------------------------------------------------------------
# tolerance
# ----------------------------------------------------------------------------------------------

# Elementwise absolute floor: fp32 accumulation error over K terms is bounded by ~K * 2^-24 *
# sum|x w| in the worst case; 2^-20 * s * sum|x w| covers any summation order for K <= 2^16 on
# these inputs with margin (random-sign sums grow like sqrt(K)).
ACC_FLOOR = 2.0 ** -20
REL_MAX_TOL = 1e-2       # max|err| / RMS(out), the stated bound
ULP_TOL_EXACT = 1.0      # ulps from the correctly rounded exact product
ULP_TOL_REFKERNEL = 2.0  # ulps from the reference kernel's arithmetic
# Share of outputs allowed to differ from the correctly rounded exact value.  fp32 accumulation moves
# a result across a bf16 rounding boundary only when the exact value lies within the accumulation
# error of a tie (~0.02% of outputs at K=5120); a kernel that truncates or rounds its accumulator
# early differs on ~half of them.
DIFF_FRAC_TOL = 0.02


def abs_sum(x: np.ndarray, w: np.ndarray, s: np.ndarray) -> np.ndarray:
    """s[n] * sum_k |x[m,k] w[n,k]| in fp64 (the scale of fp32 accumulation error)."""
    xa = np.abs(bf16_to_f32(x).astype(np.float64))
    out = np.empty((x.shape[0], w.shape[0]))
    for i in range(0, w.shape[0], 8192):
        out[:, i:i + 8192] = (xa @ np.abs(w[i:i + 8192].astype(np.float64)).T) * np.abs(s[i:i + 8192].astype(np.float64))
    return out


@dataclass
class Report:
    ok: bool
    rel_excess: float       # max(|y - exact| - ulp(exact), 0) / RMS: the 1e-2 bound beyond the output quantum
    rel_max: float          # max|y - bf16(exact)| / RMS(exact)   (informational: one ulp flip at an
    #                         output of 1.3x RMS already exceeds 1e-2)
    rel_max_f32: float      # max|y - exact| / RMS(exact): the bound read literally against the unrounded
    #                         fp32-dequant result (informational: bf16 output rounding alone gives ~2e-2)
    rel_l2: float           # ||y - exact|| / ||exact||  (the reference's published metric, 0.0016-0.0017)
    max_ulp_exact: float    # max over elements of |y - bf16(exact)| / ulp(exact)  (floor excluded)
    n_over_exact: int       # elements beyond 1 ulp + floor of the exact value
    n_over_ref: int         # elements beyond 2 ulp + floor of the reference-kernel value (-1: n/a)
    n_diff_exact: int       # elements not equal to the correctly rounded exact value

    def __str__(self):
        return (f"ok={self.ok} rel_excess={self.rel_excess:.2e} rel_max={self.rel_max:.2e} "
                f"rel_max_f32={self.rel_max_f32:.2e} rel_l2={self.rel_l2:.3e} max_ulp={self.max_ulp_exact:.2f} "
                f"over_exact={self.n_over_exact} over_ref={self.n_over_ref} diff={self.n_diff_exact}")


def check_w8a16(y_bits: np.ndarray, x: np.ndarray, w: np.ndarray, s: np.ndarray,
                exact=None, ref_bits: np.ndarray | None = None) -> Report:
    """Apply the tolerance rule to a bf16 result y_bits [M, N].  Passes when
      (1) every output is within 1 bf16 ulp (+ the fp32-accumulation floor) of the exact product,
      (2) every output is within 2 bf16 ulp (+ floor) of the reference-kernel arithmetic (if given),
      (3) at most DIFF_FRAC_TOL of outputs differ from the correctly rounded exact value,
      (4) max(|y - exact| - ulp(exact), 0) / RMS(exact) <= 1e-2.

    exact: optional precomputed (bf16 bits, fp64) from w8a16_exact (or w8a16_f64 + bf16_from_f64).
    ref_bits: optional reference-kernel result (w8a16_refkernel) for (2).
    """
    if exact is None:
        exact = w8a16_exact(x, w, s)
    e_bits, e64 = exact
    y = bf16_to_f32(y_bits).astype(np.float64)
    eb = bf16_to_f32(e_bits).astype(np.float64)
    rms = float(np.sqrt(np.mean(e64 ** 2))) if e64.size else 0.0
    rms = rms if rms > 0 else 1.0
    err = np.abs(y - eb)
    err64 = np.abs(y - e64)
    floor = ACC_FLOOR * abs_sum(x, w, s)
    ulp = bf16_ulp(e64)
    rel_excess = float(np.maximum(err64 - ulp, 0.0).max() / rms) if err.size else 0.0
    rel_max = float(err.max() / rms) if err.size else 0.0
    rel_max_f32 = float(err64.max() / rms) if err.size else 0.0
    denom = float(np.linalg.norm(e64))
    rel_l2 = float(np.linalg.norm(y - e64) / denom) if denom > 0 else 0.0
    over_exact = int(np.count_nonzero(err > ULP_TOL_EXACT * ulp + floor))
    max_ulp = float((err / ulp).max()) if err.size else 0.0
    n_over_ref = -1
    if ref_bits is not None:
        rb = bf16_to_f32(ref_bits).astype(np.float64)
        n_over_ref = int(np.count_nonzero(np.abs(y - rb) > ULP_TOL_REFKERNEL * bf16_ulp(rb) + floor))
    n_diff = int(np.count_nonzero(err))
    ok = (over_exact == 0 and n_over_ref <= 0 and n_diff <= max(8, DIFF_FRAC_TOL * err.size)
          and rel_excess <= REL_MAX_TOL)
    return Report(ok=ok, rel_excess=rel_excess, rel_max=rel_max, rel_max_f32=rel_max_f32, rel_l2=rel_l2,
                  max_ulp_exact=max_ulp, n_over_exact=over_exact, n_over_ref=n_over_ref, n_diff_exact=n_diff)


def check_w8a16_f32(y32: np.ndarray, x: np.ndarray, w: np.ndarray, s: np.ndarray, exact=None) -> float:
    """max|y - exact| / RMS(exact) for an fp32 result (the op run with an fp32 output): the 1e-2
    bound against the reference's fp32-dequant form, at the precision that form produces."""
    if exact is None:
        exact = w8a16_exact(x, w, s)
    e64 = exact[1]
    rms = float(np.sqrt(np.mean(e64 ** 2))) or 1.0
    return float(np.abs(np.asarray(y32, dtype=np.float64) - e64).max() / rms)
