/*
 * qf_oracle.c — CPU restatement of the W8A16 decode GEMM path, used only as a checker.
 *
 * TEST INFRASTRUCTURE.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only to check or time the reference algorithm; the product never calls it.
 *
 * Functions (reference paths relative to the reference repository):
 *   qf_oracle_bf16_from_f64     round-to-nearest-even fp64 -> bf16 (the final .to(bfloat16) of
 *                               plugin/qwen_fastpath/w8a16.py:42,83 applied to an exact value)
 *   qf_oracle_w8a16_exact       bf16_rne( s[n] * sum_k x[m,k] w[n,k] ) computed with 128-bit
 *                               integers: no intermediate rounding at all (the closed form of
 *                               bench/test_w8a16.py:15 and plugin/qwen_fastpath/w8a16.py:34-42)
 *   qf_oracle_w8a16_refkernel   the reference Triton kernel's fp32 arithmetic, w8a16.py:19-44,83:
 *                               split j walks BLOCK_K chunks j, j+SK, ...; fp32 accumulation per
 *                               16-wide MMA k-block; scale per split; split sum in fp32; RNE
 *   qf_oracle_quantize_rows     draft-head quantiser, plugin/qwen_fastpath/patches.py:139-147
 *
 * Build: oracle/Makefile (gcc, no fast-math: IEEE division and rint are relied upon).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef __int128 i128;
typedef unsigned __int128 u128;

/* ---------------------------------------------------------------------------------------------
 * bf16 rounding
 * ------------------------------------------------------------------------------------------- */

static uint16_t bf16_special(double v) {
  if (v != v) return 0x7FC0;
  return (v > 0) ? 0x7F80 : 0xFF80;
}

/* Round mag * 2^e2 (mag > 0 an exact integer, `sticky` = some nonzero value lies below mag's last
 * bit) to bf16 with round-to-nearest-even; returns the magnitude bits (no sign). */
static uint16_t round_mag_to_bf16(u128 mag, int e2, int sticky) {
  if (mag == 0) return 0; /* sticky-only values are far below the smallest subnormal here */
  int L = 0;
  for (u128 t = mag; t; t >>= 1) ++L;  /* bit length */
  const int E = L - 1 + e2;            /* exponent of the leading bit */
  int q_exp2;                          /* exponent of the quantum */
  if (E >= -126) q_exp2 = E - 7;       /* normal: 8 significant bits */
  else q_exp2 = -133;                  /* subnormal quantum 2^-133 */
  const int sh = q_exp2 - e2;          /* bits of mag below the quantum */
  u128 q;
  if (sh <= 0) {
    q = mag << (-sh);                  /* exact, fits: q < 2^8 */
  } else if (sh >= 128) {
    q = 0;                             /* below half a quantum */
  } else {
    q = mag >> sh;
    const u128 rem = mag & ((((u128)1) << sh) - 1);
    const u128 half = ((u128)1) << (sh - 1);
    if (rem > half || (rem == half && (sticky || (q & 1)))) q += 1; /* ties to even */
  }
  /* q is the significand in units of 2^q_exp2 */
  if (q_exp2 == -133 && E < -126) {
    if (q >= 128) return 0x0080;       /* rounded up to the smallest normal */
    return (uint16_t)q;
  }
  int ef = q_exp2 + 7 + 127;           /* exponent field of a normal result */
  if (q >= 256) { q >>= 1; ef += 1; }
  if (ef >= 255) return 0x7F80;
  return (uint16_t)((ef << 7) | (int)(q - 128));
}

uint16_t qf_oracle_bf16_from_f64(double v) {
  if (isnan(v) || isinf(v)) return bf16_special(v);
  if (v == 0) return signbit(v) ? 0x8000 : 0x0000;
  const uint16_t sign = signbit(v) ? 0x8000 : 0;
  int e;
  const double m = frexp(fabs(v), &e); /* |v| = m 2^e, m in [0.5, 1) */
  const u128 mag = (u128)(uint64_t)ldexp(m, 53);  /* exact 53-bit integer */
  return (uint16_t)(sign | round_mag_to_bf16(mag, e - 53, 0));
}

void qf_oracle_bf16_from_f64_array(const double* v, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = qf_oracle_bf16_from_f64(v[i]);
}

/* ---------------------------------------------------------------------------------------------
 * exact product
 * ------------------------------------------------------------------------------------------- */

/* bf16 bits -> (signed integer significand, exponent) with value = sig * 2^ex.  Returns 0 for
 * inf/nan (not representable exactly as an integer). */
static int bf16_decompose(uint16_t b, int32_t* sig, int* ex) {
  const int sign = b >> 15;
  const int ef = (b >> 7) & 0xFF;
  const int mant = b & 0x7F;
  if (ef == 0xFF) return 0;
  int32_t s;
  if (ef == 0) { s = mant; *ex = -133; }
  else { s = 128 + mant; *ex = ef - 127 - 7; }
  *sig = sign ? -s : s;
  return 1;
}

/* y[m,n] = bf16_rne(s[n] * sum_k x[m,k] * w[n,k]) exactly.  x: bf16 bits [M, ldx], w: int8 [N, ldw],
 * s: fp32 [N].  Optional y64 receives the fp64 rounding of the same exact value.  Returns 0 on
 * success, or 1 + m for the first row whose exponent range does not fit the 128-bit accumulator
 * (or holds inf/nan), in which case nothing is written for that row. */
int qf_oracle_w8a16_exact(const uint16_t* x, int64_t ldx, const int8_t* w, int64_t ldw, const float* s,
                          uint16_t* y, double* y64, int M, int N, int K) {
  i128* xs = (i128*)malloc(sizeof(i128) * (size_t)K);
  int32_t* sig = (int32_t*)malloc(sizeof(int32_t) * (size_t)K);
  int* ex = (int*)malloc(sizeof(int) * (size_t)K);
  int status = 0;
  int kbits = 0;
  while ((1LL << kbits) < (int64_t)K) ++kbits;
  for (int m = 0; m < M && status == 0; ++m) {
    int emin = 1 << 30, emax = -(1 << 30);
    for (int k = 0; k < K; ++k) {
      if (!bf16_decompose(x[m * ldx + k], &sig[k], &ex[k])) { status = 1 + m; break; }
      if (sig[k] != 0) { if (ex[k] < emin) emin = ex[k]; if (ex[k] > emax) emax = ex[k]; }
    }
    if (status) break;
    if (emin > emax) emin = emax = 0; /* all zeros */
    /* |term| < 2^(emax-emin) * 2^8 * 2^7; sum of K terms adds kbits; keep below 2^126 */
    if ((emax - emin) + 8 + 7 + kbits > 125) { status = 1 + m; break; }
    for (int k = 0; k < K; ++k) xs[k] = (i128)sig[k] << (ex[k] - emin);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n) {
      const int8_t* wr = w + (int64_t)n * ldw;
      i128 acc = 0;
      for (int k = 0; k < K; ++k) acc += xs[k] * (i128)wr[k];
      /* value = acc * 2^emin * s[n] */
      const float sf = s[n];
      uint16_t out;
      double out64;
      if (acc == 0 || sf == 0.0f) {
        /* an exact zero: IEEE sign of the product (sum +0 when acc == 0) */
        const int neg = (acc < 0) != (signbit(sf) != 0);
        out = neg ? 0x8000 : 0;
        out64 = neg ? -0.0 : 0.0;
      } else if (isnan(sf) || isinf(sf)) {
        const double v = (double)sf * (acc < 0 ? -1.0 : 1.0);
        out = bf16_special(v); out64 = v;
      } else {
        int es;
        const float ms = frexpf(fabsf(sf), &es);         /* |s| = ms 2^es */
        const u128 S = (u128)(uint32_t)ldexpf(ms, 24);    /* exact 24-bit */
        const int e_s = es - 24;
        const int neg = (acc < 0) != (sf < 0);
        u128 A = (u128)(acc < 0 ? -acc : acc);
        int L = 0;
        for (u128 t = A; t; t >>= 1) ++L;
        int shift = 0, sticky = 0;
        if (L > 100) {
          shift = L - 100;
          sticky = (A & ((((u128)1) << shift) - 1)) != 0;
          A >>= shift;
        }
        const u128 P = A * S;                             /* < 2^124 */
        const int e2 = shift + emin + e_s;
        out = (uint16_t)((neg ? 0x8000 : 0) | round_mag_to_bf16(P, e2, sticky));
        /* fp64 rounding of the same value (used for error norms) */
        out64 = ldexp((double)P, e2) * (neg ? -1.0 : 1.0);
      }
      y[(int64_t)m * N + n] = out;
      if (y64) y64[(int64_t)m * N + n] = out64;
    }
  }
  free(xs); free(sig); free(ex);
  return status;
}

/* ---------------------------------------------------------------------------------------------
 * reference-kernel arithmetic (plugin/qwen_fastpath/w8a16.py:19-44,83)
 * ------------------------------------------------------------------------------------------- */

static float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* fp32 -> bf16 RNE (torch .to(bfloat16) on a finite fp32) */
static uint16_t f32_to_bf16_rne(float f) { return qf_oracle_bf16_from_f64((double)f); }

/* Returns 0, or 1 when K % (bk * sk) != 0 (the reference kernel has no K mask, w8a16.py:28). */
int qf_oracle_w8a16_refkernel(const uint16_t* x, int64_t ldx, const int8_t* w, int64_t ldw, const float* s,
                              uint16_t* y, float* y32, int M, int N, int K, int bk, int sk) {
  if (bk <= 0 || sk <= 0 || K % (bk * sk) != 0 || bk % 16 != 0) return 1;
  const int iters = K / (bk * sk);
  for (int m = 0; m < M; ++m) {
    const uint16_t* xr = x + (int64_t)m * ldx;
    for (int n = 0; n < N; ++n) {
      const int8_t* wr = w + (int64_t)n * ldw;
      float total = 0.0f;
      for (int j = 0; j < sk; ++j) {
        float acc = 0.0f;
        for (int it = 0; it < iters; ++it) {
          const int k0 = (it * sk + j) * bk; /* rk = pid_k*BK + it*BK*SK */
          for (int kb = k0; kb < k0 + bk; kb += 16) {
            double blk = 0.0; /* 16 products of <= 15-bit significands: exact in fp64 */
            for (int k = kb; k < kb + 16; ++k) blk += (double)bf16_to_f32(xr[k]) * (double)wr[k];
            acc = acc + (float)blk;
          }
        }
        acc = acc * s[n];
        if (sk == 1) total = acc;
        else total = total + acc; /* atomic_add order fixed to ascending split */
      }
      if (y) y[(int64_t)m * N + n] = f32_to_bf16_rne(total);
      if (y32) y32[(int64_t)m * N + n] = total;
    }
  }
  return 0;
}

/* ---------------------------------------------------------------------------------------------
 * draft-head quantiser (plugin/qwen_fastpath/patches.py:139-147)
 *   s = amax|row|.clamp(min=1e-8) / 127.0   -> a CUDA tensor divided by a Python scalar, which
 *                                              PyTorch evaluates as a multiply by fl32(1/127)
 *   q = round(row / s).clamp(-127, 127)     -> IEEE fp32 division, round half to even
 * ------------------------------------------------------------------------------------------- */
void qf_oracle_quantize_rows(const uint16_t* wbf, int64_t ldw, int8_t* q, float* s, int V, int H) {
  const float inv127 = 1.0f / 127.0f;
  for (int v = 0; v < V; ++v) {
    const uint16_t* row = wbf + (int64_t)v * ldw;
    float amax = 0.0f;
    for (int h = 0; h < H; ++h) { const float a = fabsf(bf16_to_f32(row[h])); if (a > amax) amax = a; }
    if (amax < 1e-8f) amax = 1e-8f;
    const float sv = amax * inv127;
    s[v] = sv;
    for (int h = 0; h < H; ++h) {
      float t = rintf(bf16_to_f32(row[h]) / sv);
      if (t > 127.0f) t = 127.0f;
      if (t < -127.0f) t = -127.0f;
      q[(int64_t)v * H + h] = (int8_t)(int)t;
    }
  }
}
