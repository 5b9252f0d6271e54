// qf_w8a16.hip — gfx950 (MI355X) kernels and C ABI of the W8A16 decode GEMM.
//
//   y[m, n] = bf16_rne( s[n] * sum_k x[m, k] * w[n, k] ),   x bf16 [M, K], w int8 [N, K], s fp32 [N]
//
// The arithmetic follows the reference Triton kernel (plugin/qwen_fastpath/w8a16.py:15-44): int8
// weights are widened to bf16 exactly (|w| <= 128 needs 8 significant bits), products are
// accumulated in fp32, the per-channel scale is applied once after the K reduction, and the result
// is rounded to bf16 with round-to-nearest-even.  Where the reference reduces split-K partials with
// fp32 atomics (w8a16.py:43-44, order-dependent), this file writes the partials to a workspace and
// sums them in split order -- in the last workgroup of each n-block to finish, or in a second
// kernel -- so every result is bitwise reproducible.
//
// Two kernels compute the product:
//   * mfma: v_mfma_f32_16x16x32_bf16 over 1 KiB weight fragments (16 output channels x 64 k).  The
//     weight fragment is the A operand (rows = output channels), the activation fragment the B
//     operand (columns = tokens, padded to 16), so one lane ends with 4 consecutive output
//     channels of one token and stores them as one 8-byte write.  Serves M = 1..16.
//   * gemv: wavefront reduction.  Each wavefront streams RPW weight rows with 16 bytes per lane
//     (1 KiB per row per step), multiplies on the VALU in fp32 and reduces across the 64 lanes at
//     the end.  Serves M = 1..4 on the row-major layout.
// Both stage the workgroup's slice of x in LDS once and read it from there; weights are loaded
// with 128-bit global loads, dequantised in registers and never written anywhere.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <mutex>
#include <unordered_set>

#include "qf_w8a16.h"

namespace qf {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr int kTileN = 16;     // output channels per MFMA tile
constexpr int kStepK = 64;     // k covered by one 16-byte-per-lane weight fragment of a tile
constexpr int kXcds = 8;       // accelerator complexes (XCDs) of an MI355X

// The hardware hands workgroup i of a launch to XCD i % kXcds.  xcd_major(i, total) renumbers the
// workgroups XCD by XCD: the workgroups of one XCD (i, i + kXcds, i + 2 kXcds, ...) get consecutive
// indices, XCD 0's first.  A bijection of [0, total) for any total.
__device__ __forceinline__ int xcd_major(int i, int total) {
  const int xcd = i % kXcds, j = i / kXcds;
  const int per = total / kXcds, rem = total % kXcds;
  return xcd < rem ? xcd * (per + 1) + j : rem * (per + 1) + (xcd - rem) * per + j;
}
constexpr size_t kLdsPerWorkgroup = 160 * 1024;     // gfx950 LDS per workgroup
constexpr size_t kMaxLds = kLdsPerWorkgroup - 256;  // the dynamic budget; static __shared__ uses the rest
constexpr size_t kDefaultLds = 64 * 1024;           // above this a kernel needs the dynamic-LDS attribute raised

struct GemmArgs {
  const uint16_t* x;
  const int8_t* w;
  const float* scale;
  void* y;
  float* partial;      // [split_k][M][n_pad] fp32 when split_k > 1
  unsigned* counters;  // arrival counters (split_k > 1), counter_stride words apart: zero on entry and on exit
  int counter_stride;
  int64_t ldx;
  int64_t ldw;
  int64_t ldy;
  int M, N, K;
  int n_pad;       // N rounded up to a multiple of 16
  int ksteps;      // K / 64
  int split_k;
  int out_f32;
  int vec_out;     // rows of y are 8-byte (bf16) / 16-byte (fp32) aligned: vector stores allowed
  int fused_reduce;  // MFMA, split_k > 1: the last workgroup of an n-block reduces (else a second kernel)
  // Fused argmax (MFMA, split_k == 1): ids[m] = index_offset + argmax over n < n_valid of the bf16
  // outputs y[m, n] (NaN highest, then value, then the lowest index); y may be null.  Each wavefront
  // column folds its candidate per token into one of the token's kArgmaxSlots slots (a 64-bit atomic
  // maximum of argmax_key); argmax_slots_kernel folds the slots into ids and clears them.
  int argmax;
  int n_valid;
  int64_t index_offset;
  int64_t* ids;
  uint64_t* am_slots;
  // Wide-M kernel: token groups per n-block and rows per group (a multiple of 16; the last group
  // takes the rest, at least one row).
  int groups;
  int group_rows;
  // W8A8 kernel: int8 activations [M][K] (row stride ldx bytes) and their per-token scales.
  const int8_t* xq;
  const float* s_tok;
  // W8A8 kernel: xq is the token-tiled image instead (the TILED weight layout applied to [M][K]: block
  // (b, s) of tokens 16 b .. 16 b + 15 and k 64 s .. 64 s + 63 at byte (b * ksteps + s) * 1024, lane
  // (g, r) = token 16 b + r, k 64 s + 16 g .. + 15 at byte 16 (16 g + r) of the block).
  int x_tiled;
  // Stream kernel: 1 = workgroup b owns tiles b, b + G, b + 2 G, ... (G = grid) instead of a contiguous run.
  int tiles_strided;
  // Kernels instantiated with NORM: the staged x rows are first scaled to unit RMS (qf_w8a16_gemm_rmsnorm).
  float norm_eps;
};

// ---------------------------------------------------------------------------------------------
// small device helpers
// ---------------------------------------------------------------------------------------------

// Upper halves of two fp32 patterns -> one dword of two bf16 (lo in bits 0..15).  Exact when the
// low 16 bits are zero, which holds for every integer of magnitude <= 256.
__device__ __forceinline__ uint32_t pack_upper16(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// 4 int8 (one dword, little endian) -> 4 bf16 in two dwords.  Each byte is sign-extended and
// converted by one v_cvt_f32_i32 with a byte-select source operand.
__device__ __forceinline__ void i8x4_to_bf16x4(uint32_t d, uint32_t& lo, uint32_t& hi) {
  const int32_t s = (int32_t)d;
  const float f0 = (float)(int8_t)(s & 0xff);
  const float f1 = (float)(int8_t)((s >> 8) & 0xff);
  const float f2 = (float)(int8_t)((s >> 16) & 0xff);
  const float f3 = (float)(s >> 24);
  lo = pack_upper16(f0, f1);
  hi = pack_upper16(f2, f3);
}

// 16 int8 weights (k..k+15 of one row) -> two bf16x8 MFMA operands (k..k+7, k+8..k+15).
__device__ __forceinline__ void dequant16(const u32x4_t v, bf16x8_t& a0, bf16x8_t& a1) {
  u32x4_t o0, o1;
  uint32_t t0, t1;
  i8x4_to_bf16x4(v.x, t0, t1); o0.x = t0; o0.y = t1;
  i8x4_to_bf16x4(v.y, t0, t1); o0.z = t0; o0.w = t1;
  i8x4_to_bf16x4(v.z, t0, t1); o1.x = t0; o1.y = t1;
  i8x4_to_bf16x4(v.w, t0, t1); o1.z = t0; o1.w = t1;
  a0 = __builtin_bit_cast(bf16x8_t, o0);
  a1 = __builtin_bit_cast(bf16x8_t, o1);
}

// Two fp32 -> two bf16 (round to nearest even) packed in a dword.
__device__ __forceinline__ uint32_t pack_bf16_rne(float a, float b) {
  bf16x2_t v;
  v.x = (__bf16)a;
  v.y = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint16_t bf16_rne(float a) {
  return __builtin_bit_cast(uint16_t, (__bf16)a);
}

template <bool kNonTemporal>
__device__ __forceinline__ u32x4_t load16(const int8_t* p) {
  const u32x4_t* q = reinterpret_cast<const u32x4_t*>(p);
  if constexpr (kNonTemporal) {
    return __builtin_nontemporal_load(q);
  } else {
    return *q;
  }
}

// Store 4 consecutive outputs n..n+3 of one token row; `cnt` < 4 only at a ragged N tail.  Without
// `vec` (a row stride that breaks vector alignment) every element is stored on its own.
__device__ __forceinline__ void store_out4(void* y, int64_t ldy, int out_f32, int vec, int m, int n, int cnt,
                                           f32x4_t v) {
  const bool full = vec && cnt == 4;
  if (out_f32) {
    float* row = reinterpret_cast<float*>(y) + (int64_t)m * ldy + n;
    if (full) {
      *reinterpret_cast<f32x4_t*>(row) = v;
    } else {
      for (int i = 0; i < cnt; ++i) row[i] = v[i];
    }
  } else {
    uint16_t* row = reinterpret_cast<uint16_t*>(y) + (int64_t)m * ldy + n;
    if (full) {
      u32x2_t p;
      p.x = pack_bf16_rne(v.x, v.y);
      p.y = pack_bf16_rne(v.z, v.w);
      *reinterpret_cast<u32x2_t*>(row) = p;
    } else {
      for (int i = 0; i < cnt; ++i) row[i] = bf16_rne(v[i]);
    }
  }
}

__device__ __forceinline__ f32x4_t load_scale4(const float* scale, int N, int n) {
  f32x4_t s = {0.f, 0.f, 0.f, 0.f};
  if (n + 4 <= N) {
    s = *reinterpret_cast<const f32x4_t*>(scale + n);
  } else {
    for (int i = 0; i < 4; ++i)
      if (n + i < N) s[i] = scale[n + i];
  }
  return s;
}

// Candidate order of the argmax: NaN is the maximum, then the larger value, then the lower index.
__device__ __forceinline__ bool argmax_better(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an != bn) return an;
  if (an) return ai < bi;
  if (av != bv) return av > bv;
  return ai < bi;
}

// Better of two (value, index) candidates, folded into (bv, bi).
__device__ __forceinline__ void argmax_fold(float v, int i, float& bv, int& bi) {
  if (argmax_better(v, i, bv, bi)) {
    bv = v;
    bi = i;
  }
}

// Slots of the fused argmax per token, spread over the workspace's counter prefix: wavefront column c of the GEMM
// folds into slot c % kArgmaxSlots of its token, slot (m, s) at 64-bit word (s * M + m) * stride, the stride the
// largest power of two that fits (64 bytes at M = 16), so the atomics on any one address and any one memory
// channel stay few (one slot per token serialised 9496 of them on the draft head: 155 against 122 us a step).
constexpr int kArgmaxSlots = 64;
__host__ __device__ __forceinline__ int argmax_slot_stride(int M) {
  int st = QF_W8A16_COUNTER_BYTES / 8 / (kArgmaxSlots * M);
  while (st & (st - 1)) st &= st - 1;
  return st;
}
static_assert(QF_W8A16_COUNTER_BYTES / 8 / (kArgmaxSlots * QF_W8A16_MAX_M) >= 8, "slots on separate 64-byte lines");

// A 64-bit key that orders candidates as argmax_better does: the larger key is the better candidate (NaN
// highest, then the larger value, -0 ranking with +0, then the lower index), and 0 is below every key.
__device__ __forceinline__ uint64_t argmax_key(float v, int i) {
  const uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);
  const uint32_t k = v != v ? 0xffffffffu : ((u >> 31) ? ~u : (u | 0x80000000u));
  return ((uint64_t)k << 32) | (uint64_t)(~(uint32_t)i);
}

// s_waitcnt immediate (gfx9 encoding) that waits for vmcnt == 0 and leaves expcnt / lgkmcnt free.
constexpr int kWaitVmcnt0 = 0x0F70;

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also orders global memory, for
// which it waits until every global load of the wavefront has returned: issued after a prefetch,
// that drains the prefetch before the first step.  Here the global loads stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Row normalisation to unit RMS, in one canonical order shared by qf_rms_norm_rows_bf16 and the GEMMs that
// normalise their staged x (qf_w8a16_gemm_rmsnorm), so that both give the same bits.  A row of N bf16 values is
// read as N / 8 pieces of 16 bytes, and lane t of one wavefront takes pieces t, t + 64, t + 128, ...  The lane
// keeps eight sums, one per value position in a piece, each adding the squares of its values over the lane's
// pieces in increasing order with fused multiply-adds (eight independent chains, N / 512 long); the lane's sum is
// ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7)).  The 64 lane sums fold within each 16-lane row by DPP adds
// (the neighbour, the other pair of the quad, the other quad of the 8 lanes, the other 8 lanes), and the four row
// sums r0..r3 (lanes 0, 16, 32, 48) add as (r0 + r1) + (r2 + r3).  Every step is an IEEE fp32 operation.

// 1 / sqrt(mean of squares + eps) (IEEE division; the same instructions wherever it is used).
__device__ __forceinline__ float rms_inv(float total, int n, float eps) {
  return 1.0f / __builtin_sqrtf(total / (float)n + eps);
}

// One 16-byte piece of 8 bf16 values scaled by inv, each product rounded to bf16 (nearest even).
__device__ __forceinline__ u32x4_t scale_piece(const u32x4_t v, float inv) {
  u32x4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = pack_bf16_rne(__uint_as_float(v[e] << 16) * inv, __uint_as_float(v[e] & 0xffff0000u) * inv);
  return o;
}

// Adds the squares of one piece's 8 values to the lane's eight sums (value e of the piece into sum e).
__device__ __forceinline__ void add_squares(float (&acc)[8], const u32x4_t x) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lo = __uint_as_float(x[e] << 16), hi = __uint_as_float(x[e] & 0xffff0000u);
    acc[2 * e] = __builtin_fmaf(lo, lo, acc[2 * e]);
    acc[2 * e + 1] = __builtin_fmaf(hi, hi, acc[2 * e + 1]);
  }
}

// Continues the lane's sums over the pieces base + 64 p + lane, for base = base0, base0 + 64 P, ... below npieces,
// read P at a time (the P loads issued before their multiply-adds).  base0 is the same for every lane, so the
// loop is uniform; a lane past the row's end adds zeros, which leaves its sums unchanged.
template <int P, typename Load>
__device__ __forceinline__ void add_row_squares(float (&acc)[8], int base0, int npieces, int lane, Load load) {
  for (int base = base0; base < npieces; base += P * kWave) {
    u32x4_t t[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int j = base + p * kWave + lane;
      t[p] = j < npieces ? load(j) : (u32x4_t){0, 0, 0, 0};
    }
#pragma unroll
    for (int p = 0; p < P; ++p)
      if (base + p * kWave < npieces) add_squares(acc, t[p]);
  }
}

template <int CTRL>
__device__ __forceinline__ float dpp_fold(float v) {
  return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}

// The row's sum of squares from the lanes' eight sums (every lane of the wavefront active); every lane returns it.
__device__ __forceinline__ float wave_square_total(const float (&a)[8]) {
  float s = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
  s = dpp_fold<0xb1>(s);   // quad_perm [1, 0, 3, 2]: the neighbour
  s = dpp_fold<0x4e>(s);   // quad_perm [2, 3, 0, 1]: the other pair of the quad
  s = dpp_fold<0x141>(s);  // row_half_mirror: the other quad of each 8 lanes
  s = dpp_fold<0x140>(s);  // row_mirror: the other 8 lanes of each 16-lane row
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 48));
  return (r0 + r1) + (r2 + r3);
}

// One row of npieces pieces normalised by one wavefront in the canonical order, through load(j) and
// store(j, piece).  The lane's first P pieces stay in registers for the scaling pass, later ones are read again.
// Each piece is read and written by its own lane only, so y may be x.
template <int P, typename Load, typename Store>
__device__ __forceinline__ void normalise_row(int npieces, int n, float eps, int lane, Load load, Store store) {
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  u32x4_t v[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int j = p * kWave + lane;
    v[p] = j < npieces ? load(j) : (u32x4_t){0, 0, 0, 0};
  }
#pragma unroll
  for (int p = 0; p < P; ++p)
    if (p * kWave < npieces) add_squares(acc, v[p]);
  add_row_squares<P>(acc, P * kWave, npieces, lane, load);
  const float inv = rms_inv(wave_square_total(acc), n, eps);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int j = p * kWave + lane;
    if (j < npieces) store(j, scale_piece(v[p], inv));
  }
  for (int j0 = P * kWave + lane; j0 < npieces; j0 += P * kWave) {
    u32x4_t t[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int j = j0 + p * kWave;
      t[p] = j < npieces ? load(j) : (u32x4_t){0, 0, 0, 0};
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int j = j0 + p * kWave;
      if (j < npieces) store(j, scale_piece(t[p], inv));
    }
  }
}

// Normalise the M staged rows of x in LDS (row m at byte m * pitch, K values) in place, in two passes between
// LDS-only barriers (the weight prefetch stays in flight across them):
// * the sums: wavefront w takes the rows w, w + WAVES, ..., each in the canonical order (the lane's pieces read
//   kStagedSumPieces at a time), and writes the row's scale factor to LDS;
// * the scaling, which has no order: piece q of the rows' M x K / 8 pieces (row-major) goes to thread
//   q mod (WAVES x 64), so every wavefront scales the same share whatever M is; each thread reads
//   kStagedScalePieces pieces before it scales and writes them (a read past the last piece is clamped to the last
//   row's first piece and not written back).
// Called by the whole workgroup after the staging barrier.  Both passes are bound by one wavefront's
// instruction issue (about one VALU instruction per 5.5 cycles on its own), not by the SIMD's throughput: the
// batches put all of a lane's loads for K = 5120 ahead of its arithmetic.
constexpr int kStagedSumPieces = 10;
constexpr int kStagedScalePieces = 8;
template <int WAVES>
__device__ __forceinline__ void normalise_staged_rows(uint8_t* smem, int pitch, int M, int K, float eps) {
  __shared__ float row_inv[QF_W8A16_MAX_M];
  constexpr int THREADS = WAVES * kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // uniform: the row fold needs every lane
  const int npieces = K / 8;
  for (int m = wave; m < M; m += WAVES) {
    const uint8_t* row = smem + m * pitch;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    add_row_squares<kStagedSumPieces>(acc, 0, npieces, lane,
                                      [&](int j) { return *reinterpret_cast<const u32x4_t*>(row + j * 16); });
    const float inv = rms_inv(wave_square_total(acc), K, eps);
    if (lane == 0) row_inv[m] = inv;
  }
  lds_barrier();
  // (m, j): the thread's next piece; a step of THREADS pieces is dm rows and dj pieces.
  const int total = M * npieces;
  const int dm = THREADS / npieces, dj = THREADS - dm * npieces;
  int m = (int)threadIdx.x / npieces;
  int j = (int)threadIdx.x - m * npieces;
  for (int q0 = threadIdx.x; q0 < total; q0 += kStagedScalePieces * THREADS) {
    u32x4_t t[kStagedScalePieces];
    int off[kStagedScalePieces];
    float inv[kStagedScalePieces];
#pragma unroll
    for (int p = 0; p < kStagedScalePieces; ++p) {
      const bool in = q0 + p * THREADS < total;
      const int mm = in ? m : M - 1;
      off[p] = mm * pitch + (in ? j : 0) * 16;
      t[p] = *reinterpret_cast<const u32x4_t*>(smem + off[p]);
      inv[p] = row_inv[mm];
      m += dm;
      j += dj;
      if (j >= npieces) j -= npieces, ++m;
    }
#pragma unroll
    for (int p = 0; p < kStagedScalePieces; ++p)
      if (q0 + p * THREADS < total) *reinterpret_cast<u32x4_t*>(smem + off[p]) = scale_piece(t[p], inv[p]);
  }
  lds_barrier();
}

// LDS row pitch (bytes) of a staged x slice of `steps` k-steps: the row bytes plus 32, so the rows
// that the 16 lanes of an MFMA fragment read start in distinct 32-byte bank groups.
__host__ __device__ __forceinline__ int x_pitch(int steps) { return steps * kStepK * 2 + 32; }

// Copy of x[0:M][64*s_begin : 64*(s_begin + steps)] into LDS (row m at byte m * x_pitch(steps)) in
// 16-byte pieces.  When one batch of kBatch pieces per thread holds the slice, the copy is done in
// two phases so that the caller can issue its weight requests in between: load_batch() requests the
// pieces into registers, store_batch() writes them to LDS (waiting only for these loads, which were
// issued first).  Larger slices are copied by copy_all() before the weight requests.
// Pieces are indexed (row << shift) | column, the column space padded to a power of two, so row and
// column come from a shift and a mask.
template <int THREADS, int BATCH = 10>
struct XStage {
  static constexpr int kBatch = BATCH;  // pieces per thread requested before the first LDS write
  u32x4_t v[kBatch];
  const uint16_t* src0;
  int row_pieces, shift, mask, span, pitch;

  __device__ __forceinline__ XStage(const GemmArgs& a, int s_begin, int steps) {
    row_pieces = steps * (kStepK / 8);
    shift = 32 - __builtin_clz((row_pieces - 1) | 1);  // ceil(log2(row_pieces)), >= 1
    mask = (1 << shift) - 1;
    span = a.M << shift;
    pitch = x_pitch(steps);
    src0 = a.x + (int64_t)s_begin * kStepK;
  }

  // Piece indices past the slice (or in a row's padding) are clamped to a piece of the slice, so
  // every thread loads and stores unconditionally: a clamped lane copies an in-slice piece again, to
  // the same LDS address.  Without branches around them, the compiler counts the loads in flight
  // exactly and lets the weight requests that follow stay in flight.
  __device__ __forceinline__ void piece(int base, int b, int& m, int& j) const {
    const int f = min(base + b * THREADS + (int)threadIdx.x, span - 1);
    m = f >> shift;
    j = min(f & mask, row_pieces - 1);
  }

  __device__ __forceinline__ void load_batch(const GemmArgs& a, int base) {
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      int m, j;
      piece(base, b, m, j);
      v[b] = *reinterpret_cast<const u32x4_t*>(src0 + (int64_t)m * a.ldx + j * 8);
    }
  }

  __device__ __forceinline__ void store_batch(uint8_t* smem, int base) {
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      int m, j;
      piece(base, b, m, j);
      *reinterpret_cast<u32x4_t*>(smem + m * pitch + j * 16) = v[b];
    }
  }

  // Whether one batch holds the whole slice (the pipelined path); otherwise copy_all() stages it.
  __device__ __forceinline__ bool single_batch() const { return span <= THREADS * kBatch; }

  __device__ __forceinline__ void copy_all(const GemmArgs& a, uint8_t* smem) {
    for (int base = 0; base < span; base += THREADS * kBatch) {
      load_batch(a, base);
      store_batch(smem, base);
    }
  }
};

// k-steps [begin, end) of split `split` out of `splits` over `ksteps` (balanced, deterministic).
__device__ __forceinline__ void split_range(int split, int splits, int ksteps, int& begin, int& end) {
  begin = (int)(((int64_t)split * ksteps) / splits);
  end = (int)(((int64_t)(split + 1) * ksteps) / splits);
}

// ---------------------------------------------------------------------------------------------
// MFMA kernel
//
// Workgroup = WN x WK wavefronts over NT-tile groups: wavefront (wn, wk) owns the NT consecutive
// 16-row n-tiles of group wn and the k-steps wk, wk + WK, ... of the workgroup's range (k-slice wk);
// blockIdx.y is the split of K
// across workgroups.  Lane l (group g = l / 16, r = l % 16) loads, for every 64-k step s:
//   rowmajor: w[tile*16 + r][s*64 + 16g .. +15]
//   tiled:    bytes [16 l, 16 l + 16) of the 1 KiB tile (tile, s), which hold the same values
// and the activation chunk x[r][s*64 + 16g .. +15] from LDS (row M - 1 when r >= M).  Both MFMA operands
// index k identically per lane, so the k order inside a step is immaterial to the product.
// LDS holds the workgroup's x slice row-major with a pitch of (row bytes + 32), so the 16 rows a
// fragment read touches start in distinct 32-byte bank groups.
//
// Reductions, all in a fixed order: the WK slices of a tile are summed through LDS in slice order;
// with split_k > 1 each workgroup writes its partial tile to the workspace, and the last workgroup
// of an n-block to finish (a per-n-block arrival counter in the workspace) sums the split_k partials
// in split order, applies the scale and writes y, then resets the counter to zero.
// ---------------------------------------------------------------------------------------------
// bf16 rounding of an fp32 value, widened back (the value a bf16 output holds)
__device__ __forceinline__ float bf16_value(float v) { return __uint_as_float((uint32_t)bf16_rne(v) << 16); }

// Fused argmax epilogue of the MFMA kernel (split_k == 1).  Each lane ranks its scaled outputs (bf16
// values, columns < n_valid) per token, the lanes of a token fold by shuffles, and each wavefront
// column folds its candidate into the token's slot with one 64-bit atomic maximum of argmax_key (the
// maximum of keys is the argmax whatever the order of arrival).  The atomics return nothing: no wait,
// no barrier, the workgroup leaves at once; argmax_slots_kernel reads the slots after the kernel.
template <int NT, int WN>
__device__ __forceinline__ void argmax_epilogue(const GemmArgs& a, const f32x4_t (&acc)[NT], bool holder, int tile0,
                                                int ntiles, int g, int wk, int wn, int lane) {
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  if (holder) {
    const int r = lane & 15;
    if (a.y != nullptr) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int tile = tile0 + t;
        const int n = tile * kTileN + 4 * g;
        if (tile < ntiles && n < a.N)
          store_out4(a.y, a.ldy, a.out_f32, a.vec_out, r, n, min(4, a.N - n), acc[t] * load_scale4(a.scale, a.N, n));
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int tile = tile0 + t;
      const int n = tile * kTileN + 4 * g;
      if (tile < ntiles && n < a.n_valid) {
        const f32x4_t v = acc[t] * load_scale4(a.scale, a.N, n);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (n + i < a.n_valid) argmax_fold(bf16_value(v[i]), n + i, bv, bi);
      }
    }
  }
  // lanes r, r + 16, r + 32, r + 48 hold token r's candidates
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
    const float ov = __shfl_xor(bv, off);
    const int oi = __shfl_xor(bi, off);
    argmax_fold(ov, oi, bv, bi);
  }
  if (wk == 0 && lane < a.M) {
    const int slot = (int)((blockIdx.x * WN + wn) % kArgmaxSlots);
    (void)__hip_atomic_fetch_max(a.am_slots + ((int64_t)slot * a.M + lane) * argmax_slot_stride(a.M),
                                 argmax_key(bv, bi), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Second pass of the fused argmax: one wavefront per token; lane s reads slot s (every atomic maximum of the
// GEMM is complete at the kernel boundary) and clears it for the next call (the workspace's counter prefix is
// zero on entry and on exit of every call); the maximum key over the lanes holds the token's index.
__global__ void __launch_bounds__(kWave) argmax_slots_kernel(uint64_t* slots, int64_t index_offset, int64_t* ids) {
  static_assert(kArgmaxSlots == kWave, "one slot per lane");
  uint64_t* p = slots + ((int64_t)threadIdx.x * gridDim.x + blockIdx.x) * argmax_slot_stride(gridDim.x);
  uint64_t key = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(p, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint64_t o = __shfl_xor(key, off, kWave);
    key = o > key ? o : key;
  }
  if (threadIdx.x == 0) ids[blockIdx.x] = (int64_t)(uint32_t)~(uint32_t)key + index_offset;
}

// Occupancy floor of the MFMA kernel.  One-tile, DEPTH-4 wavefronts fit in 80 VGPRs (the compiler's
// own choice is 84-92), which allows 6 wavefronts per SIMD instead of 5: three 8-wavefront workgroups
// per CU where the x slice leaves LDS for three (gate_up 34816x5120 at M = 5, 1088 workgroups, then
// runs in 1.4 rounds instead of 2.1: 33.05 -> 32.43 us, results unchanged).  The normalising builds
// (NORM) take a floor of 5 (96 VGPRs), room for the staged rows' loads in flight beside the ring; the
// shapes that select them run at most 2.5 wavefronts a SIMD (qkv 10240x5120: 160 workgroups of 8
// wavefronts at M = 5, 640 of 4 at M = 1).  Other shapes keep the compiler's allocation: forcing them
// to 6 wavefronts makes them spill.
template <int NT, int DEPTH, int WAVES, bool NORM = false>
struct MfmaMinWaves {
  static constexpr int value = (NT == 1 && DEPTH == 4) ? (NORM ? 5 : 6) : (WAVES >= 8 ? 2 : 1);
};

template <int LAYOUT, int NT, int WN, int WK, int DEPTH, bool NTH, bool XRING, bool NORM = false>
__global__ void __launch_bounds__(WN * WK * kWave)
    __attribute__((amdgpu_waves_per_eu(MfmaMinWaves<NT, DEPTH, WN * WK, NORM>::value, 8)))
    w8a16_mfma_kernel(const GemmArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ int last_arrival;
  constexpr int WAVES = WN * WK;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // uniform: scalar registers
  const int wn = wave % WN;
  const int wk = wave / WN;
  const int g = lane >> 4;
  const int r = lane & 15;
  const int split = blockIdx.y;
  int s_begin, s_end;
  split_range(split, a.split_k, a.ksteps, s_begin, s_end);
  const int wg_steps = s_end - s_begin;  // k-steps staged by this workgroup
  // The WK k-waves of a tile group interleave at step granularity: k-wave wk takes the steps
  // wk, wk + WK, wk + 2 WK, ... of the workgroup's range, so the group's waves read adjacent KiB of
  // the weight stream at any moment (one stream per tile rather than WK).  wg_steps >= WK.
  const int k_lo = wk;
  const int k_count = (wg_steps - wk + WK - 1) / WK;
  const int ntiles = a.n_pad / kTileN;
  const int tile0 = (blockIdx.x * WN + wn) * NT;
  // >= 1: the host keeps wg_steps >= WK.  A wavefront whose tiles lie past N (only in the last
  // workgroup column) runs one clamped step instead of skipping the loop, so no branch surrounds
  // the loads; its results are never stored.
  const int nsteps = tile0 < ntiles ? k_count : 1;

  // Weight fragment pointers at this wavefront's first step, and the byte stride between steps.
  const int8_t* wp[NT];
  constexpr int64_t step_bytes = ((LAYOUT == QF_LAYOUT_ROWMAJOR) ? kStepK : kTileN * kStepK) * WK;
  const int s0 = s_begin + k_lo;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int tile = min(tile0 + t, ntiles - 1);
    if constexpr (LAYOUT == QF_LAYOUT_ROWMAJOR) {
      const int row = min(tile * kTileN + r, a.N - 1);
      wp[t] = a.w + (int64_t)row * a.ldw + (int64_t)s0 * kStepK + g * 16;
    } else {
      wp[t] = a.w + (((int64_t)tile * a.ksteps + s0) * kWave + lane) * 16;
    }
  }

  // Every weight load in this kernel is unconditional: step indices past the slice are clamped to its
  // last step (an in-bounds re-read of a line just fetched) and their math is skipped.  Keeping
  // branches away from the loads lets the compiler keep DEPTH steps of loads in flight.
  // The ring has DEPTH + 1 slots: at step s the load for step s + DEPTH goes into the slot freed at
  // step s - 1, so it can be issued before step s's fragment is consumed.  In both x staging modes
  // the x requests go out first, then the first DEPTH steps of weights; writing x to LDS waits only
  // for the x requests (vmcnt retires in issue order), so the weight requests stay in flight across
  // the barriers.
  constexpr int RING = DEPTH + 1;
  u32x4_t buf[RING][NT];
  f32x4_t acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
  auto prologue = [&]() {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int sd = min(d, nsteps - 1);
#pragma unroll
      for (int t = 0; t < NT; ++t) buf[d][t] = load16<NTH>(wp[t] + sd * step_bytes);
    }
  };
  // One k-step: request the weights DEPTH steps ahead into the slot freed by the previous step, then
  // (for steps of the slice) dequantise ring slot d and multiply by the x fragments at xp.
  auto step = [&](int s, int d, const uint8_t* xp) {
    const int sn = min(s + DEPTH, nsteps - 1);
#pragma unroll
    for (int t = 0; t < NT; ++t) buf[(d + DEPTH) % RING][t] = load16<NTH>(wp[t] + (int64_t)sn * step_bytes);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch issue ahead of this step's math
    if (s < nsteps) {                   // uniform: steps past the slice only keep loads in flight
      const u32x4_t* p = reinterpret_cast<const u32x4_t*>(xp);
      const bf16x8_t xb0 = __builtin_bit_cast(bf16x8_t, p[0]);
      const bf16x8_t xb1 = __builtin_bit_cast(bf16x8_t, p[1]);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        bf16x8_t w0, w1;
        dequant16(buf[d][t], w0, w1);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0, xb0, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1, xb1, acc[t], 0, 0, 0);
      }
    }
  };
  // Lane (g, r) reads x[r][k + 16g .. +15] of each step.  Lanes of token rows r >= M read row M - 1
  // instead: MFMA column r only feeds output column r, which is never stored.
  const int xr = min(r, a.M - 1);

  if constexpr (!XRING) {
    // The workgroup's whole x slice (all WK k-slices) is staged once, before the first step.
    const int pitch = x_pitch(wg_steps);
    XStage<WAVES * kWave> xst(a, s_begin, wg_steps);
    if (xst.single_batch()) {  // uniform
      xst.load_batch(a, 0);
      __builtin_amdgcn_sched_barrier(0);  // the x requests go out before the weight requests
      prologue();
      __builtin_amdgcn_sched_barrier(0);
      xst.store_batch(smem, 0);
    } else {
      xst.copy_all(a, smem);
      prologue();
    }
    lds_barrier();  // the weight requests issued above stay in flight across it
    if constexpr (NORM) normalise_staged_rows<WAVES>(smem, pitch, a.M, a.K, a.norm_eps);
    const uint8_t* xs = smem + xr * pitch + (k_lo * kStepK + 16 * g) * 2;
    constexpr int xs_stride = kStepK * 2 * WK;
    for (int base = 0; base < nsteps; base += RING) {
#pragma unroll
      for (int d = 0; d < RING; ++d) step(base + d, d, xs + (size_t)(base + d) * xs_stride);
    }
  } else {
    // x through a two-slot LDS ring (k_waves == 1, so a wavefront's steps are the workgroup's): chunk
    // c holds steps [c RING, (c + 1) RING) of every token row, and block c of the loop computes them.
    // Each thread requests its pieces of chunk c + 1 into registers at the start of block c and
    // writes them to the other slot at the start of block c + 1, before the barrier that opens it;
    // the slot is free because every wavefront passed that barrier after finishing block c - 1.
    // Only a RING-step chunk is staged before the first step, instead of the whole slice.
    static_assert(WK == 1, "the x ring serves one k-slice per workgroup");
    constexpr int THREADS = WAVES * kWave;
    constexpr int CP = RING * 8;                               // 16-byte pieces per token row of a chunk
    constexpr int XP = (QF_W8A16_MAX_M * CP + THREADS - 1) / THREADS;  // pieces per thread, at most
    constexpr int SWM = CP % 16 == 0 ? 7 : 3;                  // the row swizzle stays inside the row
    const int cpieces = a.M * CP;
    const int slot_bytes = cpieces * 16;
    // Every wavefront runs every block, including one whose tiles lie past N (nsteps == 1): the
    // block barriers must match across the workgroup, and its threads stage their share of x.
    const int nchunks = (k_count + RING - 1) / RING;
    const int64_t kmax = (int64_t)s_end * kStepK - 8;          // last 8-element piece of the range
    u32x4_t xv[XP];
    // Piece q of a chunk lies at LDS byte 16 q and holds row m = q / CP, piece (q % CP) ^ sw(m) of
    // the row's steps: the XOR moves the rows' fragment reads onto different banks, as the +32-byte
    // row pitch of the whole-slice layout does.  Pieces past the chunk are clamped to its last piece.
    auto load_chunk = [&](int c) {
#pragma unroll
      for (int j = 0; j < XP; ++j) {
        const int q = min(j * THREADS + (int)threadIdx.x, cpieces - 1);
        const int m = q / CP;
        const int jx = (q - m * CP) ^ ((m & SWM) << 1);
        const int64_t k = min((int64_t)(s_begin + c * RING) * kStepK + jx * 8, kmax);
        xv[j] = *reinterpret_cast<const u32x4_t*>(a.x + (int64_t)m * a.ldx + k);
      }
    };
    auto store_chunk = [&](int c) {
      uint8_t* slot = smem + (c & 1) * slot_bytes;
#pragma unroll
      for (int j = 0; j < XP; ++j)
        *reinterpret_cast<u32x4_t*>(slot + min(j * THREADS + (int)threadIdx.x, cpieces - 1) * 16) = xv[j];
    };
    load_chunk(0);
    __builtin_amdgcn_sched_barrier(0);  // the x requests go out before the weight requests
    prologue();
    __builtin_amdgcn_sched_barrier(0);
    store_chunk(0);
    const int xsw = (xr & SWM) << 1;
    for (int c = 0; c < nchunks; ++c) {
      if (c > 0) store_chunk(c);
      lds_barrier();  // the weight requests stay in flight across it
      if (c + 1 < nchunks) load_chunk(c + 1);
      __builtin_amdgcn_sched_barrier(0);
      const uint8_t* xrow = smem + (c & 1) * slot_bytes + xr * (CP * 16);
#pragma unroll
      for (int d = 0; d < RING; ++d) step(c * RING + d, d, xrow + (((d * 8 + 2 * g) ^ xsw) << 4));
    }
  }

  // Sum the WK slices through LDS (the x slice is no longer read): slice 0 adds slices 1.. WK-1.
  if constexpr (WK > 1) {
    lds_barrier();
    f32x4_t* red = reinterpret_cast<f32x4_t*>(smem);
    if (wk > 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) red[((wk * WN + wn) * NT + t) * kWave + lane] = acc[t];
    }
    lds_barrier();
    if (wk == 0) {
      for (int j = 1; j < WK; ++j) {
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] += red[((j * WN + wn) * NT + t) * kWave + lane];
      }
    }
  }

  // Lane (g, r) of slice 0 holds C[n = tile*16 + 4g + i][m = r], i = 0..3.
  const bool holder = wk == 0 && tile0 < ntiles && r < a.M;
  if (a.split_k == 1) {
    if constexpr (!NORM) {  // the normalising builds serve qf_w8a16_gemm_rmsnorm only, never the fused argmax
      if (a.argmax) {
        argmax_epilogue<NT, WN>(a, acc, holder, tile0, ntiles, g, wk, wn, lane);
        return;
      }
    }
    if (holder) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int tile = tile0 + t;
        const int n = tile * kTileN + 4 * g;
        if (tile < ntiles && n < a.N) {
          const f32x4_t sc = load_scale4(a.scale, a.N, n);
          store_out4(a.y, a.ldy, a.out_f32, a.vec_out, r, n, min(4, a.N - n), acc[t] * sc);
        }
      }
    }
    return;
  }

  // split_k > 1: publish this workgroup's partial tiles, then count arrivals for the n-block.
  const int64_t plane = (int64_t)a.M * a.n_pad;
  if (!a.fused_reduce) {  // the second-pass kernel reduces
    if (holder) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int tile = tile0 + t;
        if (tile < ntiles) {
          float* dst = a.partial + (int64_t)split * plane + (int64_t)r * a.n_pad + tile * kTileN + 4 * g;
          *reinterpret_cast<f32x4_t*>(dst) = acc[t];
        }
      }
    }
    return;
  }
  // The partials are written with device-scope stores (written through to the device's coherence
  // point) and every wavefront waits for its stores to complete; after the barrier, thread 0 counts
  // the workgroup's arrival.  The last arrival reads the partials with device-scope loads, which are
  // served by the coherence point and are issued only once the increment has returned and selected
  // this workgroup: every other split's stores had completed there before its own increment.  The
  // ordering is that of the hardware, not a release/acquire pair of the memory model: a device-scope
  // release fence writes back the XCD's whole L2 (measured: once per workgroup, slower than the
  // second-pass kernel), and an acquire fence on the last arrival invalidates it (measured: down
  // 5120x17408 at M = 5, 80 last arrivals in the kernel's tail, 18.5 -> 22.1 us).  reduce = 1 (the
  // second-pass kernel) orders the partials by the kernel boundary instead.
  if (holder) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int tile = tile0 + t;
      if (tile < ntiles) {
        float* dst = a.partial + (int64_t)split * plane + (int64_t)r * a.n_pad + tile * kTileN + 4 * g;
#pragma unroll
        for (int i = 0; i < 4; ++i) __hip_atomic_store(dst + i, acc[t][i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(a.counters + blockIdx.x * a.counter_stride, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    last_arrival = prev == (unsigned)(a.split_k - 1);
  }
  __syncthreads();
  if (!last_arrival) return;
  if (holder) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int tile = tile0 + t;
      const int n = tile * kTileN + 4 * g;
      if (tile < ntiles && n < a.N) {
        float* src = a.partial + (int64_t)r * a.n_pad + n;
        f32x4_t sum = {0.f, 0.f, 0.f, 0.f};
        for (int j = 0; j < a.split_k; ++j) {
          f32x4_t v;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            v[i] = __hip_atomic_load(src + j * plane + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          sum = j == 0 ? v : sum + v;
        }
        const f32x4_t sc = load_scale4(a.scale, a.N, n);
        store_out4(a.y, a.ldy, a.out_f32, a.vec_out, r, n, min(4, a.N - n), sum * sc);
      }
    }
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(a.counters + blockIdx.x * a.counter_stride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------------------
// Stream kernel (QF_KERNEL_MFMA_STREAM), TILED layout, M <= 16: the whole weight image in one resident
// round of workgroups.
//
// The grid is G workgroups, one per CU (G = the device's CU count), so every workgroup starts at once and
// none stages x after another has begun streaming.  Workgroup b owns the contiguous run of 16-row tiles
// [b * ntiles / G, (b + 1) * ntiles / G).  Its W wavefronts interleave over k: wavefront v takes the k-steps
// v, v + W, v + 2 W, ... of every tile of the run, tile after tile, as one stream, with a DEPTH-step prefetch
// ring that runs across tile boundaries (W * DEPTH KiB of weight loads in flight per CU).  At any moment the
// W wavefronts read W adjacent KiB of one tile.  x (the whole [M, K] slice) is staged in LDS once, with the
// first DEPTH steps of weights requested before the barrier.
//
// Sums, in a fixed order: wavefront v sums its k-steps of a tile in increasing k (two MFMAs a step); when it
// leaves the tile it writes that partial tile to LDS ([tile][wavefront] slots, 1 KiB each).  After the run,
// wavefront v reduces tiles v, v + W, ...: the W partials in wavefront order, then the scale, then one bf16
// rounding.  Results are bitwise reproducible; they differ from w8a16_mfma_kernel's (whose k-slices are
// interleaved four ways) only in fp32 summation order.
// ---------------------------------------------------------------------------------------------
__host__ __device__ __forceinline__ int align16i(int n) { return (n + 15) & ~15; }

template <int W, int DEPTH, bool NTH, bool NORM = false>
__global__ void __launch_bounds__(W * kWave) w8a16_stream_kernel(const GemmArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int RING = DEPTH + 1;
  const int lane = threadIdx.x & (kWave - 1);
  const int v = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int g = lane >> 4;
  const int r = lane & 15;
  const int ntiles = a.n_pad / kTileN;
  // The workgroup's tiles: t0, t0 + tstep, ..., nt of them (a contiguous run, or every G-th tile).
  const int tstep = a.tiles_strided ? (int)gridDim.x : 1;
  const int t0 = a.tiles_strided ? (int)blockIdx.x : (int)(((int64_t)blockIdx.x * ntiles) / gridDim.x);
  const int nt = a.tiles_strided ? (ntiles - (int)blockIdx.x + tstep - 1) / tstep
                                 : (int)(((int64_t)(blockIdx.x + 1) * ntiles) / gridDim.x) - t0;
  if (nt <= 0) return;  // uniform over the workgroup: more workgroups than tiles
  const int ksteps = a.ksteps;
  const int S = (ksteps - v + W - 1) / W;  // k-steps of this wavefront in each tile, >= 1 (ksteps >= W)
  const int total = nt * S;                // steps of this wavefront over the run
  const int pitch = x_pitch(ksteps);
  f32x4_t* part = reinterpret_cast<f32x4_t*>(smem + align16i(a.M * pitch));  // [nt][W][64 lanes]

  // Prefetch cursor: the weight fragment of step pi (tile pi / S, k-step v + (pi % S) W) for this lane.
  // Past the last step the cursor stays on it (an in-bounds re-read), so every load is unconditional.
  const int8_t* pf = a.w + (((int64_t)t0 * ksteps + v) * kWave + lane) * 16;
  const int64_t step_b = (int64_t)W * kTileN * kStepK;
  const int64_t wrap_b = ((int64_t)(tstep - 1) * ksteps + ksteps - (S - 1) * W) * kTileN * kStepK;
  int pi = 0, pj = 0;
  auto advance = [&]() {
    if (pi < total - 1) {
      ++pi;
      if (++pj < S) {
        pf += step_b;
      } else {
        pj = 0;
        pf += wrap_b;
      }
    }
  };

  u32x4_t buf[RING];
  // 16 pieces a thread at 8 wavefronts (10 at 16): one batch stages M = 8 rows of K = 5120 or 8192
  XStage<W * kWave, W >= 16 ? 10 : 16> xst(a, 0, ksteps);
  auto prologue = [&]() {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      buf[d] = load16<NTH>(pf);
      advance();
    }
  };
  if (xst.single_batch()) {  // uniform
    xst.load_batch(a, 0);
    __builtin_amdgcn_sched_barrier(0);  // the x requests go out before the weight requests
    prologue();
    __builtin_amdgcn_sched_barrier(0);
    xst.store_batch(smem, 0);
  } else {  // larger slices: the weight requests first, so they are in flight while x is staged
    prologue();
    __builtin_amdgcn_sched_barrier(0);
    xst.copy_all(a, smem);
  }
  lds_barrier();  // the weight requests issued above stay in flight across it
  if constexpr (NORM) normalise_staged_rows<W>(smem, pitch, a.M, a.K, a.norm_eps);

  // Lane (g, r) reads x[min(r, M - 1)][k + 16 g .. + 15] of each step (token rows r >= M are never stored).
  const uint8_t* xrow = smem + min(r, a.M - 1) * pitch + 32 * g;
  const uint32_t x0 = (uint32_t)v * (kStepK * 2);
  uint32_t xoff = x0;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  int cj = 0, tl = 0;
  for (int base = 0; base < total; base += RING) {
#pragma unroll
    for (int d = 0; d < RING; ++d) {
      buf[(d + DEPTH) % RING] = load16<NTH>(pf);
      advance();
      __builtin_amdgcn_sched_barrier(0);  // keep the prefetch issue ahead of this step's math
      if (base + d < total) {             // uniform
        const u32x4_t* xp = reinterpret_cast<const u32x4_t*>(xrow + xoff);
        const bf16x8_t xb0 = __builtin_bit_cast(bf16x8_t, xp[0]);
        const bf16x8_t xb1 = __builtin_bit_cast(bf16x8_t, xp[1]);
        bf16x8_t w0, w1;
        dequant16(buf[d], w0, w1);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0, xb0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1, xb1, acc, 0, 0, 0);
        if (++cj < S) {
          xoff += W * kStepK * 2;
        } else {  // this wavefront's share of the tile is done: park its partial
          part[(tl * W + v) * kWave + lane] = acc;
          acc = (f32x4_t){0.f, 0.f, 0.f, 0.f};
          ++tl;
          cj = 0;
          xoff = x0;
        }
      }
    }
  }
  lds_barrier();
  // Lane (g, r) holds C[n = tile * 16 + 4 g + i][m = r], i = 0..3, in each partial.
  for (int t = v; t < nt; t += W) {
    f32x4_t sum = part[(t * W) * kWave + lane];
#pragma unroll
    for (int u = 1; u < W; ++u) sum += part[(t * W + u) * kWave + lane];
    const int n = (t0 + t * tstep) * kTileN + 4 * g;
    if (r < a.M && n < a.N)
      store_out4(a.y, a.ldy, a.out_f32, a.vec_out, r, n, min(4, a.N - n), sum * load_scale4(a.scale, a.N, n));
  }
}

// The stream kernel with each wavefront's x fragments in registers instead of a staged LDS slice
// (QF_KERNEL_MFMA_STREAM, reduce = 1): wavefront v uses the x fragments of its k-steps v, v + W, ..., the same
// S = K / (64 W) steps in every tile, so it loads those 2 S fragments (16 bytes per lane each) once, before
// its first weight requests, and no barrier precedes the first step.  S is a multiple of the ring size, so
// both the ring slot and the x register of every step are compile-time.  Sums and results are those of
// w8a16_stream_kernel<W, DEPTH> bit for bit (the same steps in the same order, the same partial slots).
template <int W, int S, int DEPTH>
__global__ void __launch_bounds__(W * kWave) w8a16_stream_xreg_kernel(const GemmArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int RING = DEPTH + 1;
  static_assert(S % RING == 0, "a tile's steps fill whole ring turns");
  const int lane = threadIdx.x & (kWave - 1);
  const int v = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int g = lane >> 4;
  const int r = lane & 15;
  const int ntiles = a.n_pad / kTileN;
  // The workgroup's tiles: t0, t0 + tstep, ..., nt of them (a contiguous run, or every G-th tile).
  const int tstep = a.tiles_strided ? (int)gridDim.x : 1;
  const int t0 = a.tiles_strided ? (int)blockIdx.x : (int)(((int64_t)blockIdx.x * ntiles) / gridDim.x);
  const int nt = a.tiles_strided ? (ntiles - (int)blockIdx.x + tstep - 1) / tstep
                                 : (int)(((int64_t)(blockIdx.x + 1) * ntiles) / gridDim.x) - t0;
  if (nt <= 0) return;  // uniform over the workgroup: more workgroups than tiles
  constexpr int ksteps = W * S;  // the host launches this kernel only for K = 64 W S
  const int total = nt * S;
  f32x4_t* part = reinterpret_cast<f32x4_t*>(smem);  // [nt][W][64 lanes]

  // x fragments: lane (g, r) holds x[min(r, M - 1)][64 (v + j W) + 16 g .. + 15] for j < S.
  const uint16_t* xp = a.x + (int64_t)min(r, a.M - 1) * a.ldx + (int64_t)v * kStepK + 16 * g;
  u32x4_t xf[S][2];
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const u32x4_t* q = reinterpret_cast<const u32x4_t*>(xp + (int64_t)j * W * kStepK);
    xf[j][0] = q[0];
    xf[j][1] = q[1];
  }
  __builtin_amdgcn_sched_barrier(0);  // the x requests go out before the weight requests

  const int8_t* pf = a.w + (((int64_t)t0 * ksteps + v) * kWave + lane) * 16;
  constexpr int64_t step_b = (int64_t)W * kTileN * kStepK;
  const int64_t wrap_b = ((int64_t)(tstep - 1) * ksteps + ksteps - (S - 1) * W) * kTileN * kStepK;
  int pi = 0, pj = 0;
  auto advance = [&]() {
    if (pi < total - 1) {  // past the last step the cursor stays on it (an in-bounds re-read)
      ++pi;
      if (++pj < S) {
        pf += step_b;
      } else {
        pj = 0;
        pf += wrap_b;
      }
    }
  };
  u32x4_t buf[RING];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    buf[d] = load16<true>(pf);
    advance();
  }
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int t = 0; t < nt; ++t) {
#pragma unroll
    for (int j = 0; j < S; ++j) {
      buf[(j + DEPTH) % RING] = load16<true>(pf);
      advance();
      __builtin_amdgcn_sched_barrier(0);  // keep the prefetch issue ahead of this step's math
      bf16x8_t w0, w1;
      dequant16(buf[j % RING], w0, w1);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0, __builtin_bit_cast(bf16x8_t, xf[j][0]), acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1, __builtin_bit_cast(bf16x8_t, xf[j][1]), acc, 0, 0, 0);
    }
    part[(t * W + v) * kWave + lane] = acc;
    acc = (f32x4_t){0.f, 0.f, 0.f, 0.f};
  }
  lds_barrier();
  for (int t = v; t < nt; t += W) {
    f32x4_t sum = part[(t * W) * kWave + lane];
#pragma unroll
    for (int u = 1; u < W; ++u) sum += part[(t * W + u) * kWave + lane];
    const int n = (t0 + t * tstep) * kTileN + 4 * g;
    if (r < a.M && n < a.N)
      store_out4(a.y, a.ldy, a.out_f32, a.vec_out, r, n, min(4, a.N - n), sum * load_scale4(a.scale, a.N, n));
  }
}

// ---------------------------------------------------------------------------------------------
// Wide-M MFMA kernel, TILED layout: M > 16 (prefill chunks, long verification batches).
//
// A workgroup owns WN * NT 16-row weight tiles over the whole K range (one wavefront per NT tiles,
// as in the decode kernel) and one group of up to MT * 16 token rows.  Each weight fragment is
// dequantised once per step and multiplied by the x fragments of all MT token tiles, so a group's
// weights cross the memory system once instead of once per 16 tokens.  x reaches LDS through the
// decode kernel's two-slot ring (chunks of DEPTH + 1 steps), sized for the group's rows.
//
// M above one group runs a.groups groups of a.group_rows rows (the last one shorter) in the same
// launch, and a.split_k > 1 splits K across workgroups (fp32 partial sums, reduced by
// splitk_reduce_kernel).  The grid is one-dimensional over (split, n-block, group).  The hardware
// hands workgroup i to XCD i % kXcds; the placement below gives the groups of one (split, n-block)
// consecutive workgroups of one XCD, so they run together and all but the first find the block's
// weights in that XCD's L2.
// ---------------------------------------------------------------------------------------------
template <int NT, int MT, int WN, int DEPTH>
__global__ void __launch_bounds__(WN * kWave) w8a16_wide_kernel(const GemmArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int THREADS = WN * kWave;
  constexpr int RING = DEPTH + 1;
  constexpr int CP = RING * 8;                               // 16-byte pieces per token row of a chunk
  constexpr int XP = (MT * 16 * CP + THREADS - 1) / THREADS;  // pieces per thread, at most
  // Chunk rows of 8-wavefront workgroups (one per CU) are padded by 16 bytes and read at plain
  // offsets.  4-wavefront workgroups keep the rows unpadded, so that a 64-row ring of DEPTH 4 fills
  // exactly half of a CU's LDS and two workgroups share a CU, and move piece j of row m to position
  // j ^ ((m & SWM) << 1) instead (measured: the padded rows gain 1-7% on 8 wavefronts; on 4 they
  // cost the second workgroup, 20% at gate_up M = 512).
  constexpr bool PAD = WN == 8;
  constexpr int SWM = PAD ? 0 : (CP % 16 == 0 ? 7 : 3);     // the row swizzle stays inside the row
  constexpr int ROW = (CP + (PAD ? 1 : 0)) * 16;
  constexpr int64_t step_bytes = kTileN * kStepK;            // one KiB block of a tile per step
  const int lane = threadIdx.x & (kWave - 1);
  const int wn = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int g = lane >> 4;
  const int r = lane & 15;

  // Workgroup -> linear index l -> (split, n-block, token group), the group fastest.  Workgroups i,
  // i + kXcds, i + 2 kXcds ... share an XCD and take consecutive l.
  const int ntiles = a.n_pad / kTileN;
  const int nblocks = (ntiles + WN * NT - 1) / (WN * NT);
  int l = blockIdx.x;
  if (a.groups > 1) {
    l = xcd_major(blockIdx.x, gridDim.x);
  }
  const int grp = l % a.groups;
  const int nb = (l / a.groups) % nblocks;
  const int split = l / a.groups / nblocks;
  int s_begin, s_end;
  split_range(split, a.split_k, a.ksteps, s_begin, s_end);
  const int m0 = grp * a.group_rows;
  const int mg = min(a.group_rows, a.M - m0);  // >= 1: the host sizes the groups so
  const uint16_t* xg = a.x + (int64_t)m0 * a.ldx;

  const int tile0 = (nb * WN + wn) * NT;
  const int k_count = s_end - s_begin;  // >= 1: split_k <= ksteps
  // A wavefront whose tiles lie past N runs one clamped step (see w8a16_mfma_kernel) but every block
  // of the x ring, whose barriers the whole workgroup must meet.
  const int nsteps = tile0 < ntiles ? k_count : 1;
  const int8_t* wp[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int tile = min(tile0 + t, ntiles - 1);
    wp[t] = a.w + (((int64_t)tile * a.ksteps + s_begin) * kWave + lane) * 16;
  }

  u32x4_t buf[RING][NT];
  f32x4_t acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = (f32x4_t){0.f, 0.f, 0.f, 0.f};

  // Lane (g, r) of token tile mt reads row min(16 mt + r, mg - 1) of the group: rows past the group
  // repeat its last row and their MFMA columns are never stored.
  int xoff[MT], xsw[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int xm = min(mt * 16 + r, mg - 1);
    xoff[mt] = xm * ROW;
    xsw[mt] = (xm & SWM) << 1;
  }

  const int cpieces = mg * CP;
  const int slot_bytes = mg * ROW;  // LDS bytes of one ring slot
  const int nchunks = (k_count + RING - 1) / RING;
  const int64_t kmax = (int64_t)s_end * kStepK - 8;  // last 8-element piece of the range
  u32x4_t xv[XP];
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      const int q = min(j * THREADS + (int)threadIdx.x, cpieces - 1);
      const int m = q / CP;
      const int jx = (q - m * CP) ^ ((m & SWM) << 1);  // the x piece that LDS position q holds
      const int64_t k = min((int64_t)(s_begin + c * RING) * kStepK + jx * 8, kmax);
      xv[j] = *reinterpret_cast<const u32x4_t*>(xg + (int64_t)m * a.ldx + k);
    }
  };
  auto store_chunk = [&](int c) {
    uint8_t* slot = smem + (c & 1) * slot_bytes;
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      const int q = min(j * THREADS + (int)threadIdx.x, cpieces - 1);
      *reinterpret_cast<u32x4_t*>(slot + q * 16 + (PAD ? q / CP * 16 : 0)) = xv[j];
    }
  };

  load_chunk(0);
  __builtin_amdgcn_sched_barrier(0);  // the x requests go out before the weight requests
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    const int sd = min(d, nsteps - 1);
#pragma unroll
    for (int t = 0; t < NT; ++t) buf[d][t] = load16<true>(wp[t] + sd * step_bytes);
  }
  __builtin_amdgcn_sched_barrier(0);
  store_chunk(0);
  for (int c = 0; c < nchunks; ++c) {
    if (c > 0) store_chunk(c);
    lds_barrier();  // the weight requests stay in flight across it
    if (c + 1 < nchunks) load_chunk(c + 1);
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* slot = smem + (c & 1) * slot_bytes;
#pragma unroll
    for (int d = 0; d < RING; ++d) {
      const int s = c * RING + d;
      const int sn = min(s + DEPTH, nsteps - 1);
#pragma unroll
      for (int t = 0; t < NT; ++t) buf[(d + DEPTH) % RING][t] = load16<true>(wp[t] + (int64_t)sn * step_bytes);
      __builtin_amdgcn_sched_barrier(0);  // keep the prefetch issue ahead of this step's math
      if (s < nsteps) {                   // uniform
        bf16x8_t w0[NT], w1[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) dequant16(buf[d][t], w0[t], w1[t]);
        bf16x8_t xb0[MT], xb1[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const u32x4_t* p = reinterpret_cast<const u32x4_t*>(slot + xoff[mt] + (((d * 8 + 2 * g) ^ xsw[mt]) << 4));
          xb0[mt] = __builtin_bit_cast(bf16x8_t, p[0]);
          xb1[mt] = __builtin_bit_cast(bf16x8_t, p[1]);
        }
        // First halves of every (tile, token tile) pair, then the second halves: no MFMA waits on
        // the one just before it.
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int t = 0; t < NT; ++t)
            acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0[t], xb0[mt], acc[t][mt], 0, 0, 0);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int t = 0; t < NT; ++t)
            acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1[t], xb1[mt], acc[t][mt], 0, 0, 0);
      }
    }
  }

  // Lane (g, r) holds C[n = tile*16 + 4g + i][m = 16 mt + r] of the group, i = 0..3.
  if (tile0 >= ntiles) return;
  if (a.split_k > 1) {  // partial sums [split][M][n_pad], summed and scaled by splitk_reduce_kernel
    float* part = a.partial + (int64_t)split * a.M * a.n_pad;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int tile = tile0 + t;
      if (tile < ntiles) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int m = mt * 16 + r;
          if (m < mg)
            *reinterpret_cast<f32x4_t*>(part + (int64_t)(m0 + m) * a.n_pad + tile * kTileN + 4 * g) = acc[t][mt];
        }
      }
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int tile = tile0 + t;
    const int n = tile * kTileN + 4 * g;
    if (tile < ntiles && n < a.N) {
      const f32x4_t sc = load_scale4(a.scale, a.N, n);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + r;
        if (m < mg) store_out4(a.y, a.ldy, a.out_f32, a.vec_out, m0 + m, n, min(4, a.N - n), acc[t][mt] * sc);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// W8A8 path for M > 16 on TILED weights: the arithmetic of the reference's fallback for M > 16
// (scaled_int8_quant + cutlass_scaled_mm, plugin/qwen_fastpath/patches.py:99-100).  Activations are
// quantised per token to int8, multiplied by the int8 weights with exact int32 sums on
// v_mfma_i32_16x16x64_i8, and scaled as (float(sum) * s_a[m]) * s_w[n].
// ---------------------------------------------------------------------------------------------

// Per-token quantiser: s_a[m] = amax_k |x[m, k]| * fl(1/127) (amax / 127.0 as torch evaluates a tensor
// divided by a scalar on the device; vLLM's kernel divides, at most an ulp away) and
// xq[m, k] = clamp(rint(x / s_a), -128, 127) with an IEEE division; a row of zeros gets s_a = 0 and
// xq = 0.  Finite inputs.  One workgroup per row, 8 values a thread per 16-byte load (K % 64 == 0,
// 16-byte-aligned rows: the GEMM's own contract).  With NP > 0 each thread keeps its (at most NP) pieces
// of the row in registers between the two passes, so the row is read once; NP == 0 reads it twice (any
// K).  The per-value arithmetic is the same, so the results are too.
__device__ __forceinline__ float quant_amax8(float amax, const u32x4_t v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    amax = fmaxf(amax, fabsf(__uint_as_float(v[i] << 16)));
    amax = fmaxf(amax, fabsf(__uint_as_float(v[i] & 0xffff0000u)));
  }
  return amax;
}

__device__ __forceinline__ u32x2_t quant_pack8(const u32x4_t v, float s) {
  uint32_t b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float f = __uint_as_float((i & 1) ? (v[i >> 1] & 0xffff0000u) : (v[i >> 1] << 16));
    float t = s > 0.f ? rintf(__fdiv_rn(f, s)) : 0.f;
    t = fminf(fmaxf(t, -128.f), 127.f);
    b[i] = (uint32_t)(int)t & 0xffu;
  }
  u32x2_t o;
  o.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
  o.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
  return o;
}

// With tiled != 0 the int8 row goes to the token-tiled image instead of a row of xq (8 values of row m
// at k land at byte ((m / 16) * ksteps + k / 64) * 1024 + 16 (16 ((k / 16) % 4) + m % 16) + k % 16), and
// the grid also covers the image's rows past M (up to the next multiple of 16), written as zeros.  A
// block's 16 rows interleave in every line they write, so they are given to workgroups of one XCD
// (workgroup i runs on XCD i % 8): its L2 then assembles whole lines before they are written back
// (rows of one block spread over the 8 XCDs: down 2048 x 17408 35.8 us, against 23.0 for row-major xq).
__device__ __forceinline__ int64_t token_tile_offset(int64_t m, int k, int ksteps) {
  return ((m >> 4) * ksteps + (k >> 6)) * 1024 + ((((k >> 4) & 3) << 4) + (m & 15)) * 16 + (k & 15);
}

template <int NP>
__global__ void __launch_bounds__(256) quantize_tokens_kernel(const uint16_t* x, int64_t ldx, int K, int8_t* xq,
                                                              int64_t ldq, float* s_a, int M, int tiled) {
  __shared__ float red[256 / kWave];
  int64_t m = blockIdx.x;
  if (tiled) m = xcd_major(blockIdx.x, gridDim.x);  // consecutive rows on one XCD
  const int pieces = K / 8;
  if (m >= M) {  // tiled only: a padding row of the last token block
    for (int c = threadIdx.x; c < pieces; c += 256)
      *reinterpret_cast<u32x2_t*>(xq + token_tile_offset(m, 8 * c, K / kStepK)) = (u32x2_t){0u, 0u};
    return;
  }
  const u32x4_t* row = reinterpret_cast<const u32x4_t*>(x + m * ldx);
  float amax = 0.f;
  u32x4_t keep[NP > 0 ? NP : 1];
  if constexpr (NP > 0) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int c = (int)threadIdx.x + i * 256;
      keep[i] = c < pieces ? row[c] : (u32x4_t){0u, 0u, 0u, 0u};
      amax = quant_amax8(amax, keep[i]);
    }
  } else {
    for (int c = threadIdx.x; c < pieces; c += 256) amax = quant_amax8(amax, row[c]);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int i = 1; i < 256 / kWave; ++i) amax = fmaxf(amax, red[i]);
  const float inv127 = 1.0f / 127.0f;  // constant-folded: the fp32 reciprocal of 127
  const float s = amax * inv127;
  if (threadIdx.x == 0) s_a[m] = s;
  const int ksteps = K / kStepK;
  auto dst = [&](int c) -> u32x2_t* {
    return reinterpret_cast<u32x2_t*>(tiled ? xq + token_tile_offset(m, 8 * c, ksteps) : xq + m * ldq + 8 * c);
  };
  if constexpr (NP > 0) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int c = (int)threadIdx.x + i * 256;
      if (c < pieces) *dst(c) = quant_pack8(keep[i], s);
    }
  } else {
    for (int c = threadIdx.x; c < pieces; c += 256) *dst(c) = quant_pack8(row[c], s);
  }
}

typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));

// The wide-M kernel's structure (tiles, 64-row token groups, XCD placement, K split, x ring) with int8
// activations: the TILED layout's 1 KiB block (lane (g, r): row r, k 16 g .. 16 g + 15 of a 64-k step)
// is the A operand of v_mfma_i32_16x16x64_i8 as loaded, and the B operand is the 16 activation bytes
// of token row r at the same k, so there is no conversion work.  The x ring rows (CP 16-byte pieces of
// 16 activations) are padded by 16 bytes: the 16 rows of a fragment read then sit on distinct 16-byte
// bank groups.  Sums are exact in int32 (|sum| <= K * 128 * 127 < 2^31 for K < 132000).
// On row-major weights lane (g, r) loads the same 16 bytes from row r of the tile directly (a 64-byte
// piece of each of 16 rows per k-step, as the decode kernel's row-major path reads them).
template <int LAYOUT, int NT, int MT, int WN, int DEPTH>
__global__ void __launch_bounds__(WN * kWave) w8a8_wide_kernel(const GemmArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int THREADS = WN * kWave;
  constexpr int RING = DEPTH + 1;
  constexpr int CP = RING * 4;                               // 16-byte pieces per token row of a chunk
  constexpr int XP = (MT * 16 * CP + THREADS - 1) / THREADS;  // pieces per thread, at most
  constexpr int ROW = (CP + 1) * 16;
  constexpr int64_t step_bytes = LAYOUT == QF_LAYOUT_ROWMAJOR ? kStepK : kTileN * kStepK;
  const int lane = threadIdx.x & (kWave - 1);
  const int wn = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int g = lane >> 4;
  const int r = lane & 15;

  const int ntiles = a.n_pad / kTileN;
  const int nblocks = (ntiles + WN * NT - 1) / (WN * NT);
  int l = blockIdx.x;
  if (a.groups > 1) {  // the groups of one (split, n-block) on consecutive workgroups of one XCD
    l = xcd_major(blockIdx.x, gridDim.x);
  }
  const int grp = l % a.groups;
  const int nb = (l / a.groups) % nblocks;
  const int split = l / a.groups / nblocks;
  int s_begin, s_end;
  split_range(split, a.split_k, a.ksteps, s_begin, s_end);
  const int m0 = grp * a.group_rows;
  const int mg = min(a.group_rows, a.M - m0);  // >= 1
  const int8_t* xg = a.xq + (int64_t)m0 * a.ldx;

  const int tile0 = (nb * WN + wn) * NT;
  const int k_count = s_end - s_begin;
  const int nsteps = tile0 < ntiles ? k_count : 1;
  const int8_t* wp[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int tile = min(tile0 + t, ntiles - 1);
    if constexpr (LAYOUT == QF_LAYOUT_ROWMAJOR) {
      const int row = min(tile * kTileN + (lane & 15), a.N - 1);
      wp[t] = a.w + (int64_t)row * a.ldw + (int64_t)s_begin * kStepK + g * 16;
    } else {
      wp[t] = a.w + (((int64_t)tile * a.ksteps + s_begin) * kWave + lane) * 16;
    }
  }

  u32x4_t buf[RING][NT];
  i32x4_t acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = (i32x4_t){0, 0, 0, 0};
  int xoff[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xoff[mt] = min(mt * 16 + r, mg - 1) * ROW + g * 16;

  const int cpieces = mg * CP;
  const int slot_bytes = mg * ROW;
  const int nchunks = (k_count + RING - 1) / RING;
  const int64_t kmax = (int64_t)s_end * kStepK - 16;  // last 16-activation piece of the range
  u32x4_t xv[XP];
  // Piece q of a chunk is 16 activations of row m, k piece p: q = m * CP + p on row-major x (a row's
  // pieces are contiguous), q = p * mg + m on the token-tiled image (16 rows of one k piece are).
  auto piece = [&](int q, int& m, int& p) {
    if (a.x_tiled) {
      p = q / mg;
      m = q - p * mg;
    } else {
      m = q / CP;
      p = q - m * CP;
    }
  };
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      int m, p;
      piece(min(j * THREADS + (int)threadIdx.x, cpieces - 1), m, p);
      const int64_t k = min((int64_t)(s_begin + c * RING) * kStepK + p * 16, kmax);
      const int8_t* src = a.x_tiled ? a.xq + token_tile_offset(m0 + m, (int)k, a.ksteps) : xg + (int64_t)m * a.ldx + k;
      xv[j] = *reinterpret_cast<const u32x4_t*>(src);
    }
  };
  auto store_chunk = [&](int c) {
    uint8_t* slot = smem + (c & 1) * slot_bytes;
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      int m, p;
      piece(min(j * THREADS + (int)threadIdx.x, cpieces - 1), m, p);
      *reinterpret_cast<u32x4_t*>(slot + m * ROW + p * 16) = xv[j];
    }
  };

  load_chunk(0);
  __builtin_amdgcn_sched_barrier(0);  // the x requests go out before the weight requests
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    const int sd = min(d, nsteps - 1);
#pragma unroll
    for (int t = 0; t < NT; ++t) buf[d][t] = load16<true>(wp[t] + sd * step_bytes);
  }
  __builtin_amdgcn_sched_barrier(0);
  store_chunk(0);
  for (int c = 0; c < nchunks; ++c) {
    if (c > 0) store_chunk(c);
    lds_barrier();  // the weight requests stay in flight across it
    if (c + 1 < nchunks) load_chunk(c + 1);
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* slot = smem + (c & 1) * slot_bytes;
    // x fragments of a step are read from LDS one step ahead, inside the chunk (its slot stays valid
    // until the next barrier), so their latency overlaps the previous step's MFMAs.
    i32x4_t xb[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xb[mt] = *reinterpret_cast<const i32x4_t*>(slot + xoff[mt]);
#pragma unroll
    for (int d = 0; d < RING; ++d) {
      const int s = c * RING + d;
      const int sn = min(s + DEPTH, nsteps - 1);
#pragma unroll
      for (int t = 0; t < NT; ++t) buf[(d + DEPTH) % RING][t] = load16<true>(wp[t] + (int64_t)sn * step_bytes);
      __builtin_amdgcn_sched_barrier(0);  // keep the prefetch issue ahead of this step's math
      i32x4_t xn[MT];
      if (d + 1 < RING) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) xn[mt] = *reinterpret_cast<const i32x4_t*>(slot + xoff[mt] + (d + 1) * 64);
      }
      if (s < nsteps) {  // uniform
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const i32x4_t wv = __builtin_bit_cast(i32x4_t, buf[d][t]);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            acc[t][mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wv, xb[mt], acc[t][mt], 0, 0, 0);
        }
      }
      if (d + 1 < RING) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) xb[mt] = xn[mt];
      }
    }
  }

  // Lane (g, r) holds C[n = tile*16 + 4g + i][m = 16 mt + r] of the group, i = 0..3.
  if (tile0 >= ntiles) return;
  if (a.split_k > 1) {  // exact int32 partial sums [split][M][n_pad], summed by splitk_reduce_w8a8_kernel
    int32_t* part = reinterpret_cast<int32_t*>(a.partial) + (int64_t)split * a.M * a.n_pad;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int tile = tile0 + t;
      if (tile < ntiles) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int m = mt * 16 + r;
          if (m < mg)
            *reinterpret_cast<i32x4_t*>(part + (int64_t)(m0 + m) * a.n_pad + tile * kTileN + 4 * g) = acc[t][mt];
        }
      }
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int tile = tile0 + t;
    const int n = tile * kTileN + 4 * g;
    if (tile < ntiles && n < a.N) {
      const f32x4_t sc = load_scale4(a.scale, a.N, n);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + r;
        if (m < mg) {
          const i32x4_t v = acc[t][mt];
          const f32x4_t f = {(float)v.x, (float)v.y, (float)v.z, (float)v.w};
          store_out4(a.y, a.ldy, a.out_f32, a.vec_out, m0 + m, n, min(4, a.N - n), (f * a.s_tok[m0 + m]) * sc);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// W8A8 LDS-tiled kernel (QF_KERNEL_MFMA_W8A8_TILE): large M, either weight layout.
//
// A workgroup of 8 wavefronts owns a 256-channel x 256-token output tile over the whole K range.  Each
// 64-k step stages 32 fragments of 1 KiB in LDS: the 16 weight tiles (16 channels x 64 k: the TILED
// block as stored, or on row-major weights lane (g, r) reading row r, bytes 16 g .. 16 g + 15 of the
// step) and the 16 activation tiles of 16 tokens (lane (g, r): token r, k 16 g .. 16 g + 15).  Each is
// copied global -> LDS with one 16-byte-per-lane direct-to-LDS load, lane l's bytes landing at 16 l, so
// a fragment read is one conflict-free ds_read_b128 and no VGPR holds staged data.  The stages go
// through a ring of kW8A8TileStages slots; each iteration waits for its own copies of the next stage,
// meets the other wavefronts at one barrier, refills the slot all of them finished reading, reads the
// next step's 12 fragments and runs this step's 32 MFMAs.
// Wavefront (wn, wm) = (wave & 1, wave >> 1) computes channels 128 wn .. +127 and tokens 64 wm .. +63:
// 8 weight fragments (the A operand of v_mfma_i32_16x16x64_i8) by 4 activation fragments (B), 128
// int32 accumulators.  Integer sums are exact in any order, so results equal the other W8A8 kernels'.
// Per step and CU: 32 KiB copied, 96 KiB of fragment reads, 256 MFMAs (measured best of 3, 4 and 5
// stages at 4; 3 leaves the copies exposed).
// The bf16 epilogue stages each wavefront's 64 x 128 block in its own 16 KiB of LDS and stores whole
// 256-byte row pieces (the MFMA layout alone would store 16 rows x 32 bytes per instruction: gate_up
// M = 2048 406 -> 379 us); fp32 output or rows without 16-byte alignment store from the registers.
// ---------------------------------------------------------------------------------------------
typedef const void __attribute__((address_space(1)))* glb_ptr_t;
typedef void __attribute__((address_space(3)))* lds_ptr_t;

constexpr int kW8A8TileStages = 4;
constexpr int kW8A8TileRows = 256;                        // tokens per workgroup
constexpr int kW8A8TileTiles = 16;                        // 16-channel weight tiles per workgroup
constexpr int kW8A8TileStageBytes = 32 * 1024;            // 16 weight + 16 activation fragments
constexpr int kW8A8TileLds = kW8A8TileStages * kW8A8TileStageBytes;
constexpr int kW8A8TileMaxSplit = 8;                      // K splits of the tile kernel (fused reduction)

// s_waitcnt with vmcnt = n (0..63) and the other counters unconstrained.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// Workgroup tile shapes: FA weight fragments by FB activation fragments a wavefront, 8 wavefronts in 2
// channel x 4 token groups, so 32 FA channels x 64 FB tokens a workgroup: (8, 4) is the 256 x 256 main
// shape, (4, 2) the 128 x 128 shape that runs the channels past the main grid's whole rounds, (8, 2) the
// 256-channel x 128-token shape of reduce 3.  A stage's fragments, weights first, are spread evenly over
// the 8 wavefronts.
template <int FA, int FB_ = FA / 2>
struct TileShape {
  static constexpr int FB = FB_;
  static constexpr int tiles = 2 * FA;            // 16-channel weight tiles a workgroup
  static constexpr int frags = 4 * FB;            // 16-token activation fragments a workgroup
  static constexpr int rows = 16 * frags;         // tokens a workgroup
  static constexpr int copies = (tiles + frags) / 8;  // fragments a wavefront copies a stage
  static_assert((tiles + frags) % 8 == 0, "the stage's fragments spread evenly over the 8 wavefronts");
  static constexpr int stage_bytes = (tiles + frags) * 1024;
  // 4 stages for the main shape; 6 for the small one, which also keeps it at one workgroup a CU
  // (96 KiB), so that a grid of 256 spreads over all CUs.
  static constexpr int stages = FA == 8 ? kW8A8TileStages : 6;
  static constexpr int lds = stages * stage_bytes;
};

template <int LAYOUT, int FA, int FB_ = FA / 2>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
    w8a8_tile_kernel(const GemmArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ int last_arrival;
  using T = TileShape<FA, FB_>;
  constexpr int FB = T::FB;
  constexpr int S = T::stages;
  constexpr int CP = T::copies;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wn = wave & 1, wm = wave >> 1;
  const int g = lane >> 4, r = lane & 15;
  const int ntiles = a.n_pad / kTileN;
  const int mblocks = (a.M + T::rows - 1) / T::rows;
  // The hardware hands workgroup i to XCD i % kXcds; consecutive logical blocks share an XCD, so the
  // token blocks of one channel block run together and share its weights in that XCD's L2.
  int l = xcd_major(blockIdx.x, gridDim.x);
  // split_k > 1: the grid is split_k copies of the tile grid, copy `split` computing k-steps
  // [s_begin, s_end) of every tile.
  const int tiles_grid = gridDim.x / a.split_k;
  const int split = l / tiles_grid;
  l -= split * tiles_grid;
  int s_begin = 0, s_end = a.ksteps;
  if (a.split_k > 1) split_range(split, a.split_k, a.ksteps, s_begin, s_end);
  const int nsteps = s_end - s_begin;  // >= 1: split_k <= ksteps
  const int tile0 = (l / mblocks) * T::tiles;
  const int m0 = (l % mblocks) * T::rows;
  const int ksteps = a.ksteps;

  // Wavefront w copies fragments CP w .. CP w + CP - 1 of the stage: the T::tiles weight fragments first, then
  // the T::frags activation fragments.  Channels and tokens past the matrix read its last row (block) instead;
  // their outputs are never stored.
  const int8_t* src[CP];
  int64_t adv[CP];  // bytes between the same fragment of consecutive steps
  auto weight_src = [&](int f) -> const int8_t* {
    const int t = min(tile0 + f, ntiles - 1);
    if constexpr (LAYOUT == QF_LAYOUT_ROWMAJOR) return a.w + (int64_t)min(t * kTileN + r, a.N - 1) * a.ldw + 16 * g;
    return a.w + ((int64_t)t * ksteps * kWave + lane) * 16;
  };
  auto act_src = [&](int i) -> const int8_t* {  // activation fragment i of the workgroup
    if (a.x_tiled) {  // one contiguous KiB per fragment, as the TILED weights
      const int b = min((m0 >> 4) + i, (a.M - 1) >> 4);
      return a.xq + ((int64_t)b * ksteps * kWave + lane) * 16;
    }
    const int row = min(m0 + 16 * i + r, a.M - 1);
    return a.xq + (int64_t)row * a.ldx + 16 * g;
  };
  const int64_t w_adv = LAYOUT == QF_LAYOUT_ROWMAJOR ? kStepK : kTileN * kStepK;
  const int64_t x_adv = a.x_tiled ? kTileN * kStepK : kStepK;
  if constexpr (T::tiles == 4 * CP) {
    // Wavefronts 0..3 copy weights, 4..7 activations: one stride a wavefront (the 256 x 256 and 128 x 128
    // shapes; the per-fragment form below measured 0.5-3% slower on them).
    const int64_t wa = wave < 4 ? w_adv : x_adv;
#pragma unroll
    for (int j = 0; j < CP; ++j) {
      src[j] = wave < 4 ? weight_src(CP * wave + j) : act_src(CP * (wave - 4) + j);
      adv[j] = wa;
    }
  } else {
#pragma unroll
    for (int j = 0; j < CP; ++j) {
      const int f = CP * wave + j;  // uniform
      src[j] = f < T::tiles ? weight_src(f) : act_src(f - T::tiles);
      adv[j] = f < T::tiles ? w_adv : x_adv;
    }
  }
#pragma unroll
  for (int j = 0; j < CP; ++j) src[j] += (int64_t)s_begin * adv[j];
  // Copy group s: stage min(s, ksteps - 1) into slot s % S.  Groups past the last stage copy it again
  // into a slot whose stage every wavefront has consumed, so every iteration issues exactly one group
  // and the vmcnt waits are constants.
  auto copy = [&](int s) {
    uint8_t* slot = smem + (s % S) * T::stage_bytes + wave * CP * 1024;
    const int64_t st = min(s, nsteps - 1);
#pragma unroll
    for (int j = 0; j < CP; ++j)
      __builtin_amdgcn_global_load_lds((glb_ptr_t)(src[j] + st * adv[j]), (lds_ptr_t)(slot + j * 1024), 16, 0, 0);
  };
  auto read_frags = [&](int s, i32x4_t (&A)[FA], i32x4_t (&B)[FB]) {
    const uint8_t* slot = smem + (s % S) * T::stage_bytes + lane * 16;
#pragma unroll
    for (int i = 0; i < FA; ++i) A[i] = *reinterpret_cast<const i32x4_t*>(slot + (FA * wn + i) * 1024);
#pragma unroll
    for (int i = 0; i < FB; ++i) B[i] = *reinterpret_cast<const i32x4_t*>(slot + (T::tiles + FB * wm + i) * 1024);
  };
  // The ring barrier: every wavefront has waited for its own copies of the stage before it; the acquire
  // keeps the stage's reads after it.  (A release fence would wait for the copies still in flight, which
  // count as LDS writes.)
  auto ring_barrier = []() {
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  };

  i32x4_t acc[FA][FB];
#pragma unroll
  for (int i = 0; i < FA; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j) acc[i][j] = (i32x4_t){0, 0, 0, 0};

#pragma unroll
  for (int s = 0; s < S - 1; ++s) copy(s);
  wait_vmcnt<CP * (S - 2)>();  // groups 1 .. S - 2 may still be in flight: stage 0 has landed
  ring_barrier();
  i32x4_t fa[FA], fb[FB], ga[FA], gb[FB];
  read_frags(0, fa, fb);
  // Step s: stage s + 1 becomes readable at the barrier (S - 3 groups were issued after its group), the
  // slot of stage s - 1 is refilled with group s + S - 1, the fragments of step s + 1 are read into
  // (na, nb) while the MFMAs of step s run on (ca, cb).  Unrolled by two so the fragment sets alternate
  // without copies.
  auto step = [&](int s, i32x4_t (&ca)[FA], i32x4_t (&cb)[FB], i32x4_t (&na)[FA], i32x4_t (&nb)[FB]) {
    wait_vmcnt<CP * (S - 3)>();
    ring_barrier();
    copy(s + S - 1);
    read_frags(min(s + 1, nsteps - 1), na, nb);
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
      for (int j = 0; j < FB; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ca[i], cb[j], acc[i][j], 0, 0, 0);
  };
  int s = 0;
  for (; s + 1 < nsteps; s += 2) {
    step(s, fa, fb, ga, gb);
    step(s + 1, ga, gb, fa, fb);
  }
  if (s < nsteps) step(s, fa, fb, ga, gb);
  wait_vmcnt<0>();  // the last groups' copies have landed before LDS is reused or released

  if (a.split_k > 1) {
    // The splits of a tile meet through the workspace: each stores its int32 accumulators lane for lane
    // (wavefront w's block of FA x FB fragments at slot (tile, split, w)) with device-scope stores and
    // waits for them to complete; then one thread counts the arrival.  The last split to arrive reads the
    // others' slots with device-scope loads, issued after its increment returned, adds them (exact in any
    // order) and runs the epilogue; it returns the counter to zero.  The ordering is the hardware's, as in
    // the decode kernel's fused split-K.
    // A fragment's slot is 1 KiB: the lanes' (x, y) words in its first 512 bytes, their (z, w) words in the
    // second, so each 8-byte-a-lane store or load covers 512 contiguous bytes (a 16-byte lane stride, half
    // of every line per instruction: down 5120 x 17408 at M = 1024 in 3 splits 122.1 against 113.2 us).
    // Plain stores with an agent-scope release fence and an acquire fence on the last arrival (an L2
    // write-back and invalidate each) measured far slower: 157.6 us.
    constexpr int kSlot = FA * FB * kWave * 4;  // int32 a wavefront
    uint64_t* const tile_slots = reinterpret_cast<uint64_t*>(a.partial) + (int64_t)l * a.split_k * 8 * (kSlot / 2);
    {
      uint64_t* mine = tile_slots + ((int64_t)split * 8 + wave) * (kSlot / 2) + lane;
#pragma unroll
      for (int i = 0; i < FA; ++i)
#pragma unroll
        for (int j = 0; j < FB; ++j) {
          uint64_t* p = mine + (i * FB + j) * 2 * kWave;
          const i32x4_t v = acc[i][j];
          __hip_atomic_store(p, (uint64_t)(uint32_t)v.x | ((uint64_t)(uint32_t)v.y << 32), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(p + kWave, (uint64_t)(uint32_t)v.z | ((uint64_t)(uint32_t)v.w << 32),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    if (threadIdx.x == 0) {
      const unsigned prev =
          __hip_atomic_fetch_add(a.counters + l * a.counter_stride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last_arrival = prev == (unsigned)(a.split_k - 1);
    }
    __syncthreads();
    if (!last_arrival) return;
    for (int o = 0; o < a.split_k; ++o) {
      if (o == split) continue;
      const uint64_t* theirs = tile_slots + ((int64_t)o * 8 + wave) * (kSlot / 2) + lane;
#pragma unroll
      for (int i = 0; i < FA; ++i)
#pragma unroll
        for (int j = 0; j < FB; ++j) {
          const uint64_t* p = theirs + (i * FB + j) * 2 * kWave;
          const uint64_t lo = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          const uint64_t hi = __hip_atomic_load(p + kWave, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          acc[i][j] += (i32x4_t){(int)(uint32_t)lo, (int)(uint32_t)(lo >> 32), (int)(uint32_t)hi,
                                 (int)(uint32_t)(hi >> 32)};
        }
    }
    if (threadIdx.x == 0)
      __hip_atomic_store(a.counters + l * a.counter_stride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // Lane (g, r) holds C[n = 16 (tile0 + FA wn + i) + 4 g + e][m = m0 + 16 FB wm + 16 j + r], e = 0..3.
  const bool staged = !a.out_f32 && a.vec_out && (a.ldy % 8) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0;
  if (staged) {
    // Each wavefront's 16 FB x 16 FA bf16 block goes to its own LDS: token row t (NC 16-byte chunks), chunk
    // c at t * 16 NC + ((c ^ (t % NC)) << 4), so the 8-byte writes and 16-byte reads spread over the banks.
    constexpr int NC = 2 * FA;                 // 16-byte chunks a token row
    constexpr int BLK = 16 * FB * 16 * NC;     // bytes a wavefront
    static_assert(8 * BLK <= T::lds, "epilogue staging fits the ring");
    __syncthreads();  // every wavefront is done with the ring
    uint8_t* blk = smem + wave * BLK;
#pragma unroll
    for (int i = 0; i < FA; ++i) {
      const int n = (tile0 + FA * wn + i) * kTileN + 4 * g;
      const f32x4_t sc = load_scale4(a.scale, a.N, min(n, a.n_pad - 4));
#pragma unroll
      for (int j = 0; j < FB; ++j) {
        const int t = 16 * j + r;
        const float st = a.s_tok[min(m0 + 16 * FB * wm + t, a.M - 1)];
        const i32x4_t v = acc[i][j];
        const f32x4_t f = {(float)v.x, (float)v.y, (float)v.z, (float)v.w};
        const f32x4_t o = (f * st) * sc;
        u32x2_t p;
        p.x = pack_bf16_rne(o.x, o.y);
        p.y = pack_bf16_rne(o.z, o.w);
        const int c = 2 * i + (g >> 1);
        *reinterpret_cast<u32x2_t*>(blk + t * 16 * NC + ((c ^ (t % NC)) << 4) + 8 * (g & 1)) = p;
      }
    }
    const int c = lane % NC;
    const int n0 = (tile0 + FA * wn) * kTileN + 8 * c;  // the first of this lane's 8 channels
#pragma unroll
    for (int q = 0; q < 16 * FB * NC / kWave; ++q) {
      const int t = (kWave / NC) * q + lane / NC;
      const int m = m0 + 16 * FB * wm + t;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(blk + t * 16 * NC + ((c ^ (t % NC)) << 4));
      if (m < a.M) {
        uint16_t* row = reinterpret_cast<uint16_t*>(a.y) + (int64_t)m * a.ldy + n0;
        if (n0 + 8 <= a.N) {
          *reinterpret_cast<u32x4_t*>(row) = v;
        } else if (n0 < a.N) {
          const int cnt = a.N - n0;  // 1 .. 7
#pragma unroll
          for (int k = 0; k < 8; ++k) {  // constant element indices: v stays in registers
            if (k < cnt) row[k] = (uint16_t)(v[k >> 1] >> (16 * (k & 1)));
          }
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < FA; ++i) {
    const int tile = tile0 + FA * wn + i;
    const int n = tile * kTileN + 4 * g;
    if (tile < ntiles && n < a.N) {
      const f32x4_t sc = load_scale4(a.scale, a.N, n);
#pragma unroll
      for (int j = 0; j < FB; ++j) {
        const int m = m0 + 16 * FB * wm + 16 * j + r;
        if (m < a.M) {
          const i32x4_t v = acc[i][j];
          const f32x4_t f = {(float)v.x, (float)v.y, (float)v.z, (float)v.w};
          store_out4(a.y, a.ldy, a.out_f32, a.vec_out, m, n, min(4, a.N - n), (f * a.s_tok[m]) * sc);
        }
      }
    }
  }
}

// Sum of the W8A8 kernel's int32 split partials (exact in any order), then the scales.
__global__ void __launch_bounds__(256) splitk_reduce_w8a8_kernel(const GemmArgs a) {
  const int groups = a.n_pad / 4;
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.M * groups) return;
  const int m = idx / groups;
  const int n = (idx - m * groups) * 4;
  if (n >= a.N) return;
  const int64_t plane = (int64_t)a.M * a.n_pad;
  const int32_t* p = reinterpret_cast<const int32_t*>(a.partial) + (int64_t)m * a.n_pad + n;
  i32x4_t sum = *reinterpret_cast<const i32x4_t*>(p);
  for (int j = 1; j < a.split_k; ++j) sum += *reinterpret_cast<const i32x4_t*>(p + j * plane);
  const f32x4_t f = {(float)sum.x, (float)sum.y, (float)sum.z, (float)sum.w};
  const f32x4_t sc = load_scale4(a.scale, a.N, n);
  store_out4(a.y, a.ldy, a.out_f32, a.vec_out, m, n, min(4, a.N - n), (f * a.s_tok[m]) * sc);
}

// ---------------------------------------------------------------------------------------------
// GEMV kernel (wavefront reduction), row-major layout, M = MM <= 4.
//
// Workgroup = WAVES wavefronts; wavefront w owns RPW consecutive rows; blockIdx.y is the K split.
// x[0:MM][k-range] is staged in LDS row-major (bf16).  Each step covers 1024 k: lane l loads
// k0 + 16 l .. +15 of each of its RPW rows and reads the matching 32 bytes of each x row.
// ---------------------------------------------------------------------------------------------
template <int MM, int RPW, int WAVES, bool NTH>
__global__ void __launch_bounds__(WAVES * kWave) w8a16_gemv_kernel(const GemmArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int split = blockIdx.y;
  int s_begin, s_end;
  split_range(split, a.split_k, a.ksteps, s_begin, s_end);
  const int klen = (s_end - s_begin) * kStepK;
  const int64_t kb = (int64_t)s_begin * kStepK;
  const int row0 = (blockIdx.x * WAVES + wave) * RPW;
  const bool wave_active = row0 < a.N;

  // Stage x rows (klen bf16 each) into LDS, row m at byte m * klen * 2.
  {
    const int per_row = klen / 8;
    for (int m = 0; m < MM; ++m) {
      for (int c = threadIdx.x; c < per_row; c += WAVES * kWave) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(a.x + (int64_t)m * a.ldx + kb + c * 8);
        *reinterpret_cast<u32x4_t*>(smem + ((size_t)m * klen + c * 8) * 2) = v;
      }
    }
  }
  __syncthreads();
  if (!wave_active) return;

  const int8_t* wrow[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int row = min(row0 + i, a.N - 1);
    wrow[i] = a.w + (int64_t)row * a.ldw + kb + lane * 16;
  }

  float acc[RPW][MM];
#pragma unroll
  for (int i = 0; i < RPW; ++i)
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[i][m] = 0.f;

  const int nq = (klen + 1023) / 1024;
  u32x4_t cur[RPW];
  if (lane * 16 < klen) {
#pragma unroll
    for (int i = 0; i < RPW; ++i) cur[i] = load16<NTH>(wrow[i]);
  }
  for (int q = 0; q < nq; ++q) {
    const int kofs = q * 1024 + lane * 16;
    if (kofs >= klen) break;
    u32x4_t nxt[RPW];
    const bool more = kofs + 1024 < klen;
    if (more) {
#pragma unroll
      for (int i = 0; i < RPW; ++i) nxt[i] = load16<NTH>(wrow[i] + (int64_t)(q + 1) * 1024);
    }
    // activations for k = kofs .. kofs+15 as fp32
    float xf[MM][16];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      const u32x4_t* p = reinterpret_cast<const u32x4_t*>(smem + ((size_t)m * klen + kofs) * 2);
      const u32x4_t h0 = p[0], h1 = p[1];
      const uint32_t hw[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        xf[m][2 * j] = __uint_as_float(hw[j] << 16);
        xf[m][2 * j + 1] = __uint_as_float(hw[j] & 0xffff0000u);
      }
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const uint32_t wd[4] = {cur[i].x, cur[i].y, cur[i].z, cur[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int32_t s = (int32_t)wd[j];
        const float wf[4] = {(float)(int8_t)(s & 0xff), (float)(int8_t)((s >> 8) & 0xff),
                             (float)(int8_t)((s >> 16) & 0xff), (float)(s >> 24)};
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int m = 0; m < MM; ++m) acc[i][m] = __builtin_fmaf(wf[b], xf[m][4 * j + b], acc[i][m]);
      }
    }
    if (more) {
#pragma unroll
      for (int i = 0; i < RPW; ++i) cur[i] = nxt[i];
    }
  }

  // Butterfly reduction across the 64 lanes (fixed pattern: deterministic).
#pragma unroll
  for (int i = 0; i < RPW; ++i)
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      float v = acc[i][m];
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
      acc[i][m] = v;
    }

  // Lane i*MM + m writes row row0+i, token m.
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      if (lane == i * MM + m) {
        const int n = row0 + i;
        if (n < a.N) {
          if (a.split_k == 1) {
            const float v = acc[i][m] * a.scale[n];
            if (a.out_f32)
              reinterpret_cast<float*>(a.y)[(int64_t)m * a.ldy + n] = v;
            else
              reinterpret_cast<uint16_t*>(a.y)[(int64_t)m * a.ldy + n] = bf16_rne(v);
          } else {
            a.partial[((int64_t)split * MM + m) * a.n_pad + n] = acc[i][m];
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Split-K second pass: y[m, n..n+3] = round(s[n] * sum_{j=0..SK-1} P[j][m][n]), summed in j order.
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const GemmArgs a) {
  const int groups = a.n_pad / 4;
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.M * groups) return;
  const int m = idx / groups;
  const int n = (idx - m * groups) * 4;
  if (n >= a.N) return;
  const int64_t plane = (int64_t)a.M * a.n_pad;
  const float* p = a.partial + (int64_t)m * a.n_pad + n;
  f32x4_t sum = *reinterpret_cast<const f32x4_t*>(p);
  for (int j = 1; j < a.split_k; ++j) sum += *reinterpret_cast<const f32x4_t*>(p + j * plane);
  const f32x4_t sc = load_scale4(a.scale, a.N, n);
  store_out4(a.y, a.ldy, a.out_f32, a.vec_out, m, n, min(4, a.N - n), sum * sc);
}

// ---------------------------------------------------------------------------------------------
// Layout change: row-major [N, K] <-> TILED.  One thread per 16-byte piece of the tiled image:
// piece p = (tile * ksteps + s) * 64 + l holds row tile*16 + (l % 16), k = s*64 + 16*(l / 16).
// ---------------------------------------------------------------------------------------------
template <bool kUnpack>
__global__ void __launch_bounds__(256) repack_kernel(const int8_t* src, int8_t* dst, int64_t ldw, int N,
                                                     int ksteps, int64_t pieces) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= pieces) return;
  const int l = (int)(p & 63);
  const int64_t ts = p >> 6;
  const int s = (int)(ts % ksteps);
  const int64_t tile = ts / ksteps;
  const int64_t row = tile * kTileN + (l & 15);
  const int64_t col = (int64_t)s * kStepK + 16 * (l >> 4);
  if constexpr (!kUnpack) {
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (row < N) v = *reinterpret_cast<const u32x4_t*>(src + row * ldw + col);
    *reinterpret_cast<u32x4_t*>(dst + p * 16) = v;
  } else {
    if (row < N) {
      *reinterpret_cast<u32x4_t*>(dst + row * ldw + col) = *reinterpret_cast<const u32x4_t*>(src + p * 16);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Exact int8 -> bf16 copy of weight rows [n0, n0 + rows) into a row-major bf16 matrix (row stride
// ldo), from either layout: the operand of a library bf16 GEMM for M beyond the wide-M kernel's
// range.  The scale is not applied (it follows the K reduction).
//
// Row-major: one thread per 16 weights of a row, a 16-byte read and a 32-byte write, both
// contiguous across the wavefront.
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) dequant_rows_kernel(const int8_t* w, int64_t ldw, int ksteps, int n0,
                                                           int64_t pieces, uint16_t* out, int64_t ldo) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= pieces) return;
  const int kp = ksteps * 4;  // 16-weight pieces per row
  const int64_t r = q / kp;   // output row
  const int c = (int)(q - r * kp);
  bf16x8_t a0, a1;
  dequant16(*reinterpret_cast<const u32x4_t*>(w + (n0 + r) * ldw + c * 16), a0, a1);
  u32x4_t* dst = reinterpret_cast<u32x4_t*>(out + r * ldo + c * 16);
  dst[0] = __builtin_bit_cast(u32x4_t, a0);
  dst[1] = __builtin_bit_cast(u32x4_t, a1);
}

// TILED: a workgroup reads 4 consecutive KiB of the image, k-steps 4 kg .. 4 kg + 3 of one 16-row
// tile (thread t: step 4 kg + t / 64, lane t % 64 = row t % 16, k piece t / 16 % 4), and writes 512
// contiguous bytes of each of the tile's rows.  Reading the image in order, instead of gathering
// each output row's pieces from 16 lanes apart, doubles the copy rate (the whole gate_up image,
// 34816 x 5120: 107 us against 222 us).
__global__ void __launch_bounds__(256) dequant_tiled_kernel(const int8_t* w, int ksteps, int n0, int rows,
                                                            int kgroups, uint16_t* out, int64_t ldo) {
  const int tile = n0 / kTileN + (int)(blockIdx.x / kgroups);
  const int kg = (int)(blockIdx.x % kgroups);
  const int lane = threadIdx.x & (kWave - 1);
  const int ks = kg * 4 + (int)(threadIdx.x / kWave);
  const int n = tile * kTileN + (lane & 15);
  if (ks >= ksteps || n < n0 || n >= n0 + rows) return;
  bf16x8_t a0, a1;
  dequant16(*reinterpret_cast<const u32x4_t*>(w + (((int64_t)tile * ksteps + ks) * kWave + lane) * 16), a0, a1);
  u32x4_t* dst = reinterpret_cast<u32x4_t*>(out + (int64_t)(n - n0) * ldo + (ks * 4 + (lane >> 4)) * 16);
  dst[0] = __builtin_bit_cast(u32x4_t, a0);
  dst[1] = __builtin_bit_cast(u32x4_t, a1);
}

// y[m, n] = bf16_rne(acc[m, n] * scale[n]): the epilogue of the library GEMM on widened weights (its
// fp32 output, scaled after the K reduction).  One thread per 8 outputs of a row: two 16-byte reads
// of acc and of the scale, one 16-byte write; `vec` is false when a pointer or a row stride breaks
// that alignment, and then every element is handled on its own.
__global__ void __launch_bounds__(256) scale_cast_kernel(const float* acc, int64_t lda, const float* scale, int M,
                                                         int N, int cpr, uint16_t* y, int64_t ldy, int vec) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= (int64_t)M * cpr) return;
  const int m = (int)(q / cpr);
  const int n = (int)(q - (int64_t)m * cpr) * 8;
  const float* a = acc + m * lda + n;
  uint16_t* o = y + m * ldy + n;
  if (vec && n + 8 <= N) {
    const f32x4_t a0 = *reinterpret_cast<const f32x4_t*>(a), a1 = *reinterpret_cast<const f32x4_t*>(a + 4);
    const f32x4_t s0 = *reinterpret_cast<const f32x4_t*>(scale + n);
    const f32x4_t s1 = *reinterpret_cast<const f32x4_t*>(scale + n + 4);
    u32x4_t v;
    v.x = pack_bf16_rne(a0.x * s0.x, a0.y * s0.y);
    v.y = pack_bf16_rne(a0.z * s0.z, a0.w * s0.w);
    v.z = pack_bf16_rne(a1.x * s1.x, a1.y * s1.y);
    v.w = pack_bf16_rne(a1.z * s1.z, a1.w * s1.w);
    *reinterpret_cast<u32x4_t*>(o) = v;
  } else {
    for (int i = 0; i < 8 && n + i < N; ++i) o[i] = bf16_rne(a[i] * scale[n + i]);
  }
}

// ---------------------------------------------------------------------------------------------
// Draft-head per-row int8 quantiser (plugin/qwen_fastpath/patches.py:139-147).  One workgroup per
// row.  s = max(amax, 1e-8) * fl(1/127): the reference divides a CUDA tensor by the Python scalar
// 127.0, which PyTorch evaluates as a multiply by the fp32 reciprocal; w / s is an IEEE division.
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) quantize_rows_kernel(const uint16_t* w, int64_t ldw, int8_t* q,
                                                            float* s_out, int H) {
  __shared__ float red[256 / kWave];
  const int64_t v = blockIdx.x;
  const uint16_t* row = w + v * ldw;
  float amax = 0.f;
  for (int h = threadIdx.x; h < H; h += 256) amax = fmaxf(amax, fabsf(__uint_as_float((uint32_t)row[h] << 16)));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int i = 1; i < 256 / kWave; ++i) amax = fmaxf(amax, red[i]);
  const float inv127 = 1.0f / 127.0f;  // constant-folded: the fp32 reciprocal of 127
  const float s = fmaxf(amax, 1e-8f) * inv127;
  if (threadIdx.x == 0) s_out[v] = s;
  int8_t* qrow = q + v * (int64_t)H;
  for (int h = threadIdx.x; h < H; h += 256) {
    const float x = __uint_as_float((uint32_t)row[h] << 16);
    float t = rintf(__fdiv_rn(x, s));
    t = fminf(fmaxf(t, -127.f), 127.f);
    qrow[h] = (int8_t)(int)t;
  }
}

// The same quantiser for 16-byte-aligned rows with H % 8 == 0 and H <= 8 * kQuantThreads * kQuantChunks:
// each thread keeps its 16-byte pieces (8 values) of the row in registers, so the row is read once
// with 16-byte loads and written with 8-byte stores; the per-value arithmetic is the one above, so
// the results are bit-identical.
constexpr int kQuantThreads = 128;
constexpr int kQuantChunks = 8;

__global__ void __launch_bounds__(kQuantThreads) quantize_rows_vec_kernel(const uint16_t* w, int64_t ldw, int8_t* q,
                                                                          float* s_out, int H) {
  __shared__ float red[kQuantThreads / kWave];
  const int64_t v = blockIdx.x;
  const u32x4_t* row = reinterpret_cast<const u32x4_t*>(w + v * ldw);
  const int nch = H / 8;
  u32x4_t x[kQuantChunks];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < kQuantChunks; ++j) {
    const int c = j * kQuantThreads + (int)threadIdx.x;
    x[j] = c < nch ? row[c] : u32x4_t{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int j = 0; j < kQuantChunks; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      amax = fmaxf(amax, fmaxf(fabsf(__uint_as_float(x[j][i] << 16)), fabsf(__uint_as_float(x[j][i] & 0xffff0000u))));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int i = 1; i < kQuantThreads / kWave; ++i) amax = fmaxf(amax, red[i]);
  const float inv127 = 1.0f / 127.0f;  // constant-folded: the fp32 reciprocal of 127
  const float s = fmaxf(amax, 1e-8f) * inv127;
  if (threadIdx.x == 0) s_out[v] = s;
  u32x2_t* qrow = reinterpret_cast<u32x2_t*>(q + v * (int64_t)H);
  auto quant = [&](float xv) {
    const float t = fminf(fmaxf(rintf(__fdiv_rn(xv, s)), -127.f), 127.f);
    return (uint32_t)(uint8_t)(int8_t)(int)t;
  };
#pragma unroll
  for (int j = 0; j < kQuantChunks; ++j) {
    const int c = j * kQuantThreads + (int)threadIdx.x;
    if (c < nch) {
      uint32_t b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t lo = x[j][2 * i], hi = x[j][2 * i + 1];
        b[i] = quant(__uint_as_float(lo << 16)) | (quant(__uint_as_float(lo & 0xffff0000u)) << 8) |
               (quant(__uint_as_float(hi << 16)) << 16) | (quant(__uint_as_float(hi & 0xffff0000u)) << 24);
      }
      qrow[c] = u32x2_t{b[0], b[1]};
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Row argmax over bf16 logits (torch.argmax semantics: NaN is the maximum, first index on ties).
// One workgroup per row.
// ---------------------------------------------------------------------------------------------
constexpr int kArgmaxThreads = 1024;

// One workgroup of 1024 threads per row.  With VEC each thread reads 8 logits per 16-byte load,
// four loads in flight, and walks each group in index order; the row tail (n_valid % 8) and
// unaligned rows are read one logit at a time.  The workgroup reduction is a fixed butterfly plus an
// LDS tree, so the result does not depend on timing; argmax_better makes it order-independent anyway.
template <bool VEC>
__global__ void __launch_bounds__(kArgmaxThreads) argmax_rows_kernel(const uint16_t* logits, int64_t ld, int n_valid,
                                                                     int64_t index_offset, int64_t* out) {
  __shared__ float sv[kArgmaxThreads / kWave];
  __shared__ int si[kArgmaxThreads / kWave];
  const uint16_t* row = logits + (int64_t)blockIdx.x * ld;
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  int scalar_from = 0;
  if constexpr (VEC) {
    const int nvec = n_valid / 8;
    const u32x4_t* vrow = reinterpret_cast<const u32x4_t*>(row);
    auto fold8 = [&](const u32x4_t v, int c) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t d = v[j];
        argmax_fold(__uint_as_float(d << 16), c * 8 + 2 * j, bv, bi);
        argmax_fold(__uint_as_float(d & 0xffff0000u), c * 8 + 2 * j + 1, bv, bi);
      }
    };
    int c = threadIdx.x;
    for (; c + 3 * kArgmaxThreads < nvec; c += 4 * kArgmaxThreads) {
      const u32x4_t v0 = vrow[c];
      const u32x4_t v1 = vrow[c + kArgmaxThreads];
      const u32x4_t v2 = vrow[c + 2 * kArgmaxThreads];
      const u32x4_t v3 = vrow[c + 3 * kArgmaxThreads];
      fold8(v0, c);
      fold8(v1, c + kArgmaxThreads);
      fold8(v2, c + 2 * kArgmaxThreads);
      fold8(v3, c + 3 * kArgmaxThreads);
    }
    for (; c < nvec; c += kArgmaxThreads) fold8(vrow[c], c);
    scalar_from = nvec * 8;
  }
  for (int n = scalar_from + threadIdx.x; n < n_valid; n += kArgmaxThreads)
    argmax_fold(__uint_as_float((uint32_t)row[n] << 16), n, bv, bi);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off, kWave);
    const int oi = __shfl_xor(bi, off, kWave);
    argmax_fold(ov, oi, bv, bi);
  }
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgmaxThreads / kWave; ++w) argmax_fold(sv[w], si[w], bv, bi);
    // every column -inf (or no valid column): torch.argmax returns the first index
    const int idx = (bi == 0x7fffffff) ? 0 : bi;
    out[blockIdx.x] = (int64_t)idx + index_offset;
  }
}

// Row split over workgroups: for rows of many logits (the draft head's 151936) one workgroup per
// row is bound by the latency of its own loads, so each row is cut into chunks of kArgmaxChunk
// logits, one 256-thread workgroup each (grid = chunks x rows).  A workgroup writes its candidate (value,
// index) with device-scope stores into a small device-resident table, waits for them, and counts
// its arrival on the row's counter; the last workgroup of the row folds all candidates (the order
// is total -- value, then index, NaN highest -- so the fold does not depend on arrival order),
// writes the index and resets the counter to zero.  The table is either the library's device-resident
// one (qf_argmax_rows_bf16: calls that overlap on one device share it and must not run at the same
// time) or the caller's workspace (qf_argmax_rows_bf16_ws: one workspace per stream).
constexpr int kArgmaxSplitThreads = 256;
constexpr int kArgmaxChunk = 8192;            // logits per workgroup (16 KiB)
constexpr int kArgmaxMaxBlocks = 64;          // chunks per row
constexpr int kArgmaxMaxRows = QF_W8A16_MAX_M;
__device__ float g_argmax_val[kArgmaxMaxRows * kArgmaxMaxBlocks];
__device__ int g_argmax_idx[kArgmaxMaxRows * kArgmaxMaxBlocks];
__device__ unsigned g_argmax_arrivals[kArgmaxMaxRows];

// Candidate table of the row-split argmax in a caller workspace: the per-row arrival counters at the
// front of the counter prefix (zero on entry, returned to zero), the (value, index) pairs after it.
struct ArgmaxTable {
  float* val;
  int* idx;
  unsigned* arrivals;
};
constexpr size_t kArgmaxTableBytes = (size_t)kArgmaxMaxRows * kArgmaxMaxBlocks * (sizeof(float) + sizeof(int));

__device__ __forceinline__ void argmax_block_reduce(float& bv, int& bi, float* sv, int* si) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off, kWave);
    const int oi = __shfl_xor(bi, off, kWave);
    argmax_fold(ov, oi, bv, bi);
  }
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x / kWave); ++w) argmax_fold(sv[w], si[w], bv, bi);
  }
}

template <bool kOwnTable>
__global__ void __launch_bounds__(kArgmaxSplitThreads) argmax_rows_split_kernel(const uint16_t* logits, int64_t ld,
                                                                                int n_valid, int64_t index_offset,
                                                                                int64_t* out, ArgmaxTable tab) {
  float* const tval = kOwnTable ? g_argmax_val : tab.val;
  int* const tidx = kOwnTable ? g_argmax_idx : tab.idx;
  unsigned* const tarr = kOwnTable ? g_argmax_arrivals : tab.arrivals;
  __shared__ float sv[kArgmaxSplitThreads / kWave];
  __shared__ int si[kArgmaxSplitThreads / kWave];
  __shared__ int last;
  const int m = blockIdx.y;
  const int b = blockIdx.x;
  const int nb = gridDim.x;
  const uint16_t* row = logits + (int64_t)m * ld;
  const int c0 = b * (kArgmaxChunk / 8);                        // first 8-logit group of the chunk
  const int c1 = min(c0 + kArgmaxChunk / 8, n_valid / 8);
  const u32x4_t* vrow = reinterpret_cast<const u32x4_t*>(row);
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  int c = c0 + threadIdx.x;
  for (; c + 3 * kArgmaxSplitThreads < c1; c += 4 * kArgmaxSplitThreads) {
    const u32x4_t v0 = vrow[c];
    const u32x4_t v1 = vrow[c + kArgmaxSplitThreads];
    const u32x4_t v2 = vrow[c + 2 * kArgmaxSplitThreads];
    const u32x4_t v3 = vrow[c + 3 * kArgmaxSplitThreads];
    const u32x4_t vs[4] = {v0, v1, v2, v3};
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int base = (c + q * kArgmaxSplitThreads) * 8 + 2 * j;
        argmax_fold(__uint_as_float(vs[q][j] << 16), base, bv, bi);
        argmax_fold(__uint_as_float(vs[q][j] & 0xffff0000u), base + 1, bv, bi);
      }
  }
  for (; c < c1; c += kArgmaxSplitThreads) {
    const u32x4_t v = vrow[c];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      argmax_fold(__uint_as_float(v[j] << 16), c * 8 + 2 * j, bv, bi);
      argmax_fold(__uint_as_float(v[j] & 0xffff0000u), c * 8 + 2 * j + 1, bv, bi);
    }
  }
  if (b == nb - 1) {  // the row tail past the last full 8-logit group
    for (int n = (n_valid / 8) * 8 + threadIdx.x; n < n_valid; n += kArgmaxSplitThreads)
      argmax_fold(__uint_as_float((uint32_t)row[n] << 16), n, bv, bi);
  }
  argmax_block_reduce(bv, bi, sv, si);
  if (threadIdx.x == 0) {
    const int slot = m * kArgmaxMaxBlocks + b;
    __hip_atomic_store(&tval[slot], bv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&tidx[slot], bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    const unsigned prev = __hip_atomic_fetch_add(&tarr[m], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = prev == (unsigned)(nb - 1);
  }
  __syncthreads();
  if (!last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  bv = -__builtin_inff();
  bi = 0x7fffffff;
  if ((int)threadIdx.x < nb) {
    const int slot = m * kArgmaxMaxBlocks + threadIdx.x;
    bv = __hip_atomic_load(&tval[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bi = __hip_atomic_load(&tidx[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();  // sv / si are reused
  argmax_block_reduce(bv, bi, sv, si);
  if (threadIdx.x == 0) {
    const int idx = (bi == 0x7fffffff) ? 0 : bi;
    out[m] = (int64_t)idx + index_offset;
    __hip_atomic_store(&tarr[m], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Row normalisation to unit RMS, bf16 in and out: y[m, :] = bf16_rne(x[m, :] * (1 / sqrt(mean(x[m, :]^2) +
// eps))).  One wavefront per row (normalise_row); rows up to 64 x kNormPieces pieces are read from memory once.
constexpr int kNormPieces = 16;  // 16-byte pieces per lane held in registers: 64 x 16 x 8 = 8192 values
__global__ void __launch_bounds__(kWave) rms_norm_rows_kernel(const uint16_t* x, int64_t ldx, int N, float eps,
                                                              uint16_t* y, int64_t ldy) {
  const uint16_t* xr = x + (int64_t)blockIdx.x * ldx;
  uint16_t* yr = y + (int64_t)blockIdx.x * ldy;
  normalise_row<kNormPieces>(
      N / 8, N, eps, (int)threadIdx.x, [&](int j) { return *reinterpret_cast<const u32x4_t*>(xr + (int64_t)j * 8); },
      [&](int j, const u32x4_t o) { *reinterpret_cast<u32x4_t*>(yr + (int64_t)j * 8) = o; });
}

// ---------------------------------------------------------------------------------------------
// Read-bandwidth probe: every byte of [buf, buf + bytes) read once with 16-byte loads, grid-stride.
// One 32-bit xor per workgroup is written to sink so the loads cannot be dropped.
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) read_probe_kernel(const u32x4_t* buf, int64_t n16, uint32_t* sink) {
  __shared__ uint32_t red[256 / kWave];
  uint32_t acc = 0;
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4_t a = __builtin_nontemporal_load(buf + i);
    const u32x4_t b = __builtin_nontemporal_load(buf + i + stride);
    const u32x4_t c = __builtin_nontemporal_load(buf + i + 2 * stride);
    const u32x4_t d = __builtin_nontemporal_load(buf + i + 3 * stride);
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n16; i += stride) {
    const u32x4_t a = __builtin_nontemporal_load(buf + i);
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc ^= __shfl_xor(acc, off, kWave);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

// Read probe in the stream kernel's shape: one workgroup per CU, workgroup b reading the contiguous KiB
// range [b U / G, (b + 1) U / G) of the U KiB of the buffer, its W wavefronts interleaved at 1 KiB (wavefront
// v reads KiB v, v + W, ... of the range) with DEPTH KiB in flight each (non-temporal 16-byte loads).  No
// math: the fastest way this device reads a GEMM's bytes in that pattern.  One xor per workgroup goes to sink.
template <int W, int DEPTH>
__global__ void __launch_bounds__(W * kWave) read_probe_stream_kernel(const int8_t* buf, int64_t units,
                                                                      uint32_t* sink) {
  __shared__ uint32_t red[W];
  constexpr int RING = DEPTH + 1;
  const int lane = threadIdx.x & (kWave - 1);
  const int v = threadIdx.x / kWave;
  const int64_t u0 = ((int64_t)blockIdx.x * units) / gridDim.x;
  const int64_t u1 = ((int64_t)(blockIdx.x + 1) * units) / gridDim.x;
  const int total = (int)((u1 - u0 - v + W - 1) / W);  // KiB read by this wavefront (may be 0)
  uint32_t acc = 0;
  if (total > 0) {  // uniform per wavefront
    // The GEMM's ring: the load for step i + DEPTH goes into the slot step i - 1 freed, and indices past the
    // last step are clamped to it (an in-bounds re-read), so every load is unconditional and DEPTH stay in
    // flight.
    const int8_t* p = buf + (u0 + v) * 1024 + lane * 16;
    const int64_t stride = (int64_t)W * 1024;
    u32x4_t ring[RING];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) ring[d] = load16<true>(p + (int64_t)min(d, total - 1) * stride);
    for (int base = 0; base < total; base += RING) {
#pragma unroll
      for (int d = 0; d < RING; ++d) {
        ring[(d + DEPTH) % RING] = load16<true>(p + (int64_t)min(base + d + DEPTH, total - 1) * stride);
        __builtin_amdgcn_sched_barrier(0);
        if (base + d < total) {
          const u32x4_t x = ring[d];
          acc ^= x.x ^ x.y ^ x.z ^ x.w;
        }
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc ^= __shfl_xor(acc, off, kWave);
  if (lane == 0) red[v] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
    for (int i = 0; i < W; ++i) t ^= red[i];
    sink[blockIdx.x] = t;
  }
}

// A kernel that touches no memory: the dispatch cost of one launch in a graph of back-to-back launches.
__global__ void __launch_bounds__(64) empty_kernel() {}

// ---------------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------------
using KernelFn = void (*)(GemmArgs);

// MFMA instantiations: layout x NT {1, 2} x (WN, WK) x DEPTH {4, 8} x load hint, whole-slice x
// staging; the x-ring staging for the k_waves == 1 shapes.
template <int L, int NT, int WN, int WK, bool XR>
KernelFn mfma_fn(int depth, int hint) {
  if (depth == 4)
    return hint ? &w8a16_mfma_kernel<L, NT, WN, WK, 4, true, XR> : &w8a16_mfma_kernel<L, NT, WN, WK, 4, false, XR>;
  if (depth == 8)
    return hint ? &w8a16_mfma_kernel<L, NT, WN, WK, 8, true, XR> : &w8a16_mfma_kernel<L, NT, WN, WK, 8, false, XR>;
  return nullptr;
}

template <int L, int NT>
KernelFn mfma_by_shape(int wn, int wk, int depth, int hint, bool xring) {
  if (xring) {
    if (wn == 4 && wk == 1) return mfma_fn<L, NT, 4, 1, true>(depth, hint);
    if (wn == 8 && wk == 1) return mfma_fn<L, NT, 8, 1, true>(depth, hint);
    return nullptr;
  }
#define QF_WNWK(A, B) \
  if (wn == A && wk == B) return mfma_fn<L, NT, A, B, false>(depth, hint);
  QF_WNWK(4, 1) QF_WNWK(8, 1) QF_WNWK(2, 2) QF_WNWK(4, 2) QF_WNWK(8, 2)
  QF_WNWK(1, 4) QF_WNWK(2, 4) QF_WNWK(4, 4) QF_WNWK(1, 8) QF_WNWK(2, 8)
#undef QF_WNWK
  return nullptr;
}

KernelFn select_mfma(int layout, int nt, int waves, int k_waves, int depth, int hint, bool xring) {
  if (k_waves < 1 || waves % k_waves) return nullptr;
  const int wn = waves / k_waves;
  if (layout == QF_LAYOUT_ROWMAJOR) {
    if (nt == 1) return mfma_by_shape<QF_LAYOUT_ROWMAJOR, 1>(wn, k_waves, depth, hint, xring);
    if (nt == 2) return mfma_by_shape<QF_LAYOUT_ROWMAJOR, 2>(wn, k_waves, depth, hint, xring);
  } else {
    if (nt == 1) return mfma_by_shape<QF_LAYOUT_TILED, 1>(wn, k_waves, depth, hint, xring);
    if (nt == 2) return mfma_by_shape<QF_LAYOUT_TILED, 2>(wn, k_waves, depth, hint, xring);
  }
  return nullptr;
}

inline bool is_mfma(int kernel) { return kernel == QF_KERNEL_MFMA || kernel == QF_KERNEL_MFMA_XRING; }

// Instantiations that normalise their staged x rows first (qf_w8a16_gemm_rmsnorm): the MFMA kernel on TILED
// weights, one tile a wavefront, depth 4, non-temporal loads, whole-slice x, as (WN, WK) = (4, 2), (2, 4),
// (1, 4) or (8, 1); the LDS-staged stream kernel with 8 wavefronts at depth 4.
KernelFn select_norm(const qf_w8a16_config& c, int layout) {
  if (layout != QF_LAYOUT_TILED || c.depth != 4 || !c.load_hint || c.tiles_per_wave != 1) return nullptr;
  if (c.kernel == QF_KERNEL_MFMA) {
    const int wn = c.waves / c.k_waves, wk = c.k_waves;
    if (wn == 4 && wk == 2) return &w8a16_mfma_kernel<QF_LAYOUT_TILED, 1, 4, 2, 4, true, false, true>;
    if (wn == 2 && wk == 4) return &w8a16_mfma_kernel<QF_LAYOUT_TILED, 1, 2, 4, 4, true, false, true>;
    if (wn == 1 && wk == 4) return &w8a16_mfma_kernel<QF_LAYOUT_TILED, 1, 1, 4, 4, true, false, true>;
    if (wn == 8 && wk == 1) return &w8a16_mfma_kernel<QF_LAYOUT_TILED, 1, 8, 1, 4, true, false, true>;
  }
  if (c.kernel == QF_KERNEL_MFMA_STREAM && c.reduce == 0 && c.waves == 8)
    return &w8a16_stream_kernel<8, 4, true, true>;
  return nullptr;
}

// Stream-kernel instantiations (TILED weights, non-temporal loads): 8 wavefronts at depth 2, 3, 4, 5, 6, 8, 12
// or 16; 16 wavefronts at depth 2, 4 or 8.  Both keep the accumulator in VGPRs.  (A 4-wavefront build, one
// wavefront per SIMD, was 20% slower on gate_up and gave wrong sums: its compiled loop moves the
// conditionally cleared accumulator between AGPRs and VGPRs; it is not instantiated.)
KernelFn select_stream(int waves, int depth, int hint) {
  if (!hint) return nullptr;
  if (waves == 8) {
    if (depth == 2) return &w8a16_stream_kernel<8, 2, true>;
    if (depth == 3) return &w8a16_stream_kernel<8, 3, true>;
    if (depth == 4) return &w8a16_stream_kernel<8, 4, true>;
    if (depth == 5) return &w8a16_stream_kernel<8, 5, true>;
    if (depth == 6) return &w8a16_stream_kernel<8, 6, true>;
    if (depth == 8) return &w8a16_stream_kernel<8, 8, true>;
    if (depth == 12) return &w8a16_stream_kernel<8, 12, true>;
    if (depth == 16) return &w8a16_stream_kernel<8, 16, true>;
  }
  if (waves == 16) {
    if (depth == 2) return &w8a16_stream_kernel<16, 2, true>;
    if (depth == 4) return &w8a16_stream_kernel<16, 4, true>;
    if (depth == 8) return &w8a16_stream_kernel<16, 8, true>;
  }
  return nullptr;
}

// The register-x stream kernel for K = 64 W S: 8 wavefronts with S = 10 (K = 5120) at depth 4 or 9, S = 16
// (K = 8192) at depth 3 or 7, S = 8 (K = 4096) at depth 3; 16 wavefronts with S = 5 (K = 5120) at depth 4.
KernelFn select_stream_xreg(int waves, int depth, int ksteps) {
  if (waves == 8) {
    if (ksteps == 80 && depth == 4) return &w8a16_stream_xreg_kernel<8, 10, 4>;
    if (ksteps == 80 && depth == 9) return &w8a16_stream_xreg_kernel<8, 10, 9>;
    if (ksteps == 128 && depth == 3) return &w8a16_stream_xreg_kernel<8, 16, 3>;
    if (ksteps == 128 && depth == 7) return &w8a16_stream_xreg_kernel<8, 16, 7>;
    if (ksteps == 64 && depth == 3) return &w8a16_stream_xreg_kernel<8, 8, 3>;
  }
  if (waves == 16 && ksteps == 80 && depth == 4) return &w8a16_stream_xreg_kernel<16, 5, 4>;
  return nullptr;
}

// Compute units of the current device (the stream kernel's grid), cached per device; 256 (an MI355X)
// when no device is visible, so that host-only configuration queries still answer.
constexpr int kMaxCuDevices = 64;
std::mutex g_cu_mutex;
int g_cu_count[kMaxCuDevices];

int device_cus() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxCuDevices) {
    (void)hipGetLastError();
    return 256;
  }
  std::lock_guard<std::mutex> lock(g_cu_mutex);
  if (g_cu_count[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) {
      (void)hipGetLastError();
      return 256;
    }
    g_cu_count[dev] = n;
  }
  return g_cu_count[dev];
}

// Wide-M instantiations: NT {1, 2} x MT {1..4} x WN {4, 8} x DEPTH {4, 8}, and NT 4 x MT {1..4} with 4
// wavefronts and DEPTH 2 (non-temporal weight loads).
template <int NT, int MT>
KernelFn wide_by_shape(int wn, int depth) {
  if (wn == 4 && depth == 4) return &w8a16_wide_kernel<NT, MT, 4, 4>;
  if (wn == 4 && depth == 8) return &w8a16_wide_kernel<NT, MT, 4, 8>;
  if (wn == 8 && depth == 4) return &w8a16_wide_kernel<NT, MT, 8, 4>;
  if (wn == 8 && depth == 8) return &w8a16_wide_kernel<NT, MT, 8, 8>;
  return nullptr;
}

template <int NT>
KernelFn wide_by_mt(int mt, int wn, int depth) {
  switch (mt) {
    case 1: return wide_by_shape<NT, 1>(wn, depth);
    case 2: return wide_by_shape<NT, 2>(wn, depth);
    case 3: return wide_by_shape<NT, 3>(wn, depth);
    case 4: return wide_by_shape<NT, 4>(wn, depth);
    default: return nullptr;
  }
}

KernelFn select_wide(int nt, int mt, int waves, int depth) {
  if (nt == 1) return wide_by_mt<1>(mt, waves, depth);
  if (nt == 2) return wide_by_mt<2>(mt, waves, depth);
  if (nt == 4 && waves == 4 && depth == 2) {
    switch (mt) {
      case 1: return &w8a16_wide_kernel<4, 1, 4, 2>;
      case 2: return &w8a16_wide_kernel<4, 2, 4, 2>;
      case 3: return &w8a16_wide_kernel<4, 3, 4, 2>;
      case 4: return &w8a16_wide_kernel<4, 4, 4, 2>;
      default: return nullptr;
    }
  }
  return nullptr;
}

// Token groups of the wide-M kernel: as few groups as 64-row groups allow, rows spread evenly and
// rounded up to whole 16-row tiles; the count is then recomputed so that every group has a row.
constexpr int kWideGroupRows = 64;
void wide_groups(int M, int& groups, int& group_rows) {
  const int g0 = (M + kWideGroupRows - 1) / kWideGroupRows;
  group_rows = ((M + g0 - 1) / g0 + 15) / 16 * 16;
  groups = (M + group_rows - 1) / group_rows;
}

template <int MM, int RPW>
KernelFn gemv_fn(int hint) {
  return hint ? &w8a16_gemv_kernel<MM, RPW, 4, true> : &w8a16_gemv_kernel<MM, RPW, 4, false>;
}

template <int MM>
KernelFn gemv_by_rpw(int rpw, int hint) {
  switch (rpw) {
    case 2: return gemv_fn<MM, 2>(hint);
    case 4: return gemv_fn<MM, 4>(hint);
    default: return nullptr;
  }
}

KernelFn select_gemv(int M, int rpw, int waves, int hint) {
  if (waves != 4) return nullptr;
  switch (M) {
    case 1: return gemv_by_rpw<1>(rpw, hint);
    case 2: return gemv_by_rpw<2>(rpw, hint);
    case 3: return gemv_by_rpw<3>(rpw, hint);
    case 4: return gemv_by_rpw<4>(rpw, hint);
    default: return nullptr;
  }
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
inline int round_up16(int n) { return (n + 15) / 16 * 16; }

// LDS bytes of one workgroup: the largest split's x slice, or, for MFMA with k_waves > 1, the
// slice-reduction buffer if that is larger.
int workgroups(const qf_w8a16_config& c, int N);

size_t lds_bytes(const qf_w8a16_config& c, int M, int ksteps, int N) {
  const int steps = ceil_div(ksteps, c.split_k);
  if (c.kernel == QF_KERNEL_MFMA_STREAM)  // the x slice (reduce 0), then a 1 KiB partial per (tile, wavefront)
    return ((c.reduce & 1) ? 0 : (size_t)align16i(M * x_pitch(ksteps))) +
           (size_t)ceil_div(round_up16(N) / kTileN, workgroups(c, N)) * c.waves * kWave * sizeof(f32x4_t);
  if (c.kernel == QF_KERNEL_GEMV) return (size_t)M * steps * kStepK * 2;
  if (c.kernel == QF_KERNEL_MFMA_WIDE) {
    int groups, rows;
    wide_groups(M, groups, rows);
    // two chunks of the group's rows, rows padded by 16 bytes in 8-wavefront workgroups
    return (size_t)2 * rows * ((c.depth + 1) * kStepK * 2 + (c.waves == 8 ? 16 : 0));
  }
  const size_t xs = c.kernel == QF_KERNEL_MFMA_XRING ? (size_t)2 * M * (c.depth + 1) * kStepK * 2  // two chunks
                                                     : (size_t)M * x_pitch(steps);
  const size_t red = c.k_waves > 1 ? (size_t)c.waves * c.tiles_per_wave * kWave * sizeof(f32x4_t) : 0;
  return xs > red ? xs : red;
}

int workgroups(const qf_w8a16_config& c, int N) {
  if (c.kernel == QF_KERNEL_GEMV) return ceil_div(N, c.waves * c.tiles_per_wave);
  if (c.kernel == QF_KERNEL_MFMA_STREAM)  // one per CU, or (reduce bit 2) runs of tiles_per_wave tiles
    return (c.reduce & 4) ? ceil_div(round_up16(N) / kTileN, c.tiles_per_wave) : device_cus();
  const int wn = c.waves / c.k_waves;
  return ceil_div(round_up16(N) / kTileN, wn * c.tiles_per_wave);
}

// Workspace: a fixed prefix of arrival counters (the same bytes for every call, so counters never
// land on memory an earlier call used for partial sums), then the split partials.
size_t workspace_for(const qf_w8a16_config& c, int M, int N) {
  if (c.split_k <= 1) return 0;
  if (c.kernel == QF_KERNEL_MFMA_W8A8_TILE)  // a 256 KiB int32 slot per (tile, split): 8 wavefronts x 32 KiB
    return QF_W8A16_COUNTER_BYTES + (size_t)ceil_div(round_up16(N) / kTileN, kW8A8TileTiles) *
                                        ceil_div(M, kW8A8TileRows) * c.split_k * (size_t)(256 * 1024);
  return QF_W8A16_COUNTER_BYTES + (size_t)c.split_k * (size_t)M * (size_t)round_up16(N) * sizeof(float);
}

// Checks a complete configuration against the instantiated kernels and the LDS budget.
int validate_config(int M, int N, int K, int layout, const qf_w8a16_config& c) {
  const int ksteps = K / kStepK;
  if (c.kernel != QF_KERNEL_GEMV && !is_mfma(c.kernel) && c.kernel != QF_KERNEL_MFMA_WIDE &&
      c.kernel != QF_KERNEL_MFMA_STREAM)
    return QF_ERR_INVALID_ARG;
  if (c.split_k < 1 || c.split_k > ksteps || c.waves < 1 || c.k_waves < 1 || c.tiles_per_wave < 1)
    return QF_ERR_INVALID_ARG;
  if (c.kernel == QF_KERNEL_MFMA_STREAM) {
    // TILED weights, M <= 16, one workgroup per CU over the whole K range, every wavefront splitting K.
    if (layout != QF_LAYOUT_TILED || M > QF_W8A16_MAX_M) return QF_ERR_UNSUPPORTED;
    if (c.split_k != 1 || c.k_waves != c.waves || ksteps < c.waves) return QF_ERR_UNSUPPORTED;
    if (c.reduce < 0 || c.reduce > 7 || ((c.reduce & 4) == 0 && c.tiles_per_wave != 1)) return QF_ERR_INVALID_ARG;
    if ((c.reduce & 1) == 0 && select_stream(c.waves, c.depth, c.load_hint) == nullptr) return QF_ERR_UNSUPPORTED;
    if ((c.reduce & 1) != 0 && (!c.load_hint || select_stream_xreg(c.waves, c.depth, ksteps) == nullptr))
      return QF_ERR_UNSUPPORTED;
    return lds_bytes(c, M, ksteps, N) > kMaxLds ? QF_ERR_UNSUPPORTED : QF_OK;
  }
  if (c.kernel == QF_KERNEL_MFMA_WIDE) {
    // TILED weights, any M, the whole K range per workgroup.
    if (layout != QF_LAYOUT_TILED || c.k_waves != 1) return QF_ERR_UNSUPPORTED;
    int groups, rows;
    wide_groups(M, groups, rows);
    if ((int64_t)workgroups(c, N) * groups * c.split_k > 0x7fffffff) return QF_ERR_UNSUPPORTED;
    if (select_wide(c.tiles_per_wave, rows / 16, c.waves, c.depth) == nullptr) return QF_ERR_UNSUPPORTED;
    return lds_bytes(c, M, ksteps, N) > kMaxLds ? QF_ERR_UNSUPPORTED : QF_OK;
  }
  if (M > QF_W8A16_MAX_M) return QF_ERR_UNSUPPORTED;
  if (c.kernel == QF_KERNEL_GEMV && (M > 4 || layout != QF_LAYOUT_ROWMAJOR || c.k_waves != 1))
    return QF_ERR_UNSUPPORTED;
  if (ksteps / c.split_k < c.k_waves) return QF_ERR_UNSUPPORTED;  // every k-slice needs a step
  if (c.kernel == QF_KERNEL_MFMA_XRING && c.k_waves != 1) return QF_ERR_UNSUPPORTED;
  if (is_mfma(c.kernel) && c.split_k > 1 && c.reduce == 0 &&
      (size_t)workgroups(c, N) * 4 > QF_W8A16_COUNTER_BYTES)
    return QF_ERR_UNSUPPORTED;  // one arrival counter per workgroup column
  if (lds_bytes(c, M, ksteps, N) > kMaxLds) return QF_ERR_UNSUPPORTED;
  if (is_mfma(c.kernel) && select_mfma(layout, c.tiles_per_wave, c.waves, c.k_waves, c.depth, c.load_hint,
                                       c.kernel == QF_KERNEL_MFMA_XRING) == nullptr)
    return QF_ERR_UNSUPPORTED;
  if (c.kernel == QF_KERNEL_GEMV && select_gemv(M, c.tiles_per_wave, c.waves, c.load_hint) == nullptr)
    return QF_ERR_UNSUPPORTED;
  return QF_OK;
}

// Automatic configuration (host only).  Returns false when unsupported.  Chosen from measured
// sweeps at M = 5 on MI355X (TILED layout): one 16-row tile per wavefront, 8 wavefronts per
// workgroup, a 4-step weight prefetch ring; the K range is split inside the workgroup (k_waves,
// reduced through LDS), and across workgroups only when K > 128 k-steps or the staged activation
// slice would not fit in LDS; such splits are summed by the last workgroup of each n-block.
// A workgroup shape measured better for a particular (N, K) overrides the k_waves rule, as the
// reference keeps a tuned table beside its heuristic (plugin/qwen_fastpath/w8a16.py:47-55).
struct TunedShape {
  int N, K, max_m, k_waves;
};
constexpr TunedShape kTuned[] = {
    {10240, 5120, 8, 2},  // dense 27B-class qkv: 4 tiles x 2 k-slices per workgroup (11.9 us against 13.6 us)
    {5120, 17408, 8, 2},  // dense 27B-class down, split 3 (19.0 us against 19.4 us)
};

bool auto_config(int M, int N, int K, int layout, qf_w8a16_config* c, bool stream_ok = true) {
  if (M < 1 || N < 1 || K < QF_W8A16_K_ALIGN || K % QF_W8A16_K_ALIGN) return false;
  if (layout != QF_LAYOUT_ROWMAJOR && layout != QF_LAYOUT_TILED) return false;
  if (stream_ok && layout == QF_LAYOUT_TILED && M >= 2 && M <= QF_W8A16_MAX_M &&
      round_up16(N) / kTileN >= 4 * device_cus()) {
    // Wide N (4 or more 16-row tiles per CU) at 2 or more tokens: the stream kernel, one workgroup per CU of
    // 8 wavefronts with 4 steps in flight each, where the x slice and the partial tiles fit in LDS (K = 5120:
    // up to 8 tokens).  Interleaved A/B on gate_up 34816 x 5120, weights rotated past the last-level cache:
    // M = 2 / 3 / 4 / 5 / 6 / 7 / 8 29.6 / 29.7 / 29.7 / 29.7 / 30.8 / 30.7 / 30.7 us against 30.1 / 31.9 /
    // 32.0 / 32.2 / 36.0 / 36.3 / 34.2 us for the shapes below; depth 3 and 5 are level with 4, depth 2, 6, 8,
    // 12 and 16 slower (30.3, 30.3, 30.9, 32.3, 33.3 us at M = 5), 4-wavefront workgroups slower (35.5 us).
    // At M = 1 the 4-wavefront shape below stays ahead (29.0 against 29.5 us).  Fewer tiles per CU leave the
    // workgroups' whole-tile shares too uneven (qkv 10240 x 5120, 2.5 tiles a CU: 12.1 against 11.8 us).
    // Where the x slice does not fit (K = 5120: M >= 9), each wavefront holds its x fragments in registers
    // (reduce 1; the same sums bit for bit): gate_up M = 12 31.8 us and M = 16 32.1 us (16 wavefronts; 32.6 with
    // 8) against 34.9 and 35.4 us for the two-slot x ring below.
    qf_w8a16_config sc = qf_w8a16_config{};
    sc.kernel = QF_KERNEL_MFMA_STREAM;
    sc.split_k = 1;
    sc.tiles_per_wave = 1;
    sc.waves = 8;
    sc.k_waves = 8;
    sc.depth = 4;
    sc.load_hint = 1;
    if (validate_config(M, N, K, layout, sc) == QF_OK) {
      *c = sc;
      return true;
    }
    const int ks = K / kStepK;
    sc.reduce = 1;
    if (M >= 13) {
      sc.waves = sc.k_waves = 16;
    }
    sc.depth = ks == 128 ? 3 : 4;
    if (validate_config(M, N, K, layout, sc) == QF_OK) {
      *c = sc;
      return true;
    }
    sc.waves = sc.k_waves = 8;
    if (validate_config(M, N, K, layout, sc) == QF_OK) {
      *c = sc;
      return true;
    }
  }
  if (M > QF_W8A16_MAX_M) {
    // Beyond the decode widths only TILED weights are served, by the wide-M kernel (64-row token
    // groups; measured on the dense 27B-class layer at M = 17 .. 2048 against 32-, 16- and 128-row
    // groups, which lose everywhere).  Once 4-wavefront workgroups of 4 tiles a wavefront number 256
    // or more, they run with 2 steps in flight: each x fragment read from LDS then feeds 4 tiles
    // (M = 1024: gate_up 403 us against 482, qkv 133 against 148, down 252 against 267).  Below
    // that: 2 tiles per wavefront, 4 steps in flight, 8 wavefronts per workgroup, or 4 once
    // 8-wavefront workgroups number 256 or more (gate_up M = 128: 88.0 us against 98.4); K is split
    // across workgroups until they number 128, at most 8 ways and 16 steps a split (M = 17: o_proj
    // 16.4 us unsplit 31.8, down 23.5 against 62.6, qkv 16.5 against 21.0).
    if (layout != QF_LAYOUT_TILED) return false;
    *c = qf_w8a16_config{};
    c->kernel = QF_KERNEL_MFMA_WIDE;
    c->k_waves = 1;
    c->load_hint = 1;
    c->reduce = 1;
    c->split_k = 1;
    c->tiles_per_wave = 4;
    c->waves = 4;
    c->depth = 2;
    int groups, rows;
    wide_groups(M, groups, rows);
    const int ksteps = K / kStepK;
    const int64_t wgs4 = (int64_t)workgroups(*c, N) * groups;
    if (wgs4 >= 256) return validate_config(M, N, K, layout, *c) == QF_OK;
    if (wgs4 >= 128 && wgs4 < 192 && ksteps >= 256) {
      // Long K (K >= 16384) and 128..191 such workgroups: split K as far as 512 workgroups (two per
      // CU slot), 4 ways and 64 steps a split at most.  down 5120 x 17408 at M = 448 / 512 (3 ways):
      // 102 / 107 us against 138 us for the 2-tile choice below, which stays ahead from M = 640.
      while (wgs4 * (c->split_k + 1) <= 512 && c->split_k < 4 && ksteps / (c->split_k + 1) >= 64) ++c->split_k;
      return validate_config(M, N, K, layout, *c) == QF_OK;
    }
    c->tiles_per_wave = 2;
    c->waves = 8;
    c->depth = 4;
    int64_t wgs = (int64_t)workgroups(*c, N) * groups;
    if (wgs >= 256) {
      c->waves = 4;
      wgs = (int64_t)workgroups(*c, N) * groups;
    }
    c->split_k = 1;
    while (wgs * c->split_k < 128 && c->split_k < 8 && ksteps / (c->split_k + 1) >= 16) ++c->split_k;
    return validate_config(M, N, K, layout, *c) == QF_OK;
  }
  *c = qf_w8a16_config{};
  c->kernel = QF_KERNEL_MFMA;
  c->tiles_per_wave = 1;
  c->depth = 4;
  c->load_hint = layout == QF_LAYOUT_TILED ? 1 : 0;
  c->waves = 8;
  c->reduce = 0;
  const int ksteps = K / kStepK;
  const bool wide_n = round_up16(N) / (kTileN * 16) >= 128;  // >= 128 groups of 256 rows
  if (layout == QF_LAYOUT_ROWMAJOR && (M == 1 || (M == 2 && wide_n))) {
    // Row-major weights at M = 1, and at M = 2 on wide N: the GEMV kernel's contiguous 1 KiB row
    // reads win over the MFMA tiles' 64-byte row pieces (M = 1: gate_up 30.9 us against 46 us, down
    // 17.7 us against 21.0 us; at M = 2 narrow N the MFMA tiles are level or ahead).
    c->kernel = QF_KERNEL_GEMV;
    c->waves = 4;
    c->k_waves = 1;
    c->tiles_per_wave = 2;  // rows per wavefront (gate_up M = 2: 37.6 us against 41.6 us with 4)
    c->load_hint = 1;
    c->split_k = 1;
    c->reduce = 1;
    while (lds_bytes(*c, M, ksteps, N) > kMaxLds && c->split_k < ksteps) ++c->split_k;
    return validate_config(M, N, K, layout, *c) == QF_OK;
  }
  // wide N only (>= 128 workgroups of 256 rows), and only on the TILED layout, whose 1 KiB fragments
  // stay contiguous however many tiles a wavefront holds (row-major gate_up at M = 8: 63 us with this
  // shape against 42 us without)
  if (M >= 8 && layout == QF_LAYOUT_TILED && wide_n) {
    // Wide M and N: a workgroup covers more weight rows per x byte -- 8 tile groups of 2 tiles, each
    // wavefront over the whole K range (gate_up: M = 8 35.0 us, M = 12 36.5 us against 44 and 48 us
    // with the M = 5 shape) -- and x goes through the two-slot ring with K unsplit: only a 5-step
    // chunk is staged before the first step, and LDS holds two chunks instead of the whole slice
    // (interleaved A/B against staging the whole slice: M = 8 34.1 us against 35.3, M = 12 34.6
    // against 36.2, and, where the slice needed a 3-way K split to fit, M = 13 35.1 against 38.2 and
    // M = 16 35.4 against 39.3 us).
    c->tiles_per_wave = 2;
    c->k_waves = 1;
    c->kernel = QF_KERNEL_MFMA_XRING;
    c->split_k = 1;
    return validate_config(M, N, K, layout, *c) == QF_OK;
  }
  if (layout == QF_LAYOUT_ROWMAJOR && (wide_n || M < 12)) {
    // Row-major weights: a wavefront's 16 rows are read as 64-byte row pieces, so workgroups are
    // kept at 4 wavefronts with one k-slice each and more of them run: wide N at M >= 8 splits K
    // 2 ways (3 from M = 12) with the second-pass sum (gate_up M = 8: 48.8 us, M = 16: 51.6 us,
    // against 53.6 and 57.6 us with the tiled-layout shape); narrow N splits K 3 ways once fewer
    // than 160 workgroups would run or M >= 8, summed in-kernel (M = 5: o_proj 11.7 us, down
    // 22.2 us, qkv 13.7 us unsplit, against 14.2, 25.9 and 14.6 us).
    if (wide_n && M < 8) {
      // M = 3..7 on wide N: the tiled-layout shape below measured best (gate_up M = 5: 43.4 us).
    } else {
      c->waves = 4;
      c->k_waves = 1;
      if (wide_n) {
        c->split_k = M >= 12 ? 3 : 2;
        c->k_waves = M >= 12 ? 1 : 2;
        c->depth = M >= 12 ? 8 : 4;
        c->reduce = 1;
      } else {
        const int wgs = ceil_div(round_up16(N) / kTileN, c->waves);
        c->split_k = (wgs >= 160 && M < 8) ? 1 : 3;
        c->reduce = 0;
      }
      if (c->split_k > ksteps) c->split_k = ksteps;
      if (ksteps / c->split_k < c->k_waves) c->k_waves = 1;
      if (!wide_n && ksteps / c->split_k >= 64) c->depth = 8;  // down: 21.2 us against 21.8 at M = 2
      while (lds_bytes(*c, M, ksteps, N) > kMaxLds && c->split_k < ksteps) ++c->split_k;
      if (c->split_k > 1 && (size_t)workgroups(*c, N) * 4 > QF_W8A16_COUNTER_BYTES) c->reduce = 1;
      return validate_config(M, N, K, layout, *c) == QF_OK;
    }
  }
  if (M >= 12) {
    // Wide M, narrow N: the x slice of a 5120-k row set is 10 KiB per token, so K is split at least
    // three ways (at most 48 k-steps a split) and the splits are summed by the second-pass kernel
    // (M = 16: qkv 14.4 us, o_proj 13.7 us, down 21.9 us against 21.0, 18.5 and 35.6 us).
    c->split_k = ceil_div(ksteps, 48);
    if (c->split_k < 3) c->split_k = 3;
    if (c->split_k > ksteps) c->split_k = ksteps;
    c->k_waves = (c->split_k <= 3 && ksteps / c->split_k >= 40) ? 2 : 1;  // o_proj: 2; qkv, down: 1
    if (layout == QF_LAYOUT_ROWMAJOR && c->k_waves == 2) {
      c->waves = 4;  // row-major o_proj M = 16: 14.3 us against 15.3 us
      c->k_waves = 1;
    }
    if (layout == QF_LAYOUT_TILED) {
      // x through the two-slot ring, one k-slice per workgroup (interleaved A/B, M = 12 / 16):
      // o_proj-like shapes (2 k-slices above) as 4 wavefronts with 8 steps in flight, 12.4 / 12.7 us
      // against 13.3 / 13.5 us; short splits (qkv, 27 steps) with 8 steps in flight, 14.0 / 14.4 us
      // against 14.3 / 14.8 us; down (45 steps a split) at DEPTH 4, 20.5 / 20.8 us, level with the
      // alternatives and ahead of the whole slice (21.3 / 21.5 us).
      c->kernel = QF_KERNEL_MFMA_XRING;
      if (c->k_waves == 2) {
        c->waves = 4;
        c->k_waves = 1;
        c->depth = 8;
      } else if (ksteps / c->split_k < 32) {
        c->depth = 8;
      }
    }
    c->reduce = 1;
    while (lds_bytes(*c, M, ksteps, N) > kMaxLds && c->split_k < ksteps) ++c->split_k;
    return validate_config(M, N, K, layout, *c) == QF_OK;
  }
  // Narrow M at 1..2 tokens: 4-wavefront workgroups (gate_up M = 1: 30.4 us against 35.1 us).
  if (M <= 2) c->waves = 4;
  c->split_k = ceil_div(ksteps, 128);
  for (;;) {
    const int per_split = ksteps / c->split_k;
    c->k_waves = per_split >= 64 ? 4 : (per_split >= 16 ? 2 : 1);
    if (lds_bytes(*c, M, ksteps, N) <= kMaxLds || c->split_k >= ksteps) break;
    ++c->split_k;
  }
  for (const TunedShape& t : kTuned) {
    if (t.N == N && t.K == K && M <= t.max_m) {
      qf_w8a16_config tc = *c;
      tc.k_waves = t.k_waves;
      if (validate_config(M, N, K, layout, tc) == QF_OK) *c = tc;
    }
  }
  // Few workgroups (narrow N, such as one tensor-parallel rank's shard): 4-wavefront workgroups run
  // twice as many, each stream being latency-bound at this size, and 8 steps in flight once a
  // wavefront has 16 or more (TP = 8 shards at M = 5: o_proj 5120x1024 4.0 us against 5.0, down
  // 5120x2176 5.1 us against 6.6, qkv 1280x5120 6.4 us against 6.9; gate_up 4352x5120, 136
  // workgroups of 8 wavefronts, stays: 7.5 us against 8.2).
  if (c->waves == 8 && (int64_t)workgroups(*c, N) * c->split_k < 128) {
    qf_w8a16_config tc = *c;
    tc.waves = 4;
    if (ksteps / tc.split_k / tc.k_waves >= 16) tc.depth = 8;
    if (validate_config(M, N, K, layout, tc) == QF_OK) *c = tc;
  }
  // The fused reduction needs one arrival counter per workgroup column.
  if (c->split_k > 1 && (size_t)workgroups(*c, N) * 4 > QF_W8A16_COUNTER_BYTES) c->reduce = 1;
  return validate_config(M, N, K, layout, *c) == QF_OK;
}

// Validate / complete a caller configuration.
// stream_ok = false for the fused argmax, whose epilogue only the MFMA kernels have.
int resolve_config(int M, int N, int K, int layout, const qf_w8a16_config* in, qf_w8a16_config* out,
                   bool stream_ok = true) {
  if (!auto_config(M, N, K, layout, out, stream_ok)) return QF_ERR_UNSUPPORTED;
  if (in == nullptr || in->kernel == QF_KERNEL_AUTO) return QF_OK;
  qf_w8a16_config c = *in;
  if (c.waves == 0) c.waves = c.kernel == QF_KERNEL_MFMA_STREAM ? 8 : 4;
  if (c.k_waves == 0) c.k_waves = c.kernel == QF_KERNEL_MFMA_STREAM ? c.waves : 1;
  if (c.tiles_per_wave == 0) c.tiles_per_wave = (c.kernel == QF_KERNEL_GEMV) ? 4 : 1;
  if (c.depth == 0) c.depth = 8;
  if (c.split_k == 0) c.split_k = c.kernel == QF_KERNEL_MFMA_WIDE ? 1 : out->split_k;
  const int rc = validate_config(M, N, K, layout, c);
  if (rc != QF_OK) return rc;
  *out = c;
  return QF_OK;
}

// Kernels that were allowed more than the default dynamic LDS (hipFuncSetAttribute is per kernel).
std::mutex g_lds_mutex;
std::unordered_set<const void*> g_lds_raised;

int launch(KernelFn fn, dim3 grid, dim3 block, size_t smem, hipStream_t stream, const GemmArgs& a) {
  void* args[] = {const_cast<GemmArgs*>(&a)};
  if (smem > kDefaultLds) {
    std::lock_guard<std::mutex> lock(g_lds_mutex);
    const void* key = reinterpret_cast<const void*>(fn);
    if (g_lds_raised.find(key) == g_lds_raised.end()) {
      // The limit is what the kernel's own static LDS leaves of the workgroup's 160 KiB.
      hipFuncAttributes attr;
      if (hipFuncGetAttributes(&attr, key) != hipSuccess) return QF_ERR_HIP;
      const size_t room = kLdsPerWorkgroup - attr.sharedSizeBytes;
      if (smem > room) return QF_ERR_UNSUPPORTED;
      if (hipFuncSetAttribute(key, hipFuncAttributeMaxDynamicSharedMemorySize, (int)room) != hipSuccess)
        return QF_ERR_HIP;
      g_lds_raised.insert(key);
    }
  }
  if (hipLaunchKernel(reinterpret_cast<const void*>(fn), grid, block, args, smem, stream) != hipSuccess)
    return QF_ERR_HIP;
  return QF_OK;
}

// Words between the arrival counters of n workgroup groups: spread over the counter prefix (up to 1 KiB apart),
// since atomics on nearby addresses share a memory channel (measured on the fused argmax: 64 slots 64 bytes apart
// cost 11 us on 9496 workgroups, 1 KiB apart about 3).
int counter_stride_for(int n) {
  int st = QF_W8A16_COUNTER_BYTES / 4 / (n > 0 ? n : 1);
  st = st < 256 ? st : 256;
  while (st & (st - 1)) st &= st - 1;
  return st > 0 ? st : 1;
}

struct ArgmaxRequest {
  int n_valid;
  int64_t index_offset;
  int64_t* ids;
};

// Workspace of the fused argmax: the counter prefix, which holds the per-token slots.
size_t argmax_workspace_for(const qf_w8a16_config&, int, int) { return QF_W8A16_COUNTER_BYTES; }

// norm_eps != nullptr: the x rows are scaled to unit RMS first (qf_w8a16_gemm_rmsnorm), by a NORM instantiation.
int run_gemm(const uint16_t* x, int64_t ldx, const int8_t* w, int64_t ldw, int layout, const float* scale, void* y,
             int64_t ldy, int out_dtype, int M, int N, int K, const qf_w8a16_config* cfg, void* workspace,
             size_t workspace_bytes, void* stream, const ArgmaxRequest* am, const float* norm_eps = nullptr) {
  if (x == nullptr || w == nullptr || scale == nullptr) return QF_ERR_INVALID_ARG;
  if (M < 1 || N < 1 || K < 1) return QF_ERR_INVALID_ARG;
  if (layout != QF_LAYOUT_ROWMAJOR && layout != QF_LAYOUT_TILED) return QF_ERR_INVALID_ARG;
  if (out_dtype != QF_DTYPE_BF16 && out_dtype != QF_DTYPE_F32) return QF_ERR_INVALID_ARG;
  if (ldx < K || (y != nullptr && ldy < N) || (layout == QF_LAYOUT_ROWMAJOR && ldw < K)) return QF_ERR_INVALID_ARG;
  if ((M > QF_W8A16_MAX_M && layout != QF_LAYOUT_TILED) || K % QF_W8A16_K_ALIGN) return QF_ERR_UNSUPPORTED;
  if (!aligned16(x) || !aligned16(w) || !aligned16(scale) || (y != nullptr && !aligned16(y))) return QF_ERR_UNSUPPORTED;
  if (ldx % 8 || (layout == QF_LAYOUT_ROWMAJOR && ldw % 16)) return QF_ERR_UNSUPPORTED;

  qf_w8a16_config c;
  const int rc = resolve_config(M, N, K, layout, cfg, &c, am == nullptr);
  if (rc != QF_OK) return rc;
  if (am != nullptr && (!is_mfma(c.kernel) || c.split_k != 1)) return QF_ERR_UNSUPPORTED;
  // The normalising GEMM needs whole rows staged: no K split, and an instantiation that normalises.
  if (norm_eps != nullptr && (c.split_k != 1 || select_norm(c, layout) == nullptr)) return QF_ERR_UNSUPPORTED;
  const size_t need = am != nullptr ? argmax_workspace_for(c, M, N) : workspace_for(c, M, N);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned16(workspace))) return QF_ERR_WORKSPACE;

  GemmArgs a;
  a.x = x;
  a.w = w;
  a.scale = scale;
  a.y = y;
  a.counters = reinterpret_cast<unsigned*>(workspace);
  a.counter_stride = counter_stride_for(workgroups(c, N));
  a.partial = need > 0 && am == nullptr
                  ? reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + QF_W8A16_COUNTER_BYTES)
                  : nullptr;
  a.ldx = ldx;
  a.ldw = ldw;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.n_pad = round_up16(N);
  a.ksteps = K / kStepK;
  a.split_k = c.split_k;
  a.out_f32 = out_dtype == QF_DTYPE_F32;
  a.vec_out = (ldy % 4) == 0;
  a.fused_reduce = is_mfma(c.kernel) && c.reduce == 0;
  a.tiles_strided = c.kernel == QF_KERNEL_MFMA_STREAM && (c.reduce & 2) != 0;
  a.norm_eps = norm_eps != nullptr ? *norm_eps : 0.f;
  a.argmax = am != nullptr;
  a.n_valid = am != nullptr ? am->n_valid : 0;
  a.index_offset = am != nullptr ? am->index_offset : 0;
  a.ids = am != nullptr ? am->ids : nullptr;
  a.am_slots = am != nullptr ? reinterpret_cast<uint64_t*>(workspace) : nullptr;
  a.groups = 1;
  a.group_rows = M;
  if (c.kernel == QF_KERNEL_MFMA_WIDE) wide_groups(M, a.groups, a.group_rows);

  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid = c.kernel == QF_KERNEL_MFMA_WIDE ? dim3(workgroups(c, N) * a.groups * c.split_k)
                                                    : dim3(workgroups(c, N), c.split_k);
  const dim3 block(c.waves * kWave);
  const size_t smem = lds_bytes(c, M, a.ksteps, N);
  KernelFn fn = (c.kernel == QF_KERNEL_GEMV)
                    ? select_gemv(M, c.tiles_per_wave, c.waves, c.load_hint)
                : (c.kernel == QF_KERNEL_MFMA_STREAM)
                    ? ((c.reduce & 1) ? select_stream_xreg(c.waves, c.depth, a.ksteps)
                                     : select_stream(c.waves, c.depth, c.load_hint))
                : (c.kernel == QF_KERNEL_MFMA_WIDE)
                    ? select_wide(c.tiles_per_wave, a.group_rows / 16, c.waves, c.depth)
                    : select_mfma(layout, c.tiles_per_wave, c.waves, c.k_waves, c.depth, c.load_hint,
                                  c.kernel == QF_KERNEL_MFMA_XRING);
  if (norm_eps != nullptr) fn = select_norm(c, layout);
  if (fn == nullptr) return QF_ERR_UNSUPPORTED;
  int st = launch(fn, grid, block, smem, s, a);
  if (st != QF_OK) return st;
  if (am != nullptr) {
    hipLaunchKernelGGL(argmax_slots_kernel, dim3(M), dim3(kWave), 0, s, a.am_slots, a.index_offset, a.ids);
    return hipGetLastError() == hipSuccess ? QF_OK : QF_ERR_HIP;
  }
  if (c.split_k > 1 && !a.fused_reduce) {
    const int threads = M * (a.n_pad / 4);
    st = launch(&splitk_reduce_kernel, dim3(ceil_div(threads, 256)), dim3(256), 0, s, a);
  }
  return st;
}

// ---------------------------------------------------------------------------------------------
// W8A8 GEMM on TILED weights (QF_KERNEL_MFMA_W8A8)
// ---------------------------------------------------------------------------------------------

// Instantiations: NT {2, 4} x MT {1..4} x WN {4, 8} x DEPTH {2, 4}, and MT {5..8} for NT 2.
template <int NT, int MT>
KernelFn w8a8_by_shape(int wn, int depth) {
  if (wn == 4 && depth == 2) return &w8a8_wide_kernel<QF_LAYOUT_TILED, NT, MT, 4, 2>;
  if (wn == 4 && depth == 4) return &w8a8_wide_kernel<QF_LAYOUT_TILED, NT, MT, 4, 4>;
  if (wn == 8 && depth == 2) return &w8a8_wide_kernel<QF_LAYOUT_TILED, NT, MT, 8, 2>;
  if (wn == 8 && depth == 4) return &w8a8_wide_kernel<QF_LAYOUT_TILED, NT, MT, 8, 4>;
  return nullptr;
}

// Row-major weights: the automatic shape only (2 tiles, 8 wavefronts, DEPTH 4), MT {1..8}.
KernelFn w8a8_rowmajor(int nt, int mt, int waves, int depth) {
  if (nt != 2 || waves != 8 || depth != 4) return nullptr;
  switch (mt) {
    case 1: return &w8a8_wide_kernel<QF_LAYOUT_ROWMAJOR, 2, 1, 8, 4>;
    case 2: return &w8a8_wide_kernel<QF_LAYOUT_ROWMAJOR, 2, 2, 8, 4>;
    case 3: return &w8a8_wide_kernel<QF_LAYOUT_ROWMAJOR, 2, 3, 8, 4>;
    case 4: return &w8a8_wide_kernel<QF_LAYOUT_ROWMAJOR, 2, 4, 8, 4>;
    case 5: return &w8a8_wide_kernel<QF_LAYOUT_ROWMAJOR, 2, 5, 8, 4>;
    case 6: return &w8a8_wide_kernel<QF_LAYOUT_ROWMAJOR, 2, 6, 8, 4>;
    case 7: return &w8a8_wide_kernel<QF_LAYOUT_ROWMAJOR, 2, 7, 8, 4>;
    case 8: return &w8a8_wide_kernel<QF_LAYOUT_ROWMAJOR, 2, 8, 8, 4>;
    default: return nullptr;
  }
}

template <int NT>
KernelFn w8a8_by_mt(int mt, int wn, int depth) {
  switch (mt) {
    case 1: return w8a8_by_shape<NT, 1>(wn, depth);
    case 2: return w8a8_by_shape<NT, 2>(wn, depth);
    case 3: return w8a8_by_shape<NT, 3>(wn, depth);
    case 4: return w8a8_by_shape<NT, 4>(wn, depth);
    default: break;
  }
  if constexpr (NT == 2) {
    switch (mt) {
      case 5: return w8a8_by_shape<NT, 5>(wn, depth);
      case 6: return w8a8_by_shape<NT, 6>(wn, depth);
      case 7: return w8a8_by_shape<NT, 7>(wn, depth);
      case 8: return w8a8_by_shape<NT, 8>(wn, depth);
      default: break;
    }
  }
  return nullptr;
}

KernelFn select_w8a8(int layout, int nt, int mt, int waves, int depth) {
  if (layout == QF_LAYOUT_ROWMAJOR) return w8a8_rowmajor(nt, mt, waves, depth);
  if (nt == 2) return w8a8_by_mt<2>(mt, waves, depth);
  if (nt == 4) return w8a8_by_mt<4>(mt, waves, depth);
  return nullptr;
}

// Token groups of the W8A8 kernel.  Without the conversion work the int8 MFMAs go twice as fast as the
// bf16 ones, and then 64-row groups leave a workgroup's k-step short of work for the weight bytes it
// loads: groups of up to 128 rows are used once the workgroups they give number 128 or more (gate_up
// M = 2048: 420 us against 552; o_proj M = 1024: 65 against 87), 64-row groups below that (narrow N at
// small M needs the workgroups; there the K split fills the machine instead).
void w8a8_groups(const qf_w8a16_config& c, int M, int N, int& groups, int& group_rows) {
  const int blocks = workgroups(c, N);
  const int max_rows = (c.tiles_per_wave == 2 && (int64_t)blocks * ((M + 127) / 128) >= 128) ? 128 : 64;
  const int g0 = (M + max_rows - 1) / max_rows;
  group_rows = ((M + g0 - 1) / g0 + 15) / 16 * 16;
  groups = (M + group_rows - 1) / group_rows;
}

// LDS of one workgroup: two chunks of the group's rows, (depth + 1) 64-byte steps and a 16-byte pad each.
size_t w8a8_lds_bytes(const qf_w8a16_config& c, int M, int N) {
  int groups, rows;
  w8a8_groups(c, M, N, groups, rows);
  return (size_t)2 * rows * ((c.depth + 1) * kStepK + 16);
}

// The tile kernel's grid: 256-channel x 256-token workgroups.
int64_t w8a8_tile_workgroups(int M, int N) {
  return (int64_t)ceil_div(round_up16(N) / kTileN, kW8A8TileTiles) * ceil_div(M, kW8A8TileRows);
}

int validate_w8a8(int M, int N, int K, int layout, const qf_w8a16_config& c) {
  if (M < 1 || N < 1 || K < QF_W8A16_K_ALIGN) return QF_ERR_INVALID_ARG;
  const int ksteps = K / kStepK;
  if (c.kernel == QF_KERNEL_MFMA_W8A8_TILE) {
    if (c.split_k < 1 || c.split_k > kW8A8TileMaxSplit || c.waves != 8 || c.tiles_per_wave != 8 ||
        c.depth != kW8A8TileStages || c.k_waves != 1 || c.reduce < 0 || c.reduce > 3 || (c.reduce == 3 && c.split_k != 1))
      return QF_ERR_INVALID_ARG;
    if ((layout != QF_LAYOUT_TILED && layout != QF_LAYOUT_ROWMAJOR) || K >= 132000) return QF_ERR_UNSUPPORTED;
    const int64_t twgs = w8a8_tile_workgroups(M, N);
    if (twgs * c.split_k > 0x7fffffff) return QF_ERR_UNSUPPORTED;
    // A K split needs a step per split and one arrival counter per tile.
    if (c.split_k > 1 && (c.split_k > ksteps || twgs * 4 > QF_W8A16_COUNTER_BYTES)) return QF_ERR_UNSUPPORTED;
    return QF_OK;
  }
  if (c.kernel != QF_KERNEL_MFMA_W8A8) return QF_ERR_INVALID_ARG;
  if (c.split_k < 1 || c.split_k > ksteps || c.waves < 1 || c.k_waves < 1 || c.tiles_per_wave < 1)
    return QF_ERR_INVALID_ARG;
  if ((layout != QF_LAYOUT_TILED && layout != QF_LAYOUT_ROWMAJOR) || c.k_waves != 1 || K >= 132000)
    return QF_ERR_UNSUPPORTED;
  int groups, rows;
  w8a8_groups(c, M, N, groups, rows);
  if ((int64_t)workgroups(c, N) * groups * c.split_k > 0x7fffffff) return QF_ERR_UNSUPPORTED;
  if (select_w8a8(layout, c.tiles_per_wave, rows / 16, c.waves, c.depth) == nullptr) return QF_ERR_UNSUPPORTED;
  return w8a8_lds_bytes(c, M, N) > kMaxLds ? QF_ERR_UNSUPPORTED : QF_OK;
}

// Automatic W8A8 configuration (either layout, any M): 8 wavefronts of 2 tiles, 4 steps in flight, and
// K split across workgroups until they number 128 (at most 8 ways and 16 steps a split), with the two
// exceptions below.  Measured on the dense 27B-class layer's four shapes at M = 17 .. 2048 against
// 2- and 4-tile, 4- and 8-wavefront shapes at depth 2 and 4 and splits of 1, 2 and 4: the best shape
// or within 5% of it everywhere (down M = 512: 106.9 us against 101.7 split in four).
bool auto_config_w8a8_wide(int M, int N, int K, int layout, qf_w8a16_config* c);

bool auto_config_w8a8(int M, int N, int K, int layout, qf_w8a16_config* c) {
  if (M < 1 || N < 1 || K < QF_W8A16_K_ALIGN || K % QF_W8A16_K_ALIGN) return false;
  if (layout != QF_LAYOUT_TILED && layout != QF_LAYOUT_ROWMAJOR) return false;
  *c = qf_w8a16_config{};
  c->kernel = QF_KERNEL_MFMA_W8A8;
  c->k_waves = 1;
  c->load_hint = 1;
  c->reduce = 1;
  c->split_k = 1;
  c->tiles_per_wave = 2;
  c->waves = 8;
  c->depth = 4;
  // The LDS-tiled kernel once its 256 x 256 workgroups number 136 or more, unless they spill a few
  // (<= 16) past a whole round of 256 that the second launch of run_w8a8 cannot take (measured on the
  // four layer shapes at M = 256 .. 4096 with token-tiled activations against the shapes below: gate_up
  // M = 512 (272 workgroups, the last 16 on the wide kernel) 107 against 148 us, M = 2048 301 against
  // 420; slower with fewer workgroups, where the shapes below split K: down M = 1024 (80) 172 against
  // 152, o_proj M = 1536 (120) 91 against 87).  Its token blocks are 256 rows whatever M is, so it also
  // needs M >= 256 with under a quarter of the rows it computes past M (gate_up M = 384: 109 against 102),
  // or one token block above 128 rows, where the shapes below go to two token groups a channel block
  // (gate_up M = 129 / 160 / 208 / 255: 61.9 / 63.0 / 67.4 / 68.1 us against 76.0 / 77.9 / 93.5 / 100.3;
  // M = 112: 66.1 against 52.1).
  const int64_t twgs = w8a8_tile_workgroups(M, N);
  const int mblocks = ceil_div(M, kW8A8TileRows);
  const int64_t tile_rows = (int64_t)mblocks * kW8A8TileRows;
  const int64_t rest = twgs % 256, whole = twgs - rest;
  // A second launch only takes a true remainder: 0 < rest <= 64 workgroups past whole rounds.
  const bool second_launch = whole > 0 && rest > 0 && rest <= 64 && whole % mblocks == 0;
  const bool rows_ok = (M >= kW8A8TileRows && 4 * (int64_t)M > 3 * tile_rows) || (mblocks == 1 && M > 128);
  if (K < 132000 && rows_ok && twgs >= 136 && !(whole > 0 && rest != 0 && rest <= 16 && !second_launch)) {
    c->kernel = QF_KERNEL_MFMA_W8A8_TILE;
    c->tiles_per_wave = 8;
    c->waves = 8;
    c->depth = kW8A8TileStages;
    c->reduce = 0;  // the tile kernel's tail rule (run_w8a8)
    return validate_w8a8(M, N, K, layout, *c) == QF_OK;
  }
  // 289 to 384 rows, where two token blocks of 256 would be under three-quarters full and three of 128 are
  // not, on grids of 136 or more 256 x 256 workgroups: 256-channel x 128-token workgroups (reduce 3; gate_up
  // M = 320 / 352 / 384 93.3 / 95.0 / 96.5 us against 102.1 / 111.6 / 112.3 on the shapes below; M = 272
  // 95.0 against 90.9, M = 416 131.9 against 112.1 on the 256-token kernel).
  if (K < 132000 && M > 288 && M <= 384 && twgs >= 136) {
    c->kernel = QF_KERNEL_MFMA_W8A8_TILE;
    c->tiles_per_wave = 8;
    c->waves = 8;
    c->depth = kW8A8TileStages;
    c->reduce = 3;
    return validate_w8a8(M, N, K, layout, *c) == QF_OK;
  }
  // 40 to 128 256 x 256 workgroups (measured from 40), with two or more token blocks: the tile kernel with K split
  // s = min(4, K / 2560, 256 / workgroups) ways (at least 40 k-steps a split) and the fused reduction.  Each
  // split moves a 256 KiB int32 partial through memory, so short K and one token block stay below
  // (token-tiled activations against the shapes below, us: down 5120 x 17408 at M = 512 / 768 / 1024 / 1536
  // 77.3 / 97.0 / 113.2 / 146.3 against 106.5 / 110.4 / 149.8 / 169.4; o_proj 5120 x 8192 53.6 / 57.7 / 68.8
  // / 81.3 against 55.9 / 56.7 / 79.4 / 87.0; qkv 10240 x 5120 at M = 512 / 768 49.8 / 59.6 against 54.5 /
  // 59.4; at M = 256 the shapes below win: down 67 against 68, o_proj 43 against 48, qkv 38 against 43).
  const int64_t sk = std::min<int64_t>(std::min(4, K / 2560), twgs > 0 ? 256 / twgs : 0);
  // Three or more token blocks at most three-quarters full take it too when K is long (>= 10240), where the
  // shapes below would run every workgroup over the whole K: down M = 520 / 544 / 576 87.0 / 89.8 / 89.2 us
  // against 113.9 / 113.9 / 113.8 (o_proj 56-60 against 58-59, qkv 57-60 against 52-58 stay below).
  const bool split_rows = 4 * (int64_t)M > 3 * tile_rows || (mblocks >= 3 && K >= 10240);
  if (K < 132000 && mblocks >= 2 && split_rows && twgs >= 40 && twgs <= 128 && sk >= 2) {
    c->kernel = QF_KERNEL_MFMA_W8A8_TILE;
    c->split_k = (int)sk;
    c->tiles_per_wave = 8;
    c->waves = 8;
    c->depth = kW8A8TileStages;
    c->reduce = 0;
    if (validate_w8a8(M, N, K, layout, *c) == QF_OK) return true;
    c->split_k = 1;
    c->kernel = QF_KERNEL_MFMA_W8A8;
    c->tiles_per_wave = 2;
    c->depth = 4;
    c->reduce = 1;
  }
  return auto_config_w8a8_wide(M, N, K, layout, c);
}

// The automatic QF_KERNEL_MFMA_W8A8 shape (c holds the defaults set above).
bool auto_config_w8a8_wide(int M, int N, int K, int layout, qf_w8a16_config* c) {
  if (M < 1 || N < 1 || K < QF_W8A16_K_ALIGN) return false;
  int groups, rows;
  w8a8_groups(*c, M, N, groups, rows);
  const int64_t wgs = (int64_t)workgroups(*c, N) * groups;
  const int ksteps = K / kStepK;
  if (layout == QF_LAYOUT_TILED && wgs < 128 && ksteps <= 128) {
    // 4-wavefront workgroups, unsplit, where they number 128 .. 255 and the 8-wavefront ones would
    // need a K split (qkv M = 128: 28.3 us against 32.4; o_proj M = 256: 37.2 against 38.7).
    qf_w8a16_config c4 = *c;
    c4.waves = 4;
    int groups4, rows4;
    w8a8_groups(c4, M, N, groups4, rows4);
    const int64_t wgs4 = (int64_t)workgroups(c4, N) * groups4;
    if (wgs4 >= 128 && wgs4 < 256) {
      *c = c4;
      return validate_w8a8(M, N, K, layout, *c) == QF_OK;
    }
  }
  while (wgs * c->split_k < 128 && c->split_k < 8 && ksteps / (c->split_k + 1) >= 16) ++c->split_k;
  // 128-row workgroups run one per CU.  On a long K range, a grid whose last round leaves the 256 CUs at
  // most a quarter busy is split in two (down M = 2048, 320 workgroups: 268 us against 290).
  if (c->split_k == 1 && rows == 128 && ksteps >= 256 && wgs > 256 && wgs % 256 != 0 && wgs % 256 <= 64)
    c->split_k = 2;
  return validate_w8a8(M, N, K, layout, *c) == QF_OK;
}

int resolve_w8a8(int M, int N, int K, int layout, const qf_w8a16_config* in, qf_w8a16_config* out) {
  if (!auto_config_w8a8(M, N, K, layout, out)) return QF_ERR_UNSUPPORTED;
  if (in == nullptr || in->kernel == QF_KERNEL_AUTO) return QF_OK;
  qf_w8a16_config c = *in;
  const bool tile = c.kernel == QF_KERNEL_MFMA_W8A8_TILE;
  if (c.waves == 0) c.waves = tile ? 8 : 4;
  if (c.k_waves == 0) c.k_waves = 1;
  if (c.tiles_per_wave == 0) c.tiles_per_wave = tile ? 8 : 4;
  if (c.depth == 0) c.depth = tile ? kW8A8TileStages : 4;
  if (c.split_k == 0) c.split_k = 1;
  const int rc = validate_w8a8(M, N, K, layout, c);
  if (rc != QF_OK) return rc;
  *out = c;
  return QF_OK;
}

// The launches of one W8A8 call, in stream order.  Each covers output channels [n0, n0 + n) of the call
// (all token rows), so the launches of a call write disjoint columns; the sums are exact integer sums, so
// how the channels are divided does not change the result.
enum W8a8LaunchKind {
  kW8a8Tile = 0,         // w8a8_tile_kernel, 256 x 256 workgroups (n a multiple of 256 when a tail follows)
  kW8a8TileHalf = 1,     // w8a8_tile_kernel, 256-channel x 128-token workgroups (reduce 3)
  kW8a8TileSmall = 2,    // w8a8_tile_kernel, 128 x 128 workgroups (the tail round)
  kW8a8Wide = 3,         // w8a8_wide_kernel with the launch's own cfg
  kW8a8SplitReduce = 4,  // splitk_reduce_w8a8_kernel after a K-split wide launch
};
struct W8a8Launch {
  int kind;
  int64_t grid;  // workgroups
  int n0, n;     // output channels of this launch
  qf_w8a16_config cfg;
};

// Fills out[0..1] with the call's launches and returns their number (1 or 2), or -(qf_status).
int w8a8_plan(int M, int N, int K, int layout, const qf_w8a16_config& c, W8a8Launch out[2]) {
  if (M < 1 || N < 1 || K < QF_W8A16_K_ALIGN) return -QF_ERR_INVALID_ARG;
  const int n_pad = round_up16(N);
  out[0] = W8a8Launch{kW8a8Tile, 0, 0, N, c};
  if (c.kernel == QF_KERNEL_MFMA_W8A8_TILE) {
    // Tail (reduce 0 or 2): when the 256 x 256 workgroups fill whole rounds of 256 and then a quarter round
    // or less, the channel blocks of the whole rounds run in the first launch and the remaining channels in
    // a second launch on the same stream: one round of 128 x 128 workgroups of the same kernel where they
    // number 128 to 256 (reduce 0), else (or with reduce 2) the wide kernel.  Token-tiled activations,
    // gate_up M = 2048 (1024 workgroups, 2048 channels left): 304.5 us, 323.1 with the wide kernel's tail,
    // 316.3 in one launch; qkv M = 2048: 92.1 / 112.9 / 111.9 us.  Past a quarter round one launch is
    // faster (gate_up M = 4096, 128 past 2048: 600 us, 613 with two rounds of 128 x 128 workgroups).
    const int nblocks = ceil_div(n_pad / kTileN, kW8A8TileTiles);
    const int mblocks = ceil_div(M, kW8A8TileRows);
    const int64_t twgs = (int64_t)nblocks * mblocks;
    if (c.split_k > 1) {  // K split with the fused last-arrival reduction: one launch
      out[0].grid = twgs * c.split_k;
      return 1;
    }
    if (c.reduce == 3) {  // 256-channel x 128-token workgroups, one launch
      out[0].kind = kW8a8TileHalf;
      out[0].grid = (int64_t)nblocks * ceil_div(M, TileShape<8, 2>::rows);
      return 1;
    }
    out[0].grid = twgs;
    const int64_t whole = twgs / 256 * 256;
    // Only a true remainder (0 < rest <= 64) is split off: with rest == 0 the whole rounds already hold
    // every channel block, and their channel count nblocks * 256 may exceed N.
    const int64_t rest = twgs - whole;
    if (c.reduce == 1 || whole == 0 || rest == 0 || rest > 64 || whole % mblocks != 0) return 1;
    const int n_main = (int)(whole / mblocks) * kW8A8TileTiles * kTileN;  // < N: the tail holds N's last block
    const int n_tail = N - n_main;
    if (n_main <= 0 || n_tail <= 0) return 1;  // not reached when rest > 0: one launch covers N
    using Small = TileShape<4>;
    const int64_t small = (int64_t)ceil_div(round_up16(n_tail) / kTileN, Small::tiles) * ceil_div(M, Small::rows);
    W8a8Launch tail{kW8a8TileSmall, small, n_main, n_tail, c};
    if (!(c.reduce == 0 && small >= 128 && small <= 256)) {
      qf_w8a16_config ct = qf_w8a16_config{};
      ct.kernel = QF_KERNEL_MFMA_W8A8;
      ct.k_waves = 1;
      ct.load_hint = 1;
      ct.reduce = 1;
      ct.split_k = 1;
      ct.tiles_per_wave = 2;
      ct.waves = 8;
      ct.depth = 4;
      if (!auto_config_w8a8_wide(M, n_tail, K, layout, &ct)) return 1;
      ct.split_k = 1;  // no workspace: the tail runs unsplit
      if (validate_w8a8(M, n_tail, K, layout, ct) != QF_OK) return 1;
      int groups, rows;
      w8a8_groups(ct, M, n_tail, groups, rows);
      tail = W8a8Launch{kW8a8Wide, (int64_t)workgroups(ct, n_tail) * groups, n_main, n_tail, ct};
    }
    out[0].grid = whole;
    out[0].n = n_main;
    out[1] = tail;
    return 2;
  }
  int groups, rows;
  w8a8_groups(c, M, N, groups, rows);
  out[0] = W8a8Launch{kW8a8Wide, (int64_t)workgroups(c, N) * groups * c.split_k, 0, N, c};
  if (c.split_k == 1) return 1;
  out[1] = W8a8Launch{kW8a8SplitReduce, ceil_div(M * (n_pad / 4), 256), 0, N, c};
  return 2;
}

// x_tiled: xq is the token-tiled image (ldq unused).
int run_w8a8(const int8_t* xq, int64_t ldq, int x_tiled, const float* s_a, const int8_t* w, int64_t ldw, int layout,
             const float* scale, void* y, int64_t ldy, int out_dtype, int M, int N, int K, const qf_w8a16_config* cfg,
             void* workspace, size_t workspace_bytes, void* stream) {
  if (x_tiled) ldq = K;
  if (xq == nullptr || s_a == nullptr || w == nullptr || scale == nullptr || y == nullptr) return QF_ERR_INVALID_ARG;
  if (M < 1 || N < 1 || K < 1 || ldq < K || ldy < N) return QF_ERR_INVALID_ARG;
  if (layout != QF_LAYOUT_ROWMAJOR && layout != QF_LAYOUT_TILED) return QF_ERR_INVALID_ARG;
  if (out_dtype != QF_DTYPE_BF16 && out_dtype != QF_DTYPE_F32) return QF_ERR_INVALID_ARG;
  if (layout == QF_LAYOUT_ROWMAJOR && ldw < K) return QF_ERR_INVALID_ARG;
  if (K % QF_W8A16_K_ALIGN || (layout == QF_LAYOUT_ROWMAJOR && ldw % 16)) return QF_ERR_UNSUPPORTED;
  if (!aligned16(xq) || !aligned16(w) || !aligned16(scale) || !aligned16(y) || ldq % 16) return QF_ERR_UNSUPPORTED;
  qf_w8a16_config c;
  const int rc = resolve_w8a8(M, N, K, layout, cfg, &c);
  if (rc != QF_OK) return rc;
  const size_t need = workspace_for(c, M, N);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned16(workspace))) return QF_ERR_WORKSPACE;

  GemmArgs a{};
  a.xq = xq;
  a.s_tok = s_a;
  a.x_tiled = x_tiled ? 1 : 0;
  a.w = w;
  a.scale = scale;
  a.y = y;
  a.partial = need > 0 ? reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + QF_W8A16_COUNTER_BYTES)
                       : nullptr;
  a.counters = need > 0 ? reinterpret_cast<unsigned*>(workspace) : nullptr;
  a.counter_stride = 1;
  a.ldx = ldq;
  a.ldw = ldw;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.n_pad = round_up16(N);
  a.ksteps = K / kStepK;
  a.split_k = c.split_k;
  a.out_f32 = out_dtype == QF_DTYPE_F32;
  a.vec_out = (ldy % 4) == 0;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  W8a8Launch plan[2];
  const int nl = w8a8_plan(M, N, K, layout, c, plan);
  if (nl < 1) return nl < 0 ? -nl : QF_ERR_UNSUPPORTED;
  const bool rm = layout == QF_LAYOUT_ROWMAJOR;
  for (int i = 0; i < nl; ++i) {
    const W8a8Launch& p = plan[i];
    GemmArgs al = a;
    if (p.n0 != 0 || p.n != N) {  // a channel range of the call: its weights, scales and output columns
      al.N = p.n;
      al.n_pad = p.kind == kW8a8Tile ? p.n : round_up16(p.n);
      al.w = a.w + (layout == QF_LAYOUT_TILED ? (int64_t)(p.n0 / kTileN) * a.ksteps * kTileN * kStepK
                                              : (int64_t)p.n0 * a.ldw);
      al.scale = a.scale + p.n0;
      al.y = reinterpret_cast<uint8_t*>(a.y) + (size_t)p.n0 * (a.out_f32 ? 4 : 2);
    }
    if (p.kind == kW8a8Tile || p.kind == kW8a8TileHalf || p.kind == kW8a8TileSmall)
      al.counter_stride = counter_stride_for((int)(p.grid / (a.split_k > 0 ? a.split_k : 1)));
    int st = QF_ERR_UNSUPPORTED;
    switch (p.kind) {
      case kW8a8Tile:
        st = launch(rm ? &w8a8_tile_kernel<QF_LAYOUT_ROWMAJOR, 8> : &w8a8_tile_kernel<QF_LAYOUT_TILED, 8>,
                    dim3((unsigned)p.grid), dim3(8 * kWave), kW8A8TileLds, s, al);
        break;
      case kW8a8TileHalf:
        st = launch(rm ? &w8a8_tile_kernel<QF_LAYOUT_ROWMAJOR, 8, 2> : &w8a8_tile_kernel<QF_LAYOUT_TILED, 8, 2>,
                    dim3((unsigned)p.grid), dim3(8 * kWave), TileShape<8, 2>::lds, s, al);
        break;
      case kW8a8TileSmall:
        st = launch(rm ? &w8a8_tile_kernel<QF_LAYOUT_ROWMAJOR, 4> : &w8a8_tile_kernel<QF_LAYOUT_TILED, 4>,
                    dim3((unsigned)p.grid), dim3(8 * kWave), TileShape<4>::lds, s, al);
        break;
      case kW8a8Wide: {
        w8a8_groups(p.cfg, M, p.n, al.groups, al.group_rows);
        KernelFn fn = select_w8a8(layout, p.cfg.tiles_per_wave, al.group_rows / 16, p.cfg.waves, p.cfg.depth);
        if (fn == nullptr) return QF_ERR_UNSUPPORTED;
        al.split_k = p.cfg.split_k;
        st = launch(fn, dim3((unsigned)p.grid), dim3(p.cfg.waves * kWave), w8a8_lds_bytes(p.cfg, M, p.n), s, al);
        break;
      }
      case kW8a8SplitReduce:
        st = launch(&splitk_reduce_w8a8_kernel, dim3((unsigned)p.grid), dim3(256), 0, s, al);
        break;
      default:
        return QF_ERR_UNSUPPORTED;
    }
    if (st != QF_OK) return st;
  }
  return QF_OK;
}

int argmax_rows(const uint16_t* logits, int64_t ld, int M, int N, int n_valid, int64_t index_offset, int64_t* out,
                const ArgmaxTable* tab, void* stream);

// ---------------------------------------------------------------------------------------------
// Static scratch of qf_w8a16_gemm_noalloc: the split-K workspace (arrival counters, then the fp32
// partials) for callers that cannot allocate.  Every device the library runs on holds one copy until
// the process ends.  Host code never uses the array's name as an address: it takes the device address
// hipGetSymbolAddress returns, once per device with that device current, and passes that pointer.
// ---------------------------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[QF_W8A16_SCRATCH_BYTES];

__global__ void __launch_bounds__(256) clear_words_kernel(unsigned* p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];

// The current device's scratch address.  The first call on a device fetches it and clears the arrival
// counters with a kernel on `stream`, ahead of the call's own launches (the array is zero at load, and
// every GEMM returns the counters it uses to zero).
int device_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return QF_ERR_HIP;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return QF_ERR_HIP;
    constexpr int words = QF_W8A16_COUNTER_BYTES / 4;
    hipLaunchKernelGGL(clear_words_kernel, dim3(ceil_div(words, 256)), dim3(256), 0, stream,
                       reinterpret_cast<unsigned*>(p), words);
    if (hipGetLastError() != hipSuccess) return QF_ERR_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return QF_OK;
}

}  // namespace qf

using namespace qf;

extern "C" {

int qf_abi_version(void) { return QF_W8A16_ABI_VERSION; }

const char* qf_status_string(int status) {
  switch (status) {
    case QF_OK: return "ok";
    case QF_ERR_INVALID_ARG: return "invalid argument";
    case QF_ERR_UNSUPPORTED: return "unsupported shape, layout or alignment (use the fallback path)";
    case QF_ERR_WORKSPACE: return "workspace missing or too small";
    case QF_ERR_HIP: return "HIP runtime error";
    default: return "unknown status";
  }
}

int qf_w8a16_pick_config(int M, int N, int K, int layout, qf_w8a16_config* cfg) {
  if (cfg == nullptr) return QF_ERR_INVALID_ARG;
  return auto_config(M, N, K, layout, cfg) ? QF_OK : QF_ERR_UNSUPPORTED;
}

size_t qf_w8a16_workspace_bytes(int M, int N, int K, int layout, const qf_w8a16_config* cfg) {
  qf_w8a16_config c;
  if (resolve_config(M, N, K, layout, cfg, &c) != QF_OK) return 0;
  return workspace_for(c, M, N);
}

size_t qf_w8a16_tiled_bytes(int N, int K) {
  if (N < 1 || K < 1) return 0;
  return (size_t)round_up16(N) * (size_t)K;
}

int qf_w8a16_gemm(const uint16_t* x, int64_t ldx, const int8_t* w, int64_t ldw, int layout, const float* scale,
                  void* y, int64_t ldy, int out_dtype, int M, int N, int K, const qf_w8a16_config* cfg,
                  void* workspace, size_t workspace_bytes, void* stream) {
  if (y == nullptr) return QF_ERR_INVALID_ARG;
  return run_gemm(x, ldx, w, ldw, layout, scale, y, ldy, out_dtype, M, N, K, cfg, workspace, workspace_bytes, stream,
                  nullptr);
}

int qf_w8a16_gemm_rmsnorm(const uint16_t* x, int64_t ldx, float eps, const int8_t* w, int64_t ldw, int layout,
                          const float* scale, void* y, int64_t ldy, int out_dtype, int M, int N, int K,
                          const qf_w8a16_config* cfg, void* workspace, size_t workspace_bytes, void* stream) {
  if (!(eps >= 0.f) || K % 8) return QF_ERR_INVALID_ARG;
  return run_gemm(x, ldx, w, ldw, layout, scale, y, ldy, out_dtype, M, N, K, cfg, workspace, workspace_bytes, stream,
                  nullptr, &eps);
}

int qf_w8a16_gemm_noalloc(const uint16_t* x, int64_t ldx, const int8_t* w, int64_t ldw, int layout, const float* scale,
                          void* y, int64_t ldy, int out_dtype, int M, int N, int K, const qf_w8a16_config* cfg,
                          void* stream) {
  const size_t need = qf_w8a16_workspace_bytes(M, N, K, layout, cfg);
  if (need > QF_W8A16_SCRATCH_BYTES) return QF_ERR_WORKSPACE;
  void* ws = nullptr;
  if (need > 0) {
    const int rc = device_scratch(reinterpret_cast<hipStream_t>(stream), &ws);
    if (rc != QF_OK) return rc;
  }
  return run_gemm(x, ldx, w, ldw, layout, scale, y, ldy, out_dtype, M, N, K, cfg, ws,
                  ws != nullptr ? QF_W8A16_SCRATCH_BYTES : 0, stream, nullptr);
}

size_t qf_w8a16_argmax_workspace_bytes(int M, int N, int K, int layout, const qf_w8a16_config* cfg) {
  qf_w8a16_config c;
  if (resolve_config(M, N, K, layout, cfg, &c, false) != QF_OK) return 0;
  if (!is_mfma(c.kernel) || c.split_k != 1) return 0;
  return argmax_workspace_for(c, M, N);
}

int qf_w8a16_gemm_argmax(const uint16_t* x, int64_t ldx, const int8_t* w, int64_t ldw, int layout, const float* scale,
                         void* y, int64_t ldy, int out_dtype, int M, int N, int K, int n_valid, int64_t index_offset,
                         int64_t* ids, const qf_w8a16_config* cfg, void* workspace, size_t workspace_bytes,
                         void* stream) {
  if (ids == nullptr || n_valid < 1 || n_valid > N) return QF_ERR_INVALID_ARG;
  ArgmaxRequest am{n_valid, index_offset, ids};
  return run_gemm(x, ldx, w, ldw, layout, scale, y, ldy, out_dtype, M, N, K, cfg, workspace, workspace_bytes, stream,
                  &am);
}

int qf_w8a16_repack(const int8_t* w_rowmajor, int64_t ldw, int8_t* w_tiled, int N, int K, void* stream) {
  if (w_rowmajor == nullptr || w_tiled == nullptr || N < 1 || K < 1 || ldw < K) return QF_ERR_INVALID_ARG;
  if (K % QF_W8A16_K_ALIGN || ldw % 16 || !aligned16(w_rowmajor) || !aligned16(w_tiled)) return QF_ERR_UNSUPPORTED;
  const int ksteps = K / kStepK;
  const int64_t pieces = (int64_t)(round_up16(N) / kTileN) * ksteps * kWave;
  const int64_t blocks = (pieces + 255) / 256;
  hipLaunchKernelGGL(repack_kernel<false>, dim3((unsigned)blocks), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), w_rowmajor, w_tiled, ldw, N, ksteps, pieces);
  return hipGetLastError() == hipSuccess ? QF_OK : QF_ERR_HIP;
}

int qf_w8a16_unpack(const int8_t* w_tiled, int8_t* w_rowmajor, int64_t ldw, int N, int K, void* stream) {
  if (w_rowmajor == nullptr || w_tiled == nullptr || N < 1 || K < 1 || ldw < K) return QF_ERR_INVALID_ARG;
  if (K % QF_W8A16_K_ALIGN || ldw % 16 || !aligned16(w_rowmajor) || !aligned16(w_tiled)) return QF_ERR_UNSUPPORTED;
  const int ksteps = K / kStepK;
  const int64_t pieces = (int64_t)(round_up16(N) / kTileN) * ksteps * kWave;
  const int64_t blocks = (pieces + 255) / 256;
  hipLaunchKernelGGL(repack_kernel<true>, dim3((unsigned)blocks), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), w_tiled, w_rowmajor, ldw, N, ksteps, pieces);
  return hipGetLastError() == hipSuccess ? QF_OK : QF_ERR_HIP;
}

int qf_w8a16_dequant_bf16(const int8_t* w, int64_t ldw, int layout, int N, int K, int n0, int rows, uint16_t* out,
                          int64_t ldo, void* stream) {
  if (w == nullptr || out == nullptr || N < 1 || K < 1 || rows < 1 || n0 < 0 || (int64_t)n0 + rows > N || ldo < K)
    return QF_ERR_INVALID_ARG;
  if (layout != QF_LAYOUT_ROWMAJOR && layout != QF_LAYOUT_TILED) return QF_ERR_INVALID_ARG;
  if (layout == QF_LAYOUT_ROWMAJOR && ldw < K) return QF_ERR_INVALID_ARG;
  if (K % QF_W8A16_K_ALIGN || ldo % 8 || !aligned16(w) || !aligned16(out)) return QF_ERR_UNSUPPORTED;
  if (layout == QF_LAYOUT_ROWMAJOR && ldw % 16) return QF_ERR_UNSUPPORTED;
  const int ksteps = K / kStepK;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (layout == QF_LAYOUT_ROWMAJOR) {
    const int64_t pieces = (int64_t)rows * ksteps * 4;
    hipLaunchKernelGGL(dequant_rows_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, s, w, ldw, ksteps,
                       n0, pieces, out, ldo);
  } else {
    const int kgroups = ceil_div(ksteps, 4);
    const int64_t tiles = (int64_t)(n0 + rows + kTileN - 1) / kTileN - n0 / kTileN;
    hipLaunchKernelGGL(dequant_tiled_kernel, dim3((unsigned)(tiles * kgroups)), dim3(256), 0, s, w, ksteps, n0, rows,
                       kgroups, out, ldo);
  }
  return hipGetLastError() == hipSuccess ? QF_OK : QF_ERR_HIP;
}

int qf_scale_cast_bf16(const float* acc, int64_t lda, const float* scale, int M, int N, uint16_t* y, int64_t ldy,
                       void* stream) {
  if (acc == nullptr || scale == nullptr || y == nullptr || M < 1 || N < 1 || lda < N || ldy < N)
    return QF_ERR_INVALID_ARG;
  const int cpr = ceil_div(N, 8);
  const int64_t threads = (int64_t)M * cpr;
  const int vec = aligned16(acc) && aligned16(scale) && aligned16(y) && lda % 4 == 0 && ldy % 8 == 0;
  hipLaunchKernelGGL(scale_cast_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), acc, lda, scale, M, N, cpr, y, ldy, vec);
  return hipGetLastError() == hipSuccess ? QF_OK : QF_ERR_HIP;
}

int qf_rms_norm_rows_bf16(const uint16_t* x, int64_t ldx, int M, int N, float eps, uint16_t* y, int64_t ldy,
                          void* stream) {
  if (x == nullptr || y == nullptr || M < 1 || N < 1 || ldx < N || ldy < N || !(eps >= 0.f)) return QF_ERR_INVALID_ARG;
  if (N % 8 || !aligned16(x) || !aligned16(y) || ldx % 8 || ldy % 8) return QF_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(rms_norm_rows_kernel, dim3((unsigned)M), dim3(kWave), 0, reinterpret_cast<hipStream_t>(stream),
                     x, ldx, N, eps, y, ldy);
  return hipGetLastError() == hipSuccess ? QF_OK : QF_ERR_HIP;
}

int qf_quantize_rows_int8(const uint16_t* w, int64_t ldw, int8_t* q, float* s, int V, int H, void* stream) {
  if (w == nullptr || q == nullptr || s == nullptr || V < 1 || H < 1 || ldw < H) return QF_ERR_INVALID_ARG;
  if (aligned16(w) && ldw % 8 == 0 && H % 8 == 0 && H <= 8 * kQuantThreads * kQuantChunks && (uintptr_t)q % 8 == 0) {
    hipLaunchKernelGGL(quantize_rows_vec_kernel, dim3(V), dim3(kQuantThreads), 0, reinterpret_cast<hipStream_t>(stream),
                       w, ldw, q, s, H);
  } else {
    hipLaunchKernelGGL(quantize_rows_kernel, dim3(V), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), w, ldw,
                       q, s, H);
  }
  return hipGetLastError() == hipSuccess ? QF_OK : QF_ERR_HIP;
}

static int quantize_tokens(const uint16_t* x, int64_t ldx, int M, int K, int8_t* xq, int64_t ldq, float* s_a,
                           int tiled, void* stream) {
  if (x == nullptr || xq == nullptr || s_a == nullptr || M < 1 || K < 1 || ldx < K || ldq < K) return QF_ERR_INVALID_ARG;
  if (K % QF_W8A16_K_ALIGN || !aligned16(x) || ldx % 8 || (uintptr_t)xq % 8 || ldq % 8) return QF_ERR_UNSUPPORTED;
  if (tiled && !aligned16(xq)) return QF_ERR_UNSUPPORTED;
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int per_thread = ceil_div(K / 8, 256);  // 16-byte pieces a thread
  const dim3 grid(tiled ? round_up16(M) : M);
  if (per_thread <= 4)
    hipLaunchKernelGGL(quantize_tokens_kernel<4>, grid, dim3(256), 0, st, x, ldx, K, xq, ldq, s_a, M, tiled);
  else if (per_thread <= 12)
    hipLaunchKernelGGL(quantize_tokens_kernel<12>, grid, dim3(256), 0, st, x, ldx, K, xq, ldq, s_a, M, tiled);
  else
    hipLaunchKernelGGL(quantize_tokens_kernel<0>, grid, dim3(256), 0, st, x, ldx, K, xq, ldq, s_a, M, tiled);
  return hipGetLastError() == hipSuccess ? QF_OK : QF_ERR_HIP;
}

int qf_quantize_tokens_int8(const uint16_t* x, int64_t ldx, int M, int K, int8_t* xq, int64_t ldq, float* s_a,
                            void* stream) {
  return quantize_tokens(x, ldx, M, K, xq, ldq, s_a, 0, stream);
}

size_t qf_tokens_tiled_bytes(int M, int K) {
  if (M < 1 || K < 1 || K % QF_W8A16_K_ALIGN) return 0;
  return (size_t)round_up16(M) * (size_t)K;
}

int qf_quantize_tokens_int8_tiled(const uint16_t* x, int64_t ldx, int M, int K, int8_t* xt, float* s_a,
                                  void* stream) {
  return quantize_tokens(x, ldx, M, K, xt, K, s_a, 1, stream);
}

int qf_w8a8_pick_config(int M, int N, int K, int layout, qf_w8a16_config* cfg) {
  if (cfg == nullptr) return QF_ERR_INVALID_ARG;
  return auto_config_w8a8(M, N, K, layout, cfg) ? QF_OK : QF_ERR_UNSUPPORTED;
}

int qf_w8a8_launch_plan(int M, int N, int K, int layout, const qf_w8a16_config* cfg, int64_t* out, int* count) {
  if (out == nullptr || count == nullptr) return QF_ERR_INVALID_ARG;
  *count = 0;
  if (M < 1 || N < 1 || K < 1) return QF_ERR_INVALID_ARG;
  if (K % QF_W8A16_K_ALIGN) return QF_ERR_UNSUPPORTED;
  qf_w8a16_config c;
  const int rc = qf::resolve_w8a8(M, N, K, layout, cfg, &c);
  if (rc != QF_OK) return rc;
  qf::W8a8Launch plan[2];
  const int nl = qf::w8a8_plan(M, N, K, layout, c, plan);
  if (nl < 1) return nl < 0 ? -nl : QF_ERR_UNSUPPORTED;
  for (int i = 0; i < nl; ++i) {
    out[4 * i + 0] = plan[i].kind;
    out[4 * i + 1] = plan[i].grid;
    out[4 * i + 2] = plan[i].n0;
    out[4 * i + 3] = plan[i].n;
  }
  *count = nl;
  return QF_OK;
}

size_t qf_w8a8_workspace_bytes(int M, int N, int K, int layout, const qf_w8a16_config* cfg) {
  qf_w8a16_config c;
  if (resolve_w8a8(M, N, K, layout, cfg, &c) != QF_OK) return 0;
  return workspace_for(c, M, N);
}

int qf_w8a8_gemm(const int8_t* xq, int64_t ldq, const float* s_a, const int8_t* w, int64_t ldw, int layout,
                 const float* scale, void* y, int64_t ldy, int out_dtype, int M, int N, int K,
                 const qf_w8a16_config* cfg, void* workspace, size_t workspace_bytes, void* stream) {
  return run_w8a8(xq, ldq, 0, s_a, w, ldw, layout, scale, y, ldy, out_dtype, M, N, K, cfg, workspace,
                  workspace_bytes, stream);
}

int qf_w8a8_gemm_xt(const int8_t* xt, const float* s_a, const int8_t* w, int64_t ldw, int layout, const float* scale,
                    void* y, int64_t ldy, int out_dtype, int M, int N, int K, const qf_w8a16_config* cfg,
                    void* workspace, size_t workspace_bytes, void* stream) {
  return run_w8a8(xt, K, 1, s_a, w, ldw, layout, scale, y, ldy, out_dtype, M, N, K, cfg, workspace, workspace_bytes,
                  stream);
}

int qf_stream_capture_info(void* stream, int* capturing, unsigned long long* id) {
  if (capturing == nullptr || id == nullptr) return QF_ERR_INVALID_ARG;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  unsigned long long cid = 0;
  if (hipStreamGetCaptureInfo(reinterpret_cast<hipStream_t>(stream), &st, &cid) != hipSuccess) return QF_ERR_HIP;
  *capturing = st == hipStreamCaptureStatusActive;
  *id = *capturing ? cid : 0;
  return QF_OK;
}

int qf_read_probe(const void* buf, size_t bytes, uint32_t* sink, int blocks, void* stream) {
  if (buf == nullptr || sink == nullptr || blocks < 1 || bytes % 16 || !aligned16(buf)) return QF_ERR_INVALID_ARG;
  hipLaunchKernelGGL(read_probe_kernel, dim3(blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<const u32x4_t*>(buf), (int64_t)(bytes / 16), sink);
  return hipGetLastError() == hipSuccess ? QF_OK : QF_ERR_HIP;
}

int qf_read_probe_stream(const void* buf, size_t bytes, uint32_t* sink, int waves, int depth, void* stream) {
  if (buf == nullptr || sink == nullptr || bytes % 1024 || bytes == 0 || !aligned16(buf)) return QF_ERR_INVALID_ARG;
  using ProbeFn = void (*)(const int8_t*, int64_t, uint32_t*);
  ProbeFn fn = nullptr;
  if (waves == 8 && depth == 4) fn = &read_probe_stream_kernel<8, 4>;
  if (waves == 8 && depth == 8) fn = &read_probe_stream_kernel<8, 8>;
  if (waves == 16 && depth == 4) fn = &read_probe_stream_kernel<16, 4>;
  if (fn == nullptr) return QF_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(fn, dim3(device_cus()), dim3(waves * kWave), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<const int8_t*>(buf), (int64_t)(bytes / 1024), sink);
  return hipGetLastError() == hipSuccess ? QF_OK : QF_ERR_HIP;
}

int qf_empty_kernel(void* stream) {
  hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, reinterpret_cast<hipStream_t>(stream));
  return hipGetLastError() == hipSuccess ? QF_OK : QF_ERR_HIP;
}

int qf_device_cus(void) { return device_cus(); }

size_t qf_argmax_rows_workspace_bytes(void) { return QF_W8A16_COUNTER_BYTES + qf::kArgmaxTableBytes; }

int qf_argmax_rows_bf16_ws(const uint16_t* logits, int64_t ld, int M, int N, int n_valid, int64_t index_offset,
                           int64_t* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (workspace == nullptr || workspace_bytes < qf_argmax_rows_workspace_bytes() || !aligned16(workspace))
    return QF_ERR_WORKSPACE;
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  ArgmaxTable tab;
  tab.arrivals = reinterpret_cast<unsigned*>(ws);
  tab.val = reinterpret_cast<float*>(ws + QF_W8A16_COUNTER_BYTES);
  tab.idx = reinterpret_cast<int*>(ws + QF_W8A16_COUNTER_BYTES + (size_t)kArgmaxMaxRows * kArgmaxMaxBlocks * sizeof(float));
  return argmax_rows(logits, ld, M, N, n_valid, index_offset, out, &tab, stream);
}

int qf_argmax_rows_bf16(const uint16_t* logits, int64_t ld, int M, int N, int n_valid, int64_t index_offset,
                        int64_t* out, void* stream) {
  return argmax_rows(logits, ld, M, N, n_valid, index_offset, out, nullptr, stream);
}

}  // extern "C"

namespace qf {

// Row argmax (qf_argmax_rows_bf16 / _ws): the row-split kernel for long aligned rows, with the
// library's own candidate table (tab == nullptr) or the caller's; one workgroup per row otherwise.
int argmax_rows(const uint16_t* logits, int64_t ld, int M, int N, int n_valid, int64_t index_offset, int64_t* out,
                const ArgmaxTable* tab, void* stream) {
  if (logits == nullptr || out == nullptr || M < 1 || N < 1 || ld < N || n_valid < 0 || n_valid > N)
    return QF_ERR_INVALID_ARG;
  const bool vec = aligned16(logits) && (ld % 8) == 0;
  const int chunks = ceil_div(n_valid, kArgmaxChunk);
  if (vec && M <= kArgmaxMaxRows && chunks >= 2 && chunks <= kArgmaxMaxBlocks) {
    const ArgmaxTable none = {nullptr, nullptr, nullptr};
    if (tab == nullptr)
      hipLaunchKernelGGL(argmax_rows_split_kernel<true>, dim3(chunks, M), dim3(kArgmaxSplitThreads), 0,
                         reinterpret_cast<hipStream_t>(stream), logits, ld, n_valid, index_offset, out, none);
    else
      hipLaunchKernelGGL(argmax_rows_split_kernel<false>, dim3(chunks, M), dim3(kArgmaxSplitThreads), 0,
                         reinterpret_cast<hipStream_t>(stream), logits, ld, n_valid, index_offset, out, *tab);
  } else if (vec)
    hipLaunchKernelGGL(argmax_rows_kernel<true>, dim3(M), dim3(kArgmaxThreads), 0, reinterpret_cast<hipStream_t>(stream),
                       logits, ld, n_valid, index_offset, out);
  else
    hipLaunchKernelGGL(argmax_rows_kernel<false>, dim3(M), dim3(kArgmaxThreads), 0, reinterpret_cast<hipStream_t>(stream),
                       logits, ld, n_valid, index_offset, out);
  return hipGetLastError() == hipSuccess ? QF_OK : QF_ERR_HIP;
}

}  // namespace qf
