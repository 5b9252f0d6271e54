/*
 * qf_w8a16.h — C ABI of the MI355X (gfx950) W8A16 decode GEMM.
 *
 *   y[m, n] = bf16_rne( scale[n] * sum_k x[m, k] * w[n, k] )      m < M
 *
 * x is bf16 [M, K] (row stride ldx elements, unit column stride), w is int8 [N, K] row-major
 * (the W8A8 checkpoint layout; the [K, N] column-major view vLLM keeps for CUTLASS is the same
 * memory), scale is fp32 per output channel [N], y is bf16 (or fp32) [M, N] with row stride ldy.
 * Accumulation is fp32; the scale is applied after the K reduction; split-K partial sums are
 * reduced in a fixed (split) order, so results are bitwise reproducible run to run.
 *
 * The ABI uses only plain pointers and sizes.  `stream` is a hipStream_t (NULL = the null stream).
 * No entry point allocates, frees, synchronises or retains a pointer after it returns, so every
 * launch entry point may be recorded into a HIP graph.  Errors are returned as qf_status codes;
 * QF_ERR_UNSUPPORTED means "this shape/layout is not handled here, use the fallback path", which
 * is how the reference's `pick_config(...) is None` branch is expressed.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   qf_w8a16_gemm            <- w8a16_mm + _w8a16_kernel   plugin/qwen_fastpath/w8a16.py:15-44,71-83
 *   qf_w8a16_pick_config     <- pick_config / TUNED / SMALL_M   plugin/qwen_fastpath/w8a16.py:12,47-68
 *   qf_w8a16_workspace_bytes <- the fp32 split-K buffer torch.zeros   plugin/qwen_fastpath/w8a16.py:78-79
 *   qf_quantize_rows_int8    <- draft-head per-row quantizer   plugin/qwen_fastpath/patches.py:139-147
 *   qf_argmax_rows_bf16      <- pad mask + argmax of draft logits   plugin/qwen_fastpath/patches.py:182-185
 *   qf_argmax_rows_bf16_ws   <- the same, with its candidate table in a caller workspace    patches.py:182-185
 *   qf_w8a16_gemm_argmax     <- draft logits + pad mask + argmax in one launch   patches.py:160-166,178-185
 *   qf_quantize_tokens_int8  <- ops.scaled_int8_quant (dynamic, symmetric)   plugin/qwen_fastpath/patches.py:99
 *   qf_w8a8_gemm             <- ops.cutlass_scaled_mm on the int8 weights      plugin/qwen_fastpath/patches.py:100
 *   qf_quantize_tokens_int8_tiled / qf_w8a8_gemm_xt / qf_tokens_tiled_bytes: the same two steps with the
 *                              activations in a tiled layout (no reference counterpart; the library's own format)
 *   qf_w8a8_pick_config / qf_w8a8_workspace_bytes: its configuration and workspace (host only)
 *   qf_w8a16_repack / qf_w8a16_unpack: load-time weight layout change (no reference counterpart;
 *                              the reference streams the checkpoint layout as is, w8a16.py:1-7)
 */
#ifndef QF_W8A16_H
#define QF_W8A16_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QF_W8A16_ABI_VERSION 1

/* Largest M of the decode kernels (the reference's SMALL_M, plugin/qwen_fastpath/w8a16.py:12), and of
 * every call on row-major weights.  On TILED weights QF_KERNEL_MFMA_WIDE serves any M. */
#define QF_W8A16_MAX_M 16
/* K must be a multiple of this (the reference's smallest BLOCK_K, w8a16.py:63-68). */
#define QF_W8A16_K_ALIGN 64
/* Bytes at the front of a split-K workspace that hold arrival counters (one per workgroup column). */
#define QF_W8A16_COUNTER_BYTES 65536
/* Size of the static device scratch of qf_w8a16_gemm_noalloc (counters + split partials), per device. */
#define QF_W8A16_SCRATCH_BYTES (4u << 20)

typedef enum qf_status {
  QF_OK = 0,
  QF_ERR_INVALID_ARG = 1,  /* null pointer, negative size, bad enum */
  QF_ERR_UNSUPPORTED = 2,  /* valid request this library does not serve: caller falls back */
  QF_ERR_WORKSPACE = 3,    /* workspace missing or smaller than qf_w8a16_workspace_bytes() */
  QF_ERR_HIP = 4           /* a HIP runtime call failed (launch error) */
} qf_status;

/* Weight layouts. */
typedef enum qf_layout {
  QF_LAYOUT_ROWMAJOR = 0,  /* int8 [N, K], row stride ldw bytes: the checkpoint / CUTLASS layout */
  QF_LAYOUT_TILED = 1      /* pre-permuted 1 KiB tiles (16 rows x 64 k), see qf_w8a16_repack */
} qf_layout;

typedef enum qf_dtype { QF_DTYPE_BF16 = 0, QF_DTYPE_F32 = 1 } qf_dtype;

typedef enum qf_kernel {
  QF_KERNEL_AUTO = 0,  /* pick by shape and M */
  QF_KERNEL_GEMV = 1,  /* wavefront-reduction GEMV, M <= 4, row-major layout only */
  QF_KERNEL_MFMA = 2,  /* v_mfma_f32_16x16x32_bf16 tiles, M <= 16, both layouts */
  QF_KERNEL_MFMA_XRING = 3, /* the same tiles with x staged in (depth + 1)-step chunks through a
                               two-slot LDS ring instead of whole; k_waves must be 1 */
  QF_KERNEL_MFMA_WIDE = 4,  /* TILED layout, any M (picked for M > 16): each weight fragment feeds
                               up to four 16-token tiles; groups of up to 64 token rows run in one
                               launch; k_waves must be 1, split_k > 1 needs the workspace;
                               tiles_per_wave 1 or 2 with 4 or 8 waves at depth 4 or 8, or 4 tiles
                               with 4 waves at depth 2 */
  QF_KERNEL_MFMA_W8A8 = 5,  /* qf_w8a8_gemm only: the same tiling on v_mfma_i32_16x16x64_i8 with int8
                               activations; tiles_per_wave 2 or 4, 4 or 8 waves, depth 2 or 4 */
  QF_KERNEL_MFMA_W8A8_TILE = 6, /* qf_w8a8_gemm only, either layout, picked for large M x N: 256-channel x
                               256-token workgroups, both operands staged in LDS by direct-to-LDS copies
                               through a 4-stage ring; waves 8, tiles_per_wave 8, depth 4; split_k 1 to 8
                               (at most K/64): split_k copies of the grid each sum a K range and the last
                               of a tile's copies to arrive adds the others' int32 partials (workspace:
                               256 KiB a workgroup) and writes the output, one launch; with split_k 1,
                               past whole rounds of 256 workgroups, a last round of at most 64 runs its
                               channels in a second launch: reduce 0 (automatic) on 128 x 128 workgroups
                               of the same kernel where they make one round of 128 to 256, else on the
                               QF_KERNEL_MFMA_W8A8 kernel; reduce 2 on the latter only; reduce 1: one
                               launch; reduce 3 (split_k 1): one launch of 256-channel x 128-token
                               workgroups */
  QF_KERNEL_MFMA_STREAM = 7 /* TILED layout, M <= 16: one workgroup per CU, each over a contiguous run of
                               16-row tiles and the whole K range; all its waves split K (k_waves == waves)
                               with a depth-step prefetch ring that runs across tile boundaries; split_k 1,
                               load_hint 1.  reduce bit 0 clear: x staged in LDS (8 waves at depth 2, 3, 4, 5,
                               6, 8, 12 or 16; 16 waves at depth 2, 4 or 8); set: each wave's x fragments held
                               in registers (8 waves: K = 5120 at depth 4 or 9, K = 8192 at depth 3 or 7, K =
                               4096 at depth 3; 16 waves: K = 5120 at depth 4).  reduce bit 1: workgroup b owns
                               tiles b, b + G, ... instead of a contiguous run.  reduce bit 2: G = ceil(tiles /
                               tiles_per_wave) workgroups of tiles_per_wave tiles each (several may share a CU)
                               instead of one per CU (tiles_per_wave 1) */
} qf_kernel;

/* Launch configuration.  A zero field means "choose automatically". */
typedef struct qf_w8a16_config {
  int32_t kernel;          /* qf_kernel */
  int32_t split_k;         /* K splits across workgroups (deterministic second-pass reduction) */
  int32_t tiles_per_wave;  /* MFMA: 16-row n-tiles per wavefront; GEMV: rows per wavefront */
  int32_t waves;           /* wavefronts per workgroup */
  int32_t depth;           /* weight prefetch depth in k-steps (MFMA) */
  int32_t load_hint;       /* 0: default weight loads, 1: non-temporal (streaming) loads */
  int32_t k_waves;         /* MFMA: wavefronts per workgroup that split K (waves % k_waves == 0) */
  int32_t reduce;          /* MFMA, split_k > 1: 0 = the last workgroup of an n-block sums the
                              splits, 1 = a second kernel does */
} qf_w8a16_config;

/* ABI version of the loaded library (QF_W8A16_ABI_VERSION). */
int qf_abi_version(void);

/* Static text for a qf_status value. */
const char* qf_status_string(int status);

/* Fill *cfg with the configuration used for (M, N, K, layout).  Returns QF_ERR_UNSUPPORTED when the
 * shape is not served (M < 1, M > 16 on row-major weights, N < 1, K % 64 != 0, unknown layout),
 * mirroring pick_config() returning None.  M > 16 on TILED weights gets QF_KERNEL_MFMA_WIDE (the
 * reference sends M > 16 to its W8A8 fallback, plugin/qwen_fastpath/patches.py:99-100, which cannot
 * read the TILED image).  Host-only; touches no device. */
int qf_w8a16_pick_config(int M, int N, int K, int layout, qf_w8a16_config* cfg);

/* Bytes of device workspace qf_w8a16_gemm needs for this call (0 when split_k == 1): arrival
 * counters followed by the split partial sums.  cfg may be NULL (automatic configuration).
 * Host-only. */
size_t qf_w8a16_workspace_bytes(int M, int N, int K, int layout, const qf_w8a16_config* cfg);

/* y = bf16/fp32( scale * (x . w^T) ).  cfg may be NULL.  Alignment contract: x, w, scale 16-byte
 * aligned, ldx % 8 == 0, ldw % 16 == 0 (row-major layout) and y 16-byte aligned; otherwise
 * QF_ERR_UNSUPPORTED.  Any ldy >= N works (vector stores when ldy % 4 == 0).
 * Workspace contract (split_k > 1): its first QF_W8A16_COUNTER_BYTES bytes are arrival counters
 * that must be zero when a call starts; every call leaves them zero again, so a workspace zeroed
 * once can be reused by any number of calls issued in order on one stream (and by graph replays).
 * Calls that may run at the same time need distinct workspaces.  The partial sums that follow need
 * no clearing. */
int qf_w8a16_gemm(const uint16_t* x, int64_t ldx,
                  const int8_t* w, int64_t ldw, int layout,
                  const float* scale,
                  void* y, int64_t ldy, int out_dtype,
                  int M, int N, int K,
                  const qf_w8a16_config* cfg,
                  void* workspace, size_t workspace_bytes,
                  void* stream);

/* qf_w8a16_gemm without a workspace argument, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid allocation).  No counterpart in
 * the reference.  The split-K workspace is a static device array of QF_W8A16_SCRATCH_BYTES per device,
 * held until the process ends; a call that needs more (qf_w8a16_workspace_bytes > QF_W8A16_SCRATCH_BYTES)
 * returns QF_ERR_WORKSPACE before launching anything.  Nothing is allocated or freed.  Every call on a
 * device shares that device's array, so calls that may overlap on one device (different streams) race:
 * issue them in order, or give them distinct workspaces through qf_w8a16_gemm.  Same results, bit for
 * bit, as qf_w8a16_gemm with the same configuration. */
int qf_w8a16_gemm_noalloc(const uint16_t* x, int64_t ldx,
                          const int8_t* w, int64_t ldw, int layout,
                          const float* scale,
                          void* y, int64_t ldy, int out_dtype,
                          int M, int N, int K,
                          const qf_w8a16_config* cfg,
                          void* stream);

/* Fused draft-head argmax: the product of qf_w8a16_gemm, and
 *   ids[m] = index_offset + argmax_{n < n_valid} bf16(y[m, n])      (int64, m < M)
 * with NaN counting as the maximum and ties going to the lowest index: the result of
 * qf_argmax_rows_bf16 on the stored logits, without writing and re-reading them.  y may be NULL (no
 * logits are stored); otherwise it is written as by qf_w8a16_gemm.  Each wavefront column of the GEMM
 * folds its candidate per token into one of 64 slots of the token in the workspace (a 64-bit atomic
 * maximum of a key that orders candidates as above; the slots spread over the counter prefix so that no
 * address or memory channel takes many of the atomics), and a second launch of one wavefront per token
 * folds the slots into the ids and clears them.
 * Served when the configuration is the MFMA kernel without a K split (else QF_ERR_UNSUPPORTED: call
 * qf_w8a16_gemm and qf_argmax_rows_bf16).  Workspace: qf_w8a16_argmax_workspace_bytes() bytes with the
 * split-K workspace contract: its first QF_W8A16_COUNTER_BYTES bytes (the slots) must be zero when a
 * call starts and are zero again when it ends, so a workspace zeroed once serves any number of calls
 * issued in order on one stream (a split-K workspace may serve); calls that may run at the same time
 * need distinct workspaces.  1 <= n_valid <= N.
 * Reference: the W8A16 logits and the pad-masked argmax of get_top_tokens,
 * plugin/qwen_fastpath/patches.py:160-166,178-185, in one launch. */
int qf_w8a16_gemm_argmax(const uint16_t* x, int64_t ldx, const int8_t* w, int64_t ldw, int layout,
                         const float* scale, void* y, int64_t ldy, int out_dtype, int M, int N, int K,
                         int n_valid, int64_t index_offset, int64_t* ids, const qf_w8a16_config* cfg,
                         void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of qf_w8a16_gemm_argmax (0 when the fused argmax does not serve the shape). */
size_t qf_w8a16_argmax_workspace_bytes(int M, int N, int K, int layout, const qf_w8a16_config* cfg);

/* Size in bytes of the TILED image of an [N, K] weight (N rounded up to 16). */
size_t qf_w8a16_tiled_bytes(int N, int K);

/* Row-major int8 [N, K] (row stride ldw) -> TILED image (qf_w8a16_tiled_bytes bytes, pad rows 0).
 * Out of place; K % 64 == 0. */
int qf_w8a16_repack(const int8_t* w_rowmajor, int64_t ldw, int8_t* w_tiled,
                    int N, int K, void* stream);

/* Inverse of qf_w8a16_repack (drops pad rows). */
int qf_w8a16_unpack(const int8_t* w_tiled, int8_t* w_rowmajor, int64_t ldw,
                    int N, int K, void* stream);

/* Exact int8 -> bf16 copy of weight rows [n0, n0 + rows) of an [N, K] weight in either layout (TILED:
 * the image made by qf_w8a16_repack) into the row-major bf16 matrix out (row stride ldo elements,
 * ldo % 8 == 0, 16-byte aligned).  No scale is applied.  It feeds a library bf16 GEMM (fp32
 * accumulation, scale after the K reduction) for M beyond the wide-M kernel's range on weights kept
 * in the TILED layout, which no W8A8 library kernel can read.  No reference counterpart: the
 * reference routes M > 16 to CUTLASS W8A8 on the checkpoint layout
 * (plugin/qwen_fastpath/patches.py:99-100). */
int qf_w8a16_dequant_bf16(const int8_t* w, int64_t ldw, int layout, int N, int K,
                          int n0, int rows, uint16_t* out, int64_t ldo, void* stream);

/* y[m, n] = bf16_rne(acc[m, n] * scale[n]) for m < M, n < N: the epilogue of that library GEMM, whose
 * fp32 output acc [M, N] (row stride lda >= N elements) is scaled after the K reduction and rounded,
 * in one pass; y is bf16 [M, N] with row stride ldy >= N.  16-byte vector accesses when acc, scale
 * and y are 16-byte aligned, lda % 4 == 0 and ldy % 8 == 0, element by element otherwise.  Every
 * non-NaN result equals torch's (acc * scale).to(bfloat16) bit for bit; NaN stays NaN.  No
 * reference counterpart (the M > 16 path above). */
int qf_scale_cast_bf16(const float* acc, int64_t lda, const float* scale, int M, int N,
                       uint16_t* y, int64_t ldy, void* stream);

/* y[m, :] = bf16_rne(x[m, :] * (1 / sqrt(mean_k(x[m, k]^2) + eps))) for m < M: each row of a bf16 [M, N] matrix
 * (row stride ldx) scaled to unit RMS, into y (row stride ldy; y may be x).  The sum of squares is formed in a
 * fixed order (the row as N / 8 pieces of 8 values; lane t of a wavefront takes pieces t, t + 64, ... and keeps
 * one fp32 sum per value position, each over its pieces in order with fused multiply-adds; the eight sums add as a
 * balanced tree, and the 64 lane sums fold within 16-lane rows, then across the four rows), the same order
 * qf_w8a16_gemm_rmsnorm uses, so results are reproducible; against torch's fp32 rms_norm of the same rows they
 * differ by at most one bf16 ulp.  N % 8 == 0,
 * x and y 16-byte aligned, ldx % 8 == 0 and ldy % 8 == 0, else QF_ERR_UNSUPPORTED.  No reference
 * counterpart: the re-normalisation between the layers of the 64-layer decode-step benchmark (each layer's
 * output to unit RMS as the next layer's input). */
int qf_rms_norm_rows_bf16(const uint16_t* x, int64_t ldx, int M, int N, float eps, uint16_t* y, int64_t ldy,
                          void* stream);

/* qf_w8a16_gemm of the rows of x scaled to unit RMS: y = qf_w8a16_gemm(qf_rms_norm_rows_bf16(x, eps)), bit for bit,
 * in one launch.  Each workgroup stages the whole rows of x (K % 8 == 0) and normalises them in LDS in the same
 * order as qf_rms_norm_rows_bf16 before its first multiply, so the normalisation costs no launch of its own.
 * Served where the configuration (automatic, or cfg) stages whole rows without a K split on TILED weights: the
 * MFMA kernel with one tile a wavefront at depth 4 and (waves / k_waves, k_waves) = (4, 2), (2, 4), (1, 4) or
 * (8, 1), or the x-in-LDS stream kernel with 8 waves at depth 4; otherwise QF_ERR_UNSUPPORTED (the caller then
 * makes the two calls).  No reference counterpart: the layer-to-layer glue of the 64-layer decode step (the
 * normalised layer output as the next layer's qkv input). */
int qf_w8a16_gemm_rmsnorm(const uint16_t* x, int64_t ldx, float eps, const int8_t* w, int64_t ldw, int layout,
                          const float* scale, void* y, int64_t ldy, int out_dtype, int M, int N, int K,
                          const qf_w8a16_config* cfg, void* workspace, size_t workspace_bytes, void* stream);

/* ---- W8A8 path for M > 16: the reference's fallback arithmetic (dynamic per-token int8 activations, int8
 * weights, exact integer sums, fp32 scales), plugin/qwen_fastpath/patches.py:99-100, on MI355X's int8
 * MFMA, for weights in either layout (CUTLASS cannot read the TILED image). ---- */

/* Per-token symmetric int8 quantisation of bf16 x [M, K] (row stride ldx elements):
 *   s_a[m] = max_k |x[m,k]| * fl(1/127)          (fp32; 0 for a row of zeros)
 *   xq[m,k] = clamp(round_half_even(x[m,k] / s_a[m]), -128, 127)   (IEEE division; 0 when s_a[m] == 0)
 * xq is int8 [M, K] with row stride ldq bytes.  Finite inputs.  K % 64 == 0, x 16-byte aligned,
 * ldx % 8 == 0, xq 8-byte aligned and ldq % 8 == 0, else QF_ERR_UNSUPPORTED.
 * Reference: vLLM's scaled_int8_quant(x, symmetric=True) at plugin/qwen_fastpath/patches.py:99, which
 * divides amax by 127 where this multiplies by the fp32 reciprocal (at most one ulp apart in s_a). */
int qf_quantize_tokens_int8(const uint16_t* x, int64_t ldx, int M, int K, int8_t* xq, int64_t ldq, float* s_a,
                            void* stream);

/* y[m, n] = out_dtype( (float(sum_k xq[m,k] * w[n,k]) * s_a[m]) * scale[n] ), the integer sums exact in
 * int32 (K < 132000).  w is the TILED image (ldw ignored) or row-major int8 [N, K] with row stride ldw >= K
 * bytes, ldw % 16 == 0 (the row-major layout runs QF_KERNEL_MFMA_W8A8_TILE or the automatic
 * QF_KERNEL_MFMA_W8A8 shape only: 2 tiles, 8 waves, depth 4);
 * xq / s_a as written by qf_quantize_tokens_int8 (xq 16-byte aligned, ldq % 16 == 0); any M >= 1.
 * cfg may be NULL (automatic); its kernel must be QF_KERNEL_MFMA_W8A8, QF_KERNEL_MFMA_W8A8_TILE or AUTO.  Workspace
 * (qf_w8a8_workspace_bytes, 0 without a K split): the int32 split partials after the counter prefix; the
 * counters (used by QF_KERNEL_MFMA_W8A8_TILE with a K split) must be zero before the first call and are
 * left at zero by every call; calls that may run at the same time need distinct workspaces.
 * Reference: ops.cutlass_scaled_mm(x_q, w_q, scale_a, scale_b, out_dtype, bias=None) at
 * plugin/qwen_fastpath/patches.py:100 (the bias is added by the caller). */
int qf_w8a8_gemm(const int8_t* xq, int64_t ldq, const float* s_a, const int8_t* w, int64_t ldw, int layout,
                 const float* scale, void* y, int64_t ldy, int out_dtype, int M, int N, int K,
                 const qf_w8a16_config* cfg, void* workspace, size_t workspace_bytes, void* stream);

/* The same quantisation written as the token-tiled image xt: the TILED weight layout applied to the
 * [M, K] int8 activations.  Block (b, s) holds tokens 16b .. 16b+15 at k 64s .. 64s+63 and lies at byte
 * (b * K/64 + s) * 1024; in it, token 16b + r at k 64s + 16g .. +15 sits at byte 16 * (16g + r).  The
 * image has ceil(M/16) blocks of rows (qf_tokens_tiled_bytes(M, K) bytes); the rows past M are zeros.
 * xt 16-byte aligned; the other requirements as qf_quantize_tokens_int8.  No reference counterpart: an
 * activation layout of this library, read by qf_w8a8_gemm_xt with one contiguous KiB per fragment
 * (row-major xq gives each copy 16 rows of 64 bytes). */
size_t qf_tokens_tiled_bytes(int M, int K);
int qf_quantize_tokens_int8_tiled(const uint16_t* x, int64_t ldx, int M, int K, int8_t* xt, float* s_a,
                                  void* stream);

/* qf_w8a8_gemm on the token-tiled image of qf_quantize_tokens_int8_tiled (same arguments without ldq; the
 * same kernels, configurations, workspace and results, bit for bit).  Reference: the same call,
 * ops.cutlass_scaled_mm at plugin/qwen_fastpath/patches.py:100. */
int qf_w8a8_gemm_xt(const int8_t* xt, const float* s_a, const int8_t* w, int64_t ldw, int layout, const float* scale,
                    void* y, int64_t ldy, int out_dtype, int M, int N, int K, const qf_w8a16_config* cfg,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Automatic configuration and workspace bytes of qf_w8a8_gemm (host only). */
int qf_w8a8_pick_config(int M, int N, int K, int layout, qf_w8a16_config* cfg);
size_t qf_w8a8_workspace_bytes(int M, int N, int K, int layout, const qf_w8a16_config* cfg);

/* The kernel launches qf_w8a8_gemm makes for (M, N, K, layout, cfg), in stream order (host only; no
 * reference counterpart: it exposes the launch plan so that it can be checked without a GPU).  Writes
 * *count (1 or 2) rows of four int64 to out[0 .. 8): kind (0: tile kernel, 256 x 256 workgroups; 1: tile
 * kernel, 256 x 128; 2: tile kernel, 128 x 128; 3: wide kernel; 4: split-K reduction), workgroups, and the
 * first output channel and channel count of the launch.  The launches' channel ranges are disjoint and
 * cover [0, N). */
int qf_w8a8_launch_plan(int M, int N, int K, int layout, const qf_w8a16_config* cfg, int64_t* out, int* count);

/* Per-row symmetric int8 quantisation of a bf16 [V, H] matrix (row stride ldw elements):
 *   s[v] = max(max_h |w[v,h]|, 1e-8) / 127   (fp32, IEEE division)
 *   q[v,h] = clamp(round_half_even(w[v,h] / s[v]), -127, 127)
 * q is int8 [V, H] row-major (row stride H).  Reference: plugin/qwen_fastpath/patches.py:139-147. */
int qf_quantize_rows_int8(const uint16_t* w, int64_t ldw, int8_t* q, float* s,
                          int V, int H, void* stream);

/* Row argmax of bf16 logits [M, N] (row stride ld): columns >= n_valid count as -inf (the padded
 * vocabulary), ties go to the lowest index, NaN counts as the maximum (torch.argmax semantics).
 * out[m] = index + index_offset (int64).  Reference: plugin/qwen_fastpath/patches.py:182-185. */
int qf_argmax_rows_bf16(const uint16_t* logits, int64_t ld, int M, int N, int n_valid,
                        int64_t index_offset, int64_t* out, void* stream);

/* qf_argmax_rows_bf16 with the candidate table of its row-split kernel in a caller workspace
 * (qf_argmax_rows_workspace_bytes() bytes, 16-byte aligned) instead of the library's device-resident
 * table, so that calls on different streams may overlap when each has its own workspace.  The first
 * QF_W8A16_COUNTER_BYTES bytes are arrival counters, zero on entry and returned to zero (the counter
 * prefix of a qf_w8a16_gemm workspace: the same buffer may serve calls of both issued in order).
 * Reference: plugin/qwen_fastpath/patches.py:182-185, as qf_argmax_rows_bf16. */
size_t qf_argmax_rows_workspace_bytes(void);
int qf_argmax_rows_bf16_ws(const uint16_t* logits, int64_t ld, int M, int N, int n_valid,
                           int64_t index_offset, int64_t* out, void* workspace, size_t workspace_bytes,
                           void* stream);

/* Host helper for callers that keep one workspace per graph capture (a workspace first used inside a
 * capture is zeroed by a kernel recorded into that graph): *capturing = 1 while `stream` is capturing
 * a HIP graph, and *id = that capture's id (unique per capture; 0 when not capturing).  No reference
 * counterpart (the reference allocates its split-K buffer per call, plugin/qwen_fastpath/w8a16.py:76-79). */
int qf_stream_capture_info(void* stream, int* capturing, unsigned long long* id);

/* Diagnostic: read every byte of [buf, buf + bytes) once with 16-byte non-temporal loads across
 * `blocks` workgroups of 256 threads, writing one xor per workgroup to sink[blocks].  The practical
 * HBM read ceiling the GEMM is compared with; the analogue of the reference's device-copy probe
 * (bench/kernels/linear_kernels.py:87-89).  bytes % 16 == 0, buf 16-byte aligned. */
int qf_read_probe(const void* buf, size_t bytes, uint32_t* sink, int blocks, void* stream);

/* Diagnostic: read [buf, buf + bytes) once in the stream kernel's pattern: one workgroup per CU (sink holds
 * qf_device_cus() words), workgroup b reading the contiguous b-th share of the buffer's KiB, its `waves`
 * wavefronts interleaved at 1 KiB with `depth` KiB in flight each (waves 8 at depth 4 or 8, waves 16 at depth
 * 4).  The fastest read of a GEMM's bytes measured on this device; the ceiling the GEMMs are compared with.
 * bytes a positive multiple of 1024, buf 16-byte aligned. */
int qf_read_probe_stream(const void* buf, size_t bytes, uint32_t* sink, int waves, int depth, void* stream);

/* Diagnostic: launch one workgroup of a kernel that touches no memory (the dispatch cost of a launch in a
 * graph of back-to-back launches). */
int qf_empty_kernel(void* stream);

/* Compute units of the current device (256 when no device is visible): the stream kernel's grid. */
int qf_device_cus(void);

#ifdef __cplusplus
}
#endif

#endif /* QF_W8A16_H */
