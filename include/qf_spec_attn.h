/*
 * qf_spec_attn.h — C ABI of the MI355X (gfx950) split-KV, GQA-packed verification attention.
 *
 * Causal attention for a uniform speculative-decode batch: num_reqs requests, each with q_len query
 * tokens (token b * q_len + i), over a paged bf16 KV cache.  Query i of request b attends the cached
 * positions 0 .. seq_lens[b] - q_len + i (this step's keys and values must already be in the cache).
 * A row that sees no position at all (seq_lens[b] - q_len + i < 0) is written as zeros.
 *
 *   out[t, h, :] = sum_j softmax_j(scale * q[t, h, :] . k[j, h / G, :]) * v[j, h / G, :],  G = H / H_kv
 *
 * Scores, the softmax and the sums are fp32; the softmax weights are rounded to bf16 before they
 * multiply V, as the reference kernel does; the output is bf16 (round to nearest even).
 *
 * Work split (fixed grids, nothing read back to the host, so both launches may be captured in a HIP
 * graph):
 *   1. per (split, request, kv head): the q_len * G query rows that share the kv head are packed into
 *      one tile, and the split's slice of the cached prefix [0, seq_len - q_len) is streamed once for
 *      all of them; the last active split also takes this step's q_len in-flight positions, masked
 *      causally per row; each split writes its normalised partial output and base-2 log-sum-exp;
 *   2. per (token, head, 64 d values): the row's partials are merged by log-sum-exp (a split that
 *      holds no position has written log-sum-exp -inf for its rows, so every split is read).
 *
 * Layouts (strides in elements, the last dimension contiguous):
 *   query      bf16 [>= num_reqs * q_len, H, D]
 *   key_cache  bf16 [num_blocks, page_size, H_kv, D]   (any block / token / head strides)
 *   value_cache bf16 likewise (it may interleave with key_cache, as a [.., H_kv, page, 2D] cache does)
 *   block_table int32 [num_reqs, >= blocks of the longest request], row stride bt_stride
 *   seq_lens   int32 [num_reqs]: cached positions of each request, this step's q_len included
 *   out        bf16 [>= num_reqs * q_len, H, D]
 * Alignment contract: every pointer 16-byte aligned and every stride a multiple of 8 elements, and
 * 64 * (token stride of either cache) below 2^31; otherwise QF_ERR_UNSUPPORTED.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   qf_spec_attention             <- gqa_packed_spec_attention + _prefix_split_kernel +
 *                                    _suffix_combine_kernel   plugin/qwen_fastpath/spec_attn.py:18-173
 *   qf_spec_attn_workspace_bytes  <- the o_part / lse_part torch.empty buffers   spec_attn.py:146-147
 */
#ifndef QF_SPEC_ATTN_H
#define QF_SPEC_ATTN_H

#include <stddef.h>
#include <stdint.h>

#include "qf_w8a16.h" /* qf_status */

#ifdef __cplusplus
extern "C" {
#endif

#define QF_SPEC_ATTN_ABI_VERSION 1
/* Largest packed tile: q_len * (H / H_kv) query rows per kv head. */
#define QF_SPEC_ATTN_MAX_ROWS 64
/* Smallest page (cache block) size in tokens. */
#define QF_SPEC_ATTN_MIN_PAGE 16
/* Prefix splits are whole multiples of this many positions (the prefix kernel's key block). */
#define QF_SPEC_ATTN_KEY_BLOCK 32

/* ABI version of the loaded library (QF_SPEC_ATTN_ABI_VERSION). */
int qf_spec_attn_abi_version(void);

/* Bytes of device workspace for the split partials: num_reqs * H_kv * num_splits * rows * (D + 1)
 * fp32 values, rows = q_len * num_heads / num_kv_heads, rounded up to 256.  0 for invalid sizes.
 * Host-only. */
size_t qf_spec_attn_workspace_bytes(int num_reqs, int q_len, int num_heads, int num_kv_heads,
                                    int head_size, int num_splits);

/* The attention described above on `stream` (a hipStream_t, NULL = the null stream).
 * head_size must be 64, 128 or 256; num_heads % num_kv_heads == 0; q_len * G <= 64; page_size >= 16;
 * 1 <= num_splits <= 65535 and min_chunk >= 1 (a split covers max(ceil(prefix / num_splits), min_chunk)
 * positions, rounded up to QF_SPEC_ATTN_KEY_BLOCK).  The workspace needs no clearing and is free
 * again when the second launch ends; calls that may run at the same time need distinct workspaces.
 * Returns a qf_status. */
int qf_spec_attention(const uint16_t* query, int64_t q_stride_tok, int64_t q_stride_head,
                      const uint16_t* key_cache, int64_t k_stride_block, int64_t k_stride_tok,
                      int64_t k_stride_head,
                      const uint16_t* value_cache, int64_t v_stride_block, int64_t v_stride_tok,
                      int64_t v_stride_head,
                      const int32_t* block_table, int64_t bt_stride,
                      const int32_t* seq_lens,
                      uint16_t* out, int64_t o_stride_tok, int64_t o_stride_head,
                      int num_reqs, int q_len, int num_heads, int num_kv_heads, int head_size,
                      int page_size, float scale, int num_splits, int min_chunk,
                      void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QF_SPEC_ATTN_H */
