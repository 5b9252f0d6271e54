"""CPU oracle for the split-KV, GQA-packed verification attention.

TEST INFRASTRUCTURE ONLY.  Imported by tests/ (as the checker), by ``__graft_entry__.smoke()`` and by
``bench.py``'s cpu_baseline leg; the product package never imports it.

What is restated here (reference paths relative to the reference repository):

* ``gen_spec_inputs``   the reference test's synthetic batch (bench/test_spec_attn.py:10-19): a cache
                        of ``B * nblk + 5`` pages laid out [page][H_kv][PAGE][2D] with K and V
                        interleaved per row (viewed as [page][PAGE][H_kv][D] by transpose + split, as
                        plugin/qwen_fastpath/patches.py:59 does), a shuffled block table, N(0,1) bf16
                        queries and values, request lengths max(ctx + Q - 7 b, 1).  numpy's PCG64
                        replaces torch's generator; the distributions and shapes are the reference's.
* ``spec_attention``    fp64 causal attention of a uniform speculative batch over the paged cache: query
                        qi of request b sees positions 0 .. seq_lens[b] - Q + qi (the semantics of
                        plugin/qwen_fastpath/spec_attn.py:135-140 and of the reference's gold,
                        bench/test_spec_attn.py:23-31); a row that sees no position is 0
                        (spec_attn.py:131).
* ``split_lse_merge``   the log-sum-exp recombination of per-part results (spec_attn.py:119-131,
                        report/main.tex:254-262), in fp64: used by the tests to pin the identity the
                        kernels rely on.
* ``check_spec_attn``   the tolerance rule for bf16 outputs: rows that see nothing are exactly 0; the
                        relative L2 error over the batch is at most 5e-3 (the acceptance bound of the
                        reference's own tuner, bench/test_spec_attn.py:48; the reference kernel
                        measures 2.2e-3 against fp32, data/measurements.json "attention_kernel"), and
                        every row's relative L2 error is at most 2e-2.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def bf16_bits_from_f32(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (finite inputs)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


@dataclass
class SpecInputs:
    q: np.ndarray            # bf16 bits [B*Q, H, D]
    kv: np.ndarray           # bf16 bits [num_pages, H_kv, PAGE, 2D]: K then V in each row
    block_table: np.ndarray  # int32 [B, nblk]
    seq_lens: np.ndarray     # int32 [B]
    B: int
    Q: int
    H: int
    HKV: int
    D: int
    page: int

    def key_cache(self) -> np.ndarray:  # fp32 view [num_pages, PAGE, H_kv, D]
        return bf16_bits_to_f32(self.kv[..., :self.D]).transpose(0, 2, 1, 3)

    def value_cache(self) -> np.ndarray:
        return bf16_bits_to_f32(self.kv[..., self.D:]).transpose(0, 2, 1, 3)

    def query(self) -> np.ndarray:
        return bf16_bits_to_f32(self.q)


def gen_spec_inputs(ctx: int, Q: int, B: int, H: int = 24, HKV: int = 4, D: int = 256, page: int = 800,
                    seed: int = 0, lens=None) -> SpecInputs:
    """The reference test's batch (bench/test_spec_attn.py:10-19) for cached context `ctx`."""
    rng = np.random.default_rng(seed)
    L = ctx + Q
    nblk = (L + page - 1) // page + 1
    npages = B * nblk + 5
    kv = bf16_bits_from_f32(rng.standard_normal((npages, HKV, page, 2 * D), dtype=np.float32))
    block_table = rng.permutation(npages)[:B * nblk].astype(np.int32).reshape(B, nblk)
    q = bf16_bits_from_f32(rng.standard_normal((B * Q, H, D), dtype=np.float32))
    if lens is None:
        lens = [max(L - 7 * i, 1) for i in range(B)]
    seq_lens = np.asarray(lens, dtype=np.int32)
    return SpecInputs(q, kv, block_table, seq_lens, B, Q, H, HKV, D, page)


def spec_attention(q: np.ndarray, key_cache: np.ndarray, value_cache: np.ndarray, seq_lens: np.ndarray,
                   block_table: np.ndarray, num_reqs: int, Q: int, num_kv_heads: int, scale: float) -> np.ndarray:
    """fp64 attention.  q [>= B*Q, H, D]; caches [num_pages, PAGE, H_kv, D] (float arrays or views);
    returns float64 [B*Q, H, D]."""
    H, D = q.shape[1], q.shape[2]
    G = H // num_kv_heads
    page = key_cache.shape[1]
    out = np.zeros((num_reqs * Q, H, D), dtype=np.float64)
    for b in range(num_reqs):
        Lb = int(seq_lens[b])
        pos = np.arange(Lb)
        blk = block_table[b, pos // page]
        off = pos % page
        Kb = np.asarray(key_cache[blk, off], dtype=np.float64)    # [Lb, H_kv, D]
        Vb = np.asarray(value_cache[blk, off], dtype=np.float64)
        qb = np.asarray(q[b * Q:(b + 1) * Q], dtype=np.float64)   # [Q, H, D]
        last = Lb - Q + np.arange(Q)                               # last visible position per query
        visible = pos[None, :] <= last[:, None]                    # [Q, Lb]
        for kv in range(num_kv_heads):
            qg = qb[:, kv * G:(kv + 1) * G, :]                     # [Q, G, D]
            s = np.einsum("qgd,ld->qgl", qg, Kb[:, kv, :]) * scale
            s = np.where(visible[:, None, :], s, -np.inf)
            m = s.max(axis=-1, keepdims=True)
            has = np.isfinite(m)
            p = np.where(has, np.exp(s - np.where(has, m, 0.0)), 0.0)
            l = p.sum(axis=-1, keepdims=True)
            o = np.einsum("qgl,ld->qgd", p, Vb[:, kv, :]) / np.where(l > 0, l, 1.0)
            out[b * Q:(b + 1) * Q, kv * G:(kv + 1) * G, :] = o
    return out


def split_lse_merge(parts):
    """Merge [(o_j, lse2_j)] -- each part's normalised output and base-2 log-sum-exp of its scaled
    scores (log2-sum-exp2 of s * log2(e)) -- into the attention over the union of the parts."""
    m = max(e for _, e in parts)
    w = np.array([2.0 ** (e - m) for _, e in parts])
    acc = sum(wi * o for wi, (o, _) in zip(w, parts))
    return acc / w.sum()


@dataclass
class AttnReport:
    ok: bool
    rel_l2: float
    worst_row_rel_l2: float
    empty_rows: int
    empty_rows_nonzero: int

    def __str__(self):
        return (f"rel_l2={self.rel_l2:.2e} worst_row={self.worst_row_rel_l2:.2e} empty_rows={self.empty_rows} "
                f"nonzero_empty={self.empty_rows_nonzero} ok={self.ok}")


def check_spec_attn(out: np.ndarray, ref: np.ndarray, seq_lens: np.ndarray, Q: int,
                    tol: float = 5e-3, row_tol: float = 2e-2) -> AttnReport:
    """out: float array [B*Q, H, D] (the kernel's bf16 outputs widened); ref: spec_attention()."""
    out = np.asarray(out, dtype=np.float64)
    B = len(seq_lens)
    empty = np.array([int(seq_lens[t // Q]) - Q + (t % Q) < 0 for t in range(B * Q)])
    nz_empty = int(np.count_nonzero(out[empty])) if empty.any() else 0
    live = ~empty
    num = np.linalg.norm(out[live] - ref[live])
    den = np.linalg.norm(ref[live])
    rel = float(num / den) if den > 0 else float(num)
    rows_o = out[live].reshape(-1, out.shape[-1])
    rows_r = ref[live].reshape(-1, ref.shape[-1])
    rn = np.linalg.norm(rows_r, axis=1)
    rr = np.linalg.norm(rows_o - rows_r, axis=1) / np.where(rn > 0, rn, 1.0)
    worst = float(rr.max()) if rr.size else 0.0
    ok = nz_empty == 0 and rel <= tol and worst <= row_tol and np.isfinite(out).all()
    return AttnReport(bool(ok), rel, worst, int(empty.sum()) * out.shape[1], nz_empty)
