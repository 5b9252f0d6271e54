"""Pins the attention oracle (oracle/attn.py) on the CPU:

* against torch's scaled_dot_product_attention in float64 with an explicit causal/visibility mask (a
  library routine), on paged batches with shuffled pages, ragged lengths and every query position;
* closed forms: one visible position gives its value row; scale 0 gives the mean of the visible
  values; equal keys give the mean; one dominant score gives that value row; no visible position
  gives 0;
* planted mistakes (in copies of the oracle made here) that a test must catch: an off-by-one causal
  bound, the kv head taken as h % H_kv instead of h // G, the block table ignored;
* the log-sum-exp recombination of parts (the identity the kernels use) against the direct result;
* the bf16 rounding used to generate inputs, against torch's own cast.
"""
import numpy as np
import pytest
import torch

from oracle import attn as A


def _torch_ref(inp: A.SpecInputs, scale: float, mutate=None) -> np.ndarray:
    """float64 SDPA per request over gathered rows (rows with no visible key come back as NaN or 0)."""
    q = torch.from_numpy(inp.query().astype(np.float64))
    kc = inp.key_cache().astype(np.float64)
    vc = inp.value_cache().astype(np.float64)
    G = inp.H // inp.HKV
    out = np.zeros((inp.B * inp.Q, inp.H, inp.D))
    for b in range(inp.B):
        L = int(inp.seq_lens[b])
        pos = np.arange(L)
        page = inp.page
        # mutation "table": the block table ignored (pages taken as stored in order)
        blk = pos // page + b * inp.block_table.shape[1] if mutate == "table" else inp.block_table[b, pos // page]
        K = torch.from_numpy(kc[blk, pos % page])  # [L, HKV, D]
        V = torch.from_numpy(vc[blk, pos % page])
        heads = np.arange(inp.H)
        kvh = heads % inp.HKV if mutate == "head" else heads // G
        Kh = K[:, kvh, :].permute(1, 0, 2)          # [H, L, D]
        Vh = V[:, kvh, :].permute(1, 0, 2)
        qb = q[b * inp.Q:(b + 1) * inp.Q].permute(1, 0, 2)  # [H, Q, D]
        last = L - inp.Q + np.arange(inp.Q)
        if mutate == "causal":
            last = last - 1
        mask = torch.from_numpy(pos[None, :] <= last[:, None])
        o = torch.nn.functional.scaled_dot_product_attention(qb, Kh, Vh, attn_mask=mask, scale=scale)
        out[b * inp.Q:(b + 1) * inp.Q] = o.permute(1, 0, 2).numpy()
    return out


CASES = [  # ctx, Q, B, H, HKV, D, page, lens
    (0, 3, 1, 6, 2, 16, 4, None),
    (1, 3, 2, 6, 2, 16, 4, None),
    (2, 4, 1, 8, 2, 32, 8, None),
    (37, 3, 2, 6, 3, 16, 4, None),
    (50, 4, 3, 8, 4, 32, 16, None),
    (200, 5, 2, 12, 2, 64, 16, [205, 2]),  # second request shorter than Q
]


@pytest.mark.parametrize("ctx,Q,B,H,HKV,D,page,lens", CASES)
def test_oracle_matches_torch_sdpa_float64(ctx, Q, B, H, HKV, D, page, lens):
    inp = A.gen_spec_inputs(ctx, Q, B, H, HKV, D, page, seed=ctx + 7 * Q + B, lens=lens)
    scale = D ** -0.5
    ours = A.spec_attention(inp.query(), inp.key_cache(), inp.value_cache(), inp.seq_lens, inp.block_table,
                            B, Q, HKV, scale)
    ref = _torch_ref(inp, scale)
    empty_tok = [t for t in range(B * Q) if inp.seq_lens[t // Q] - Q + t % Q < 0]
    live = np.ones(B * Q, dtype=bool)
    live[empty_tok] = False
    assert np.abs(ours[live] - ref[live]).max() <= 1e-12
    # rows that see no position: torch gives NaN or 0 depending on the backend; the oracle writes 0
    assert np.all(ours[empty_tok] == 0)
    assert np.all(np.isnan(ref[empty_tok]) | (ref[empty_tok] == 0))


@pytest.mark.parametrize("mutate", ["causal", "head", "table"])
def test_planted_mistakes_are_caught(mutate):
    inp = A.gen_spec_inputs(40, 3, 2, 6, 2, 16, 4, seed=3)
    scale = 0.25
    ours = A.spec_attention(inp.query(), inp.key_cache(), inp.value_cache(), inp.seq_lens, inp.block_table,
                            inp.B, inp.Q, inp.HKV, scale)
    bad = np.nan_to_num(_torch_ref(inp, scale, mutate=mutate))
    rep = A.check_spec_attn(bad, ours, inp.seq_lens, inp.Q)
    assert not rep.ok, (mutate, rep)


def _closed_form_inputs(L, Q, H=4, HKV=2, D=8, page=4, seed=0):
    inp = A.gen_spec_inputs(L - Q, Q, 1, H, HKV, D, page, seed=seed)
    return inp


def test_closed_forms():
    D = 8
    # one visible position: query 0 of a request with seq_len == Q sees only position 0
    inp = _closed_form_inputs(3, 3, D=D)
    kc, vc = inp.key_cache(), inp.value_cache()
    out = A.spec_attention(inp.query(), kc, vc, inp.seq_lens, inp.block_table, 1, 3, 2, 0.3)
    blk0 = inp.block_table[0, 0]
    for h in range(4):
        assert np.allclose(out[0, h], vc[blk0, 0, h // 2], rtol=0, atol=1e-12)
    # scale 0: the mean of the visible value rows
    inp = _closed_form_inputs(20, 3, D=D, seed=1)
    kc, vc = inp.key_cache(), inp.value_cache()
    out = A.spec_attention(inp.query(), kc, vc, inp.seq_lens, inp.block_table, 1, 3, 2, 0.0)
    pos = np.arange(20)
    V = vc[inp.block_table[0, pos // 4], pos % 4].astype(np.float64)
    for qi in range(3):
        vis = 20 - 3 + qi + 1
        for h in range(4):
            assert np.allclose(out[qi, h], V[:vis, h // 2].mean(axis=0), atol=1e-12)
    # equal keys everywhere: the mean again, whatever the scale
    kc2 = np.broadcast_to(kc[:1, :1], kc.shape)
    out = A.spec_attention(inp.query(), kc2, vc, inp.seq_lens, inp.block_table, 1, 3, 2, 5.0)
    for qi in range(3):
        vis = 20 - 3 + qi + 1
        assert np.allclose(out[qi, 1], V[:vis, 0].mean(axis=0), atol=1e-12)
    # one dominant score: that value row
    kc3 = np.array(kc, dtype=np.float64)
    q = inp.query().astype(np.float64)
    b7 = inp.block_table[0, 7 // 4]
    kc3[b7, 7 % 4, 0] = q[0, 0] * 1e3
    out = A.spec_attention(q, kc3, vc, inp.seq_lens, inp.block_table, 1, 3, 2, 1.0)
    assert np.allclose(out[0, 0], vc[b7, 7 % 4, 0], atol=1e-9)
    # no visible position: zeros
    inp = A.gen_spec_inputs(0, 3, 1, 4, 2, D, 4, seed=2, lens=[1])
    out = A.spec_attention(inp.query(), inp.key_cache(), inp.value_cache(), inp.seq_lens, inp.block_table,
                           1, 3, 2, 0.5)
    assert np.all(out[:2] == 0) and np.any(out[2] != 0)


def test_lse_merge_of_parts_equals_direct():
    rng = np.random.default_rng(5)
    L, D = 300, 16
    s = rng.standard_normal(L) * 3.0          # natural-log-domain scores
    V = rng.standard_normal((L, D))
    p = np.exp(s - s.max())
    direct = p @ V / p.sum()
    for cuts in ([0, 300], [0, 100, 300], [0, 7, 64, 65, 200, 300]):
        parts = []
        for a, b in zip(cuts[:-1], cuts[1:]):
            sj = s[a:b] * np.log2(np.e)           # base 2, as the kernels keep scores
            m = sj.max()
            pj = 2.0 ** (sj - m)
            parts.append((pj @ V[a:b] / pj.sum(), m + np.log2(pj.sum())))
        assert np.allclose(A.split_lse_merge(parts), direct, atol=1e-12)
    # a dropped part is not the direct result
    assert not np.allclose(A.split_lse_merge(parts[1:]), direct, atol=1e-6)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(11)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32),
                        np.float32([0.0, -0.0, 1.0, 1.00390625, 1.005859375, 3.0e38, 1e-40, -2.5e-39])])
    ours = A.bf16_bits_from_f32(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


def test_check_rejects_wrong_outputs():
    inp = A.gen_spec_inputs(60, 3, 2, 6, 2, 16, 8, seed=9, lens=[63, 2])
    ref = A.spec_attention(inp.query(), inp.key_cache(), inp.value_cache(), inp.seq_lens, inp.block_table,
                           2, 3, 2, 0.25)
    good = A.bf16_bits_to_f32(A.bf16_bits_from_f32(ref.astype(np.float32)))
    assert A.check_spec_attn(good, ref, inp.seq_lens, 3).ok
    bad = good.copy()
    bad[1, 2] *= 1.05                                  # one row 5% off
    assert not A.check_spec_attn(bad, ref, inp.seq_lens, 3).ok
    bad = good.copy()
    bad[3] = 1e-3                                      # an empty row (request 1, query 0) not zero
    assert not A.check_spec_attn(bad, ref, inp.seq_lens, 3).ok
