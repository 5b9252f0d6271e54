"""GPU parity of the split-KV verification attention (libqf_spec_attn.so through its C ABI) against
the fp64 oracle (oracle/attn.py), with the tolerance rule of oracle.attn.check_spec_attn.

The case matrix follows the reference's own test (bench/test_spec_attn.py:7-19): H = 24, H_kv = 4,
D = 256, 800-position pages laid out [page][H_kv][PAGE][2D] with K and V interleaved, shuffled
pages, requests of lengths ctx + Q - 7 b, contexts 0 .. 8000 (and 38000) with (Q, B) in
{(3, 1), (4, 1), (3, 2)}.  Further cases cover the other head sizes, every packed-row count class,
vLLM's separate [page][PAGE][H_kv][D] caches with 16-position pages, the split settings, a split
spanning more pages than one block-table window, rows that see no position, determinism and HIP
graph replay.
"""
import numpy as np
import pytest

from oracle import attn as A

pytestmark = pytest.mark.gpu


def _dev(inp: A.SpecInputs, separate: bool = False):
    import torch
    dev = torch.device("cuda:0")
    kv = torch.from_numpy(inp.kv.view(np.int16)).to(dev).view(torch.bfloat16)
    key_cache, value_cache = kv.transpose(1, 2).split(inp.D, dim=-1)
    if separate:
        key_cache, value_cache = key_cache.contiguous(), value_cache.contiguous()
    q = torch.from_numpy(inp.q.view(np.int16)).to(dev).view(torch.bfloat16)
    bt = torch.from_numpy(inp.block_table).to(dev)
    sl = torch.from_numpy(inp.seq_lens).to(dev)
    return q, key_cache, value_cache, bt, sl


def _run(inp, separate=False, **kw):
    import torch
    import qwen_fastpath as qf
    q, kc, vc, bt, sl = _dev(inp, separate)
    out = torch.full_like(q, float("nan"))
    qf.gqa_packed_spec_attention(q, kc, vc, out, sl, bt, inp.B, inp.Q, inp.HKV, inp.D ** -0.5, **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _check(inp, out, tag):
    ref = A.spec_attention(inp.query(), inp.key_cache(), inp.value_cache(), inp.seq_lens, inp.block_table,
                           inp.B, inp.Q, inp.HKV, inp.D ** -0.5)
    rep = A.check_spec_attn(out, ref, inp.seq_lens, inp.Q)
    print(f"spec_attn {tag}: {rep}", flush=True)
    assert rep.ok, (tag, rep)


@pytest.mark.parametrize("ctx", [0, 1, 2, 50, 1000, 8000])
@pytest.mark.parametrize("Q,B", [(3, 1), (4, 1), (3, 2)])
def test_reference_matrix(ctx, Q, B):
    inp = A.gen_spec_inputs(ctx, Q, B, seed=ctx * 10 + Q + B)
    _check(inp, _run(inp), f"ctx={ctx} Q={Q} B={B}")


def test_long_context_38k():
    inp = A.gen_spec_inputs(38000, 3, 1, seed=38)
    _check(inp, _run(inp), "ctx=38000 Q=3 B=1")


@pytest.mark.parametrize("H,HKV,D,Q", [
    (32, 8, 128, 4),    # G = 4, 16 packed rows
    (16, 2, 64, 8),     # G = 8, 64 packed rows
    (24, 4, 256, 8),    # G = 6, 48 packed rows
    (24, 4, 256, 1),    # a single query token
    (8, 8, 128, 2),     # no grouping
])
def test_head_shapes(H, HKV, D, Q):
    inp = A.gen_spec_inputs(3000, Q, 2, H=H, HKV=HKV, D=D, page=800, seed=H + D + Q)
    _check(inp, _run(inp), f"H={H} HKV={HKV} D={D} Q={Q}")


@pytest.mark.parametrize("D", [64, 128, 256])
def test_separate_caches_small_pages(D):
    inp = A.gen_spec_inputs(2500, 3, 2, H=24, HKV=4, D=D, page=16, seed=D)
    _check(inp, _run(inp, separate=True), f"separate D={D} page=16")


@pytest.mark.parametrize("num_splits,min_chunk", [(1, 128), (7, 1), (64, 32), (256, 32), (1000, 1)])
def test_split_settings(num_splits, min_chunk):
    inp = A.gen_spec_inputs(5000, 3, 2, seed=num_splits)
    _check(inp, _run(inp, num_splits=num_splits, min_chunk=min_chunk), f"splits={num_splits} min_chunk={min_chunk}")


def test_split_spanning_several_table_windows():
    # one split over 20000 positions of 16-position pages: 1251 pages, more than one 1024-entry window
    inp = A.gen_spec_inputs(20000, 3, 1, H=16, HKV=2, D=128, page=16, seed=77)
    _check(inp, _run(inp, num_splits=1), "windows page=16 splits=1")


def test_rows_that_see_nothing_are_zero():
    inp = A.gen_spec_inputs(0, 4, 3, seed=5, lens=[1, 2, 4])
    out = _run(inp)
    _check(inp, out, "short requests")
    assert np.all(out[0:3] == 0) and np.all(out[4:6] == 0)


def test_deterministic():
    inp = A.gen_spec_inputs(6000, 3, 2, seed=9)
    a, b = _run(inp), _run(inp)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_graph_replay_matches_eager():
    import torch
    import qwen_fastpath as qf
    inp = A.gen_spec_inputs(4000, 3, 2, seed=12)
    q, kc, vc, bt, sl = _dev(inp)
    scale = inp.D ** -0.5
    eager = torch.empty_like(q)
    qf.gqa_packed_spec_attention(q, kc, vc, eager, sl, bt, inp.B, inp.Q, inp.HKV, scale)
    torch.cuda.synchronize()
    out = torch.zeros_like(q)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        qf.gqa_packed_spec_attention(q, kc, vc, out, sl, bt, inp.B, inp.Q, inp.HKV, scale)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        qf.gqa_packed_spec_attention(q, kc, vc, out, sl, bt, inp.B, inp.Q, inp.HKV, scale)
    for i in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {i}"
        _ = (q.float() * 2).sum().item()  # unrelated eager work between replays
    _check(inp, eager.float().cpu().numpy(), "graph eager")


def test_unsupported_shapes_raise():
    import torch
    import qwen_fastpath as qf
    from qwen_fastpath._lib import QFError
    inp = A.gen_spec_inputs(100, 3, 1, H=8, HKV=2, D=64, page=16, seed=1)
    q, kc, vc, bt, sl = _dev(inp)
    out = torch.empty_like(q)
    with pytest.raises(QFError):  # 3 * 32 packed rows > 64
        qf.gqa_packed_spec_attention(q.repeat(1, 8, 1), kc, vc, out.repeat(1, 8, 1), sl, bt, 1, 3, 2, 0.125)


def test_default_split_count_is_one_workgroup_per_cu():
    import torch
    from qwen_fastpath import spec_attn as SA
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    assert SA.auto_num_splits(dev, 1, 4) == max(1, cus // 4)
    assert SA.auto_num_splits(dev, 2, 4) == max(1, cus // 8)
    assert SA.auto_num_splits(dev, cus, 8) == 1
    inp = A.gen_spec_inputs(7000, 3, 2, seed=31)
    auto = _run(inp)
    explicit = _run(inp, num_splits=max(1, cus // (2 * inp.HKV)))
    assert np.array_equal(auto.view(np.uint32), explicit.view(np.uint32))
    _check(inp, auto, "default splits")
