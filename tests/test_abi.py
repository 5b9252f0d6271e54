"""The C ABI library loads, exports every symbol include/qf_w8a16.h declares, and its host-only entry
points behave as documented.  No call here reaches the GPU: every qf_w8a16_gemm call is rejected by
argument validation before any HIP call."""
import ctypes
import os
import re

import pytest

from qwen_fastpath import _lib as L

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "qf_w8a16.h")


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(qf_\w+)\(", text, flags=re.M)))


def test_header_declares_the_python_export_list():
    assert header_symbols() == sorted(L.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = L.load()
    for name in header_symbols():
        assert hasattr(lib, name), name


def test_abi_version_matches_header():
    m = re.search(r"#define QF_W8A16_ABI_VERSION (\d+)", open(HEADER).read())
    assert L.load().qf_abi_version() == int(m.group(1)) == L.ABI_VERSION


def test_status_strings():
    for st in (L.OK, L.ERR_INVALID_ARG, L.ERR_UNSUPPORTED, L.ERR_WORKSPACE, L.ERR_HIP):
        assert L.status_string(st) and L.status_string(st) != "unknown status"
    assert L.status_string(99) == "unknown status"


@pytest.mark.parametrize("M,N,K,layout", [(0, 64, 64, 0), (17, 64, 64, 0), (5, 64, 100, 0), (5, 64, 0, 0),
                                          (5, 0, 64, 0), (5, 64, 64, 7)])
def test_pick_config_unsupported(M, N, K, layout):
    assert L.pick_config(M, N, K, layout) is None


@pytest.mark.parametrize("M", range(1, 17))
def test_pick_config_supported_and_lds_bounded(M):
    for (N, K) in ((10240, 5120), (5120, 8192), (34816, 5120), (5120, 17408), (151936, 5120), (100, 64)):
        c = L.pick_config(M, N, K)
        assert c is not None
        assert c.kernel in (L.KERNEL_GEMV, L.KERNEL_MFMA, L.KERNEL_MFMA_XRING)
        ksteps = K // 64
        assert 1 <= c.split_k <= ksteps
        steps = -(-ksteps // c.split_k)
        pitch = steps * 128 + 32
        assert max(M * pitch, c.waves * c.tiles_per_wave * 1024 * (c.k_waves > 1)) <= 160 * 1024 - 256
        ws = L.workspace_bytes(M, N, K, 0, None)
        n_pad = (N + 15) // 16 * 16
        assert ws == (0 if c.split_k == 1 else 65536 + c.split_k * M * n_pad * 4)
        assert ksteps // c.split_k >= c.k_waves


def test_pick_config_covers_every_supported_shape():
    """The automatic configuration is valid (instantiated kernel, LDS budget, k-slices) for every
    M <= 16 and a wide range of N and K multiples of 64."""
    Ks = [64 * k for k in (1, 2, 3, 5, 7, 8, 13, 20, 31, 64, 80, 96, 128, 200, 272, 300, 512)]
    Ns = [1, 15, 16, 17, 100, 1000, 5120, 10240, 34816, 151936, 248320, 1 << 20]
    for M in range(1, 17):
        for K in Ks:
            for N in Ns:
                for layout in (0, 1):
                    c = L.pick_config(M, N, K, layout)
                    assert c is not None, (M, N, K, layout)
                    if c.kernel == L.KERNEL_MFMA_STREAM:  # every wavefront splits K; TILED weights only
                        assert layout == 1 and c.k_waves == c.waves in (8, 16) and c.split_k == 1, (M, N, K, c.to_tuple())
                        assert K // 64 >= c.waves and M >= 2, (M, N, K)
                        continue
                    assert c.k_waves in (1, 2, 4) and c.waves % c.k_waves == 0


def test_stream_kernel_rule_host_only():
    """The stream kernel (one workgroup per CU) for TILED weights at M >= 2 with 4 or more 16-row tiles per CU
    (256 CUs without a visible device) where its x slice and partial tiles fit in LDS; never row-major, M = 1,
    narrow N, or the fused argmax (qf_w8a16_argmax_workspace_bytes resolves without it)."""
    lib = L.load()
    for M in range(2, 9):
        c = L.pick_config(M, 34816, 5120, 1)
        assert c.to_tuple() == (L.KERNEL_MFMA_STREAM, 1, 1, 8, 4, 1, 8, 0), (M, c.to_tuple())
        assert L.workspace_bytes(M, 34816, 5120, 1, None) == 0
        assert L.pick_config(M, 34816, 5120, 0).kernel != L.KERNEL_MFMA_STREAM
    for M in range(9, 17):  # the x slice no longer fits beside the partial tiles: x fragments in registers
        want = (L.KERNEL_MFMA_STREAM, 1, 1, 16 if M >= 13 else 8, 4, 1, 16 if M >= 13 else 8, 1)
        assert L.pick_config(M, 34816, 5120, 1).to_tuple() == want, M
    assert L.pick_config(12, 16384, 8192, 1).to_tuple() == (L.KERNEL_MFMA_STREAM, 1, 1, 8, 3, 1, 8, 1)
    assert L.pick_config(12, 16384, 8256, 1).kernel != L.KERNEL_MFMA_STREAM  # no register-x build for this K
    assert L.pick_config(1, 34816, 5120, 1).kernel != L.KERNEL_MFMA_STREAM
    assert L.pick_config(5, 10240, 5120, 1).kernel != L.KERNEL_MFMA_STREAM          # 2.5 tiles per CU
    assert L.pick_config(5, 16384, 5120, 1).kernel == L.KERNEL_MFMA_STREAM          # 4 tiles per CU
    assert L.pick_config(5, 151936, 5120, 1).kernel != L.KERNEL_MFMA_STREAM         # partial tiles exceed LDS
    assert L.pick_config(5, 5120, 17408, 1).kernel != L.KERNEL_MFMA_STREAM
    # the fused argmax keeps an MFMA kernel: a non-zero candidate table for a shape the stream kernel takes
    assert lib.qf_w8a16_argmax_workspace_bytes(4, 34816, 5120, 1, None) > 0
    # explicit stream configurations: TILED only, k_waves == waves, one split, instantiated depths
    ok = L.Config.from_seq((L.KERNEL_MFMA_STREAM, 1, 1, 8, 6, 1, 8, 0))
    assert L.workspace_bytes(5, 34816, 5120, 1, ok) == 0
    for bad in ((L.KERNEL_MFMA_STREAM, 2, 1, 8, 4, 1, 8, 0), (L.KERNEL_MFMA_STREAM, 1, 1, 8, 4, 1, 4, 0),
                (L.KERNEL_MFMA_STREAM, 1, 1, 8, 7, 1, 8, 0), (L.KERNEL_MFMA_STREAM, 1, 1, 8, 4, 0, 8, 0),
                (L.KERNEL_MFMA_STREAM, 1, 1, 4, 4, 1, 4, 0)):
        fake = 1 << 20
        assert _gemm(x=fake, w=fake, s=fake, y=fake, layout=1, K=5120, ldx=5120, ldw=5120, N=34816, ldy=34816,
                     cfg=L.Config.from_seq(bad)) == L.ERR_UNSUPPORTED, bad


def test_workspace_for_explicit_config():
    c = L.Config.from_seq((2, 4, 2, 4, 4, 0, 1))      # 63 tiles / (4 x 2) -> 8 workgroups
    assert L.workspace_bytes(5, 1000, 1024, 0, c) == 65536 + 4 * 5 * 1008 * 4
    c1 = L.Config.from_seq((2, 1, 2, 4, 4, 0, 1))
    assert L.workspace_bytes(5, 1000, 1024, 0, c1) == 0
    c2 = L.Config.from_seq((2, 2, 1, 16, 8, 1, 4))    # 4 tile groups x 4 k-slices
    assert L.workspace_bytes(5, 1000, 1024, 0, c2) == 65536 + 2 * 5 * 1008 * 4
    bad = L.Config.from_seq((2, 8, 1, 16, 8, 1, 4))   # 16 steps / 8 splits < 4 k-slices
    assert L.workspace_bytes(5, 1000, 1024, 0, bad) == 0


def _gemm(x=16, ldx=64, w=16, ldw=64, layout=0, s=16, y=16, ldy=64, dt=0, M=5, N=64, K=64, cfg=None,
          ws=None, wsb=0):
    lib = L.load()
    return lib.qf_w8a16_gemm(x, ldx, w, ldw, layout, s, y, ldy, dt, M, N, K,
                             ctypes.byref(cfg) if cfg is not None else None, ws, wsb, None)


def test_gemm_argument_validation_host_only():
    fake = 1 << 20  # never dereferenced: every call below is rejected before launch
    assert _gemm(x=None) == L.ERR_INVALID_ARG
    assert _gemm(x=fake, w=fake, s=fake, y=fake, M=0) == L.ERR_INVALID_ARG
    assert _gemm(x=fake, w=fake, s=fake, y=fake, layout=5) == L.ERR_INVALID_ARG
    assert _gemm(x=fake, w=fake, s=fake, y=fake, dt=9) == L.ERR_INVALID_ARG
    assert _gemm(x=fake, w=fake, s=fake, y=fake, ldx=32) == L.ERR_INVALID_ARG       # ldx < K
    assert _gemm(x=fake, w=fake, s=fake, y=fake, M=17) == L.ERR_UNSUPPORTED         # > SMALL_M
    assert _gemm(x=fake, w=fake, s=fake, y=fake, K=96, ldx=96, ldw=96) == L.ERR_UNSUPPORTED  # K % 64
    assert _gemm(x=fake + 2, w=fake, s=fake, y=fake) == L.ERR_UNSUPPORTED           # misaligned x
    assert _gemm(x=fake, w=fake, s=fake, y=fake, ldx=68) == L.ERR_UNSUPPORTED       # ldx % 8
    gemv_big_m = L.Config.from_seq((L.KERNEL_GEMV, 1, 4, 4, 4, 0, 1))
    assert _gemm(x=fake, w=fake, s=fake, y=fake, cfg=gemv_big_m) == L.ERR_UNSUPPORTED  # gemv needs M <= 4
    bad_tiles = L.Config.from_seq((L.KERNEL_MFMA, 1, 3, 4, 4, 0, 1))
    assert _gemm(x=fake, w=fake, s=fake, y=fake, cfg=bad_tiles) == L.ERR_UNSUPPORTED
    split = L.Config.from_seq((L.KERNEL_MFMA, 4, 2, 4, 4, 0, 1))
    assert _gemm(x=fake, w=fake, s=fake, y=fake, K=1024, ldx=1024, ldw=1024, cfg=split) == L.ERR_WORKSPACE
    too_many = L.Config.from_seq((L.KERNEL_MFMA, 99, 2, 4, 4, 0, 1))
    bad_shape = L.Config.from_seq((L.KERNEL_MFMA, 1, 1, 6, 4, 0, 4))   # 6 waves not divisible by 4
    assert _gemm(x=fake, w=fake, s=fake, y=fake, cfg=bad_shape) == L.ERR_UNSUPPORTED
    assert _gemm(x=fake, w=fake, s=fake, y=fake, cfg=too_many) == L.ERR_INVALID_ARG


def test_tiled_bytes():
    lib = L.load()
    assert lib.qf_w8a16_tiled_bytes(34816, 5120) == 34816 * 5120
    assert lib.qf_w8a16_tiled_bytes(100, 64) == 112 * 64
    assert lib.qf_w8a16_tiled_bytes(0, 64) == 0


def test_other_entry_points_validate_host_only():
    lib = L.load()
    assert lib.qf_w8a16_repack(None, 64, None, 16, 64, None) == L.ERR_INVALID_ARG
    assert lib.qf_w8a16_repack(1 << 20, 64, 1 << 21, 16, 96, None) == L.ERR_INVALID_ARG  # ldw < K
    assert lib.qf_w8a16_unpack(1 << 20, 1 << 21, 96, 16, 96, None) == L.ERR_UNSUPPORTED  # K % 64
    assert lib.qf_quantize_rows_int8(None, 8, None, None, 1, 8, None) == L.ERR_INVALID_ARG
    assert lib.qf_argmax_rows_bf16(1 << 20, 8, 1, 8, 9, 0, 1 << 21, None) == L.ERR_INVALID_ARG  # n_valid > N


# ---- libqf_spec_attn.so (include/qf_spec_attn.h) ----

ATTN_HEADER = os.path.join(os.path.dirname(HEADER), "qf_spec_attn.h")


def test_attention_header_declares_the_python_export_list():
    from qwen_fastpath import _attn_lib as AL
    text = open(ATTN_HEADER).read()
    syms = sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(qf_\w+)\(", text, flags=re.M)))
    assert syms == sorted(AL.EXPORTS)
    lib = AL.load()
    for name in syms:
        assert hasattr(lib, name), name
    m = re.search(r"#define QF_SPEC_ATTN_ABI_VERSION (\d+)", text)
    assert lib.qf_spec_attn_abi_version() == int(m.group(1)) == AL.ABI_VERSION
    for macro, value in (("MAX_ROWS", AL.MAX_ROWS), ("MIN_PAGE", AL.MIN_PAGE), ("KEY_BLOCK", AL.KEY_BLOCK)):
        assert int(re.search(rf"#define QF_SPEC_ATTN_{macro} (\d+)", text).group(1)) == value


def test_attention_workspace_bytes():
    from qwen_fastpath import _attn_lib as AL
    B, Q, H, HKV, D, S = 2, 3, 24, 4, 256, 64
    R = Q * H // HKV
    n = B * HKV * S * R * (D + 1) * 4
    assert AL.workspace_bytes(B, Q, H, HKV, D, S) == (n + 255) // 256 * 256
    assert AL.workspace_bytes(0, Q, H, HKV, D, S) == 0
    assert AL.workspace_bytes(B, Q, 25, HKV, D, S) == 0   # H not a multiple of H_kv


def _attn_call(lib, *, D=256, H=24, HKV=4, Q=3, page=800, splits=64, min_chunk=128, ws_bytes=None,
               stride=None, ptr_offset=0):
    """qf_spec_attention on 16-byte aligned host dummies: every case here is rejected before any HIP call."""
    buf = (ctypes.c_uint8 * 4096)()
    base = (ctypes.addressof(buf) + 15) // 16 * 16
    p = base + ptr_offset
    st = 8 if stride is None else stride
    ws = lib.qf_spec_attn_workspace_bytes(1, Q, H, HKV, D, splits) if ws_bytes is None else ws_bytes
    return lib.qf_spec_attention(p, st, st, p, st, st, st, p, st, st, st, base, 1, base, p, st, st,
                                 1, Q, H, HKV, D, page, 0.0625, splits, min_chunk, base, ws, None)


def test_attention_rejects_before_launch():
    from qwen_fastpath import _attn_lib as AL
    lib = AL.load()
    assert _attn_call(lib, D=96) == L.ERR_UNSUPPORTED
    assert _attn_call(lib, Q=11) == L.ERR_UNSUPPORTED          # 66 packed rows
    assert _attn_call(lib, HKV=5) == L.ERR_UNSUPPORTED         # 24 % 5
    assert _attn_call(lib, page=8) == L.ERR_UNSUPPORTED
    assert _attn_call(lib, stride=12) == L.ERR_UNSUPPORTED
    assert _attn_call(lib, ptr_offset=8) == L.ERR_UNSUPPORTED
    assert _attn_call(lib, splits=0) == L.ERR_INVALID_ARG
    assert _attn_call(lib, min_chunk=0) == L.ERR_INVALID_ARG
    assert _attn_call(lib, ws_bytes=1024) == L.ERR_WORKSPACE


def _wide_groups(M):
    """Token grouping of the wide-M kernel: the fewest 64-row groups, rows spread evenly in whole
    16-row tiles, then the count that leaves no group empty."""
    g0 = -(-M // 64)
    rows = -(-(-(-M // g0)) // 16) * 16
    return -(-M // rows), rows


def test_wide_groups_cover_every_row():
    for M in range(1, 5000):
        groups, rows = _wide_groups(M)
        assert rows % 16 == 0 and 16 <= rows <= 64
        assert (groups - 1) * rows < M <= groups * rows, M  # every group holds at least one row


def test_pick_config_wide_m_on_tiled_weights():
    """M > 16 is served on TILED weights only, by the wide-M kernel (kind 4, one k-slice, K split at most 8 ways),
    for every N and K; row-major weights stay unsupported above 16 rows."""
    Ks = [64 * k for k in (1, 2, 3, 7, 80, 128, 272, 512)]
    Ns = [1, 15, 16, 17, 1000, 5120, 34816, 151936]
    for M in (17, 31, 32, 48, 63, 64, 65, 100, 129, 192, 256, 1000, 4096):
        for K in Ks:
            for N in Ns:
                assert L.pick_config(M, N, K, 0) is None
                c = L.pick_config(M, N, K, 1)
                assert c is not None, (M, N, K)
                assert c.kernel == L.KERNEL_MFMA_WIDE and c.k_waves == 1 and 1 <= c.split_k <= 8
                assert c.split_k == 1 or K // 64 // c.split_k >= 16
                n_pad = -(-N // 16) * 16
                assert L.workspace_bytes(M, N, K, 1, c) == (0 if c.split_k == 1 else
                                                            65536 + c.split_k * M * n_pad * 4)
    # explicit wide configurations outside the instantiated ones (tiles {1, 2} x waves {4, 8} x depth
    # {4, 8}; 4 tiles x 4 waves at depth 2) or with k-slices are refused before any launch; a K split
    # needs the workspace
    fake = 1 << 20
    for bad in ((L.KERNEL_MFMA_WIDE, 1, 4, 8, 4, 1, 1, 0), (L.KERNEL_MFMA_WIDE, 1, 2, 16, 4, 1, 1, 0),
                (L.KERNEL_MFMA_WIDE, 1, 4, 4, 4, 1, 1, 0), (L.KERNEL_MFMA_WIDE, 1, 2, 4, 2, 1, 1, 0),
                (L.KERNEL_MFMA_WIDE, 1, 2, 8, 4, 1, 2, 0),
                (L.KERNEL_MFMA_WIDE, 1, 2, 8, 6, 1, 1, 0)):
        c = L.Config.from_seq(bad)
        assert _gemm(x=fake, w=fake, s=fake, y=fake, layout=1, M=40, K=1024, ldx=1024, ldw=1024,
                     cfg=c) == L.ERR_UNSUPPORTED, bad
    c = L.Config.from_seq((L.KERNEL_MFMA_WIDE, 4, 2, 8, 4, 1, 1, 1))
    assert L.workspace_bytes(40, 1000, 1024, 1, c) == 65536 + 4 * 40 * 1008 * 4
    assert _gemm(x=fake, w=fake, s=fake, y=fake, layout=1, M=40, K=1024, ldx=1024, ldw=1024,
                 cfg=c) == L.ERR_WORKSPACE
    c = L.Config.from_seq((L.KERNEL_MFMA_WIDE, 1, 2, 8, 4, 1, 1, 0))
    assert _gemm(x=fake, w=fake, s=fake, y=fake, layout=0, M=40, cfg=c) == L.ERR_UNSUPPORTED  # row-major
    assert _gemm(x=fake, w=fake, s=fake, y=fake, layout=0, M=40) == L.ERR_UNSUPPORTED


def test_prefill_arithmetic_switch(monkeypatch):
    """QWEN_FAST_LINEAR_PREFILL picks the arithmetic of M > 16 calls on TILED layers: the reference's W8A8
    by default, W8A16 on request; anything else is an error rather than a silent choice."""
    from qwen_fastpath import patches as P
    monkeypatch.delenv("QWEN_FAST_LINEAR_PREFILL", raising=False)
    assert P.prefill_arithmetic() == "w8a8"
    for v, want in (("w8a16", "w8a16"), (" W8A8 ", "w8a8"), ("W8A16", "w8a16")):
        monkeypatch.setenv("QWEN_FAST_LINEAR_PREFILL", v)
        assert P.prefill_arithmetic() == want
    monkeypatch.setenv("QWEN_FAST_LINEAR_PREFILL", "fp8")
    with pytest.raises(ValueError):
        P.prefill_arithmetic()


def test_w8a8_launch_plan_host_only():
    """The launches qf_w8a8_gemm makes: their channel ranges are disjoint and cover [0, N) in order, every
    grid is non-empty, and a second launch is taken only for a true remainder of 1 to 64 workgroups past whole
    rounds of 256.  Grids that are whole rounds (rest 0) run in one launch, including N not a multiple of
    256 (N = 8000 at M = 2048: 32 x 8 = 256 workgroups), where a split would give the first launch more
    channels than N."""
    def check_plan(M, N, K, layout=1, cfg=None):
        plan = L.w8a8_launch_plan(M, N, K, layout, cfg)
        assert 1 <= len(plan) <= 2, (M, N, K, plan)
        n = 0
        for kind, grid, n0, cnt in plan:
            if kind == "split_reduce":
                assert (n0, cnt) == (0, N) and grid > 0, (M, N, K, plan)
                continue
            assert grid > 0 and cnt > 0 and n0 == n, (M, N, K, plan)
            n += cnt
        assert n == N, (M, N, K, plan)
        return plan
    tile = L.Config.from_seq((L.KERNEL_MFMA_W8A8_TILE, 1, 8, 8, 4, 1, 1, 0))
    tile2 = L.Config.from_seq((L.KERNEL_MFMA_W8A8_TILE, 1, 8, 8, 4, 1, 1, 2))
    # whole rounds, rest 0: one launch over all N (the automatic rule and the explicit tile configs)
    for M, N, K in ((8192, 10240, 5120), (8192, 34816, 5120), (16384, 5120, 8192), (16384, 5120, 17408),
                    (2048, 8000, 128), (2048, 8192, 128), (4096, 8000, 5120)):
        for layout in (1, 0):
            for cfg in (None, tile, tile2):
                plan = check_plan(M, N, K, layout, cfg)
                assert len(plan) == 1 and plan[0][0] == "tile", (M, N, K, layout, plan)
                assert plan[0][1] == -(-N // 256) * -(-M // 256), (M, N, K, plan)
    # a true remainder: whole rounds on the 256 x 256 kernel, the rest on 128 x 128 workgroups or the wide kernel
    plan = check_plan(2048, 34816, 5120)  # 1088 = 4 x 256 + 64
    assert plan == [("tile", 1024, 0, 32768), ("tile_128x128", 256, 32768, 2048)], plan
    plan = check_plan(4096, 4352, 256, 1, tile)  # 272 = 256 + 16: the last block on the wide kernel
    assert [p[0] for p in plan] == ["tile", "wide"] and plan[0][3] == 4096, plan
    plan = check_plan(4096, 4700, 128, 1, tile2)
    assert [p[0] for p in plan] == ["tile", "wide"], plan
    # the other kinds
    assert check_plan(384, 34816, 5120)[0][0] == "tile_256x128"
    assert [p[0] for p in check_plan(17, 5120, 17408)] == ["wide", "split_reduce"]
    assert [p[0] for p in check_plan(1024, 5120, 17408)] == ["tile"]  # K split, fused reduction
    # a sweep of shapes around whole rounds
    for N in (4096, 4100, 8000, 8192, 8200, 10240, 12288, 16384, 34816):
        for M in (256, 512, 1000, 1024, 2048, 4096, 8192):
            for layout in (1, 0):
                check_plan(M, N, 128, layout)
                check_plan(M, N, 128, layout, tile)
                check_plan(M, N, 128, layout, tile2)
    out = (ctypes.c_int64 * 8)()
    cnt = ctypes.c_int(7)
    assert L.load().qf_w8a8_launch_plan(40, 0, 1024, 1, None, out, ctypes.byref(cnt)) == L.ERR_INVALID_ARG
    assert cnt.value == 0
    assert L.load().qf_w8a8_launch_plan(40, 100, 1000, 1, None, out, ctypes.byref(cnt)) == L.ERR_UNSUPPORTED


def test_w8a8_configs_host_only():
    """qf_w8a8_gemm: either layout (row-major: the automatic shape only), its own kernel kind, any M;
    refused before any launch otherwise."""
    lib = L.load()
    for M in (1, 17, 64, 300, 2048):
        for (N, K) in ((34816, 5120), (5120, 17408), (1000, 1024), (16, 64)):
            tile = M == 2048 and N >= 5120  # 1088 and 160 workgroups of 256 x 256
            tile128 = M == 300 and N == 34816  # 136 x 3 workgroups of 256 x 128
            for layout in (1, 0):  # TILED, row-major (the automatic 2-tile shape or the tile kernel)
                c = L.w8a8_pick_config(M, N, K, layout)
                assert c is not None and c.k_waves == 1, (M, N, K, layout)
                if tile:
                    assert c.to_tuple()[:5] == (L.KERNEL_MFMA_W8A8_TILE, 1, 8, 8, 4), (M, N, K, layout)
                elif tile128:
                    assert c.to_tuple() == (L.KERNEL_MFMA_W8A8_TILE, 1, 8, 8, 4, 1, 1, 3), (M, N, K, layout)
                else:
                    assert c.kernel == L.KERNEL_MFMA_W8A8, (M, N, K, layout)
                    if layout == 0:
                        assert c.to_tuple()[2:5] == (2, 8, 4), (M, N, K)
    # The tile kernel's rule: 136 or more workgroups, not 1-16 past a whole round unless the second launch
    # takes them, M >= 256 with under a quarter of the computed rows past M, or one token block above 128 rows.
    assert L.w8a8_pick_config(256, 34816, 5120).kernel == L.KERNEL_MFMA_W8A8_TILE      # 136 workgroups
    assert L.w8a8_pick_config(128, 34816, 5120).kernel == L.KERNEL_MFMA_W8A8           # one 128-row group
    assert L.w8a8_pick_config(129, 34816, 5120).to_tuple()[:2] == (L.KERNEL_MFMA_W8A8_TILE, 1)  # one block
    assert L.w8a8_pick_config(255, 34816, 5120).to_tuple()[:2] == (L.KERNEL_MFMA_W8A8_TILE, 1)
    assert L.w8a8_pick_config(192, 10240, 5120).kernel == L.KERNEL_MFMA_W8A8           # 40 workgroups
    # 289..384 rows on a grid of 136 or more: 256-channel x 128-token workgroups (reduce 3)
    assert L.w8a8_pick_config(384, 34816, 5120).to_tuple() == (L.KERNEL_MFMA_W8A8_TILE, 1, 8, 8, 4, 1, 1, 3)
    assert L.w8a8_pick_config(289, 34816, 5120).to_tuple()[::7] == (L.KERNEL_MFMA_W8A8_TILE, 3)
    assert L.w8a8_pick_config(288, 34816, 5120).kernel == L.KERNEL_MFMA_W8A8           # 2 x 128 rows + 32
    assert L.w8a8_pick_config(385, 34816, 5120).to_tuple()[::7] == (L.KERNEL_MFMA_W8A8_TILE, 0)
    assert L.w8a8_pick_config(320, 10240, 5120).kernel == L.KERNEL_MFMA_W8A8           # 80 workgroups
    assert L.w8a8_pick_config(512, 34816, 5120).kernel == L.KERNEL_MFMA_W8A8_TILE      # 272 = 256 + 16, split
    assert L.w8a8_pick_config(3328, 10240, 5120).kernel == L.KERNEL_MFMA_W8A8          # 520 = 512 + 8, 13 blocks
    assert L.w8a8_pick_config(768, 34816, 5120).kernel == L.KERNEL_MFMA_W8A8_TILE      # 408
    assert L.w8a8_pick_config(1024, 34816, 5120).kernel == L.KERNEL_MFMA_W8A8_TILE     # 544 = 512 + 32
    assert L.w8a8_pick_config(513, 34816, 5120).kernel == L.KERNEL_MFMA_W8A8           # 513 of 768 rows
    assert L.w8a8_pick_config(600, 34816, 5120).kernel == L.KERNEL_MFMA_W8A8_TILE      # 600 of 768 rows
    assert L.w8a8_pick_config(1024, 10240, 5120).kernel == L.KERNEL_MFMA_W8A8_TILE     # 160
    # 40 to 128 workgroups of 256 x 256 with two or more token blocks: the tile kernel with a K split of
    # min(4, K / 2560, 256 / workgroups), at least 2; M = 256 (one token block), short K and fewer
    # workgroups stay below.
    assert L.w8a8_pick_config(1536, 5120, 8192).to_tuple()[:5] == (L.KERNEL_MFMA_W8A8_TILE, 2, 8, 8, 4)  # 120
    assert L.w8a8_pick_config(1024, 5120, 17408).to_tuple()[:5] == (L.KERNEL_MFMA_W8A8_TILE, 3, 8, 8, 4)  # 80
    assert L.w8a8_pick_config(512, 5120, 17408).to_tuple()[:5] == (L.KERNEL_MFMA_W8A8_TILE, 4, 8, 8, 4)  # 40
    assert L.w8a8_pick_config(512, 5120, 8192).to_tuple()[:5] == (L.KERNEL_MFMA_W8A8_TILE, 3, 8, 8, 4)  # 40
    assert L.w8a8_pick_config(768, 10240, 5120, 0).to_tuple()[:5] == (L.KERNEL_MFMA_W8A8_TILE, 2, 8, 8, 4)
    assert L.w8a8_pick_config(256, 5120, 17408).kernel == L.KERNEL_MFMA_W8A8          # one token block
    assert L.w8a8_pick_config(544, 5120, 17408).to_tuple()[:2] == (L.KERNEL_MFMA_W8A8_TILE, 4)  # long K, 3 blocks
    assert L.w8a8_pick_config(544, 5120, 8192).kernel == L.KERNEL_MFMA_W8A8           # 3 blocks, K < 10240
    assert L.w8a8_pick_config(384, 5120, 17408).kernel == L.KERNEL_MFMA_W8A8          # 2 blocks, 384 of 512
    assert L.w8a8_pick_config(1600, 1280, 5120).kernel == L.KERNEL_MFMA_W8A8          # 35 workgroups
    assert L.w8a8_pick_config(1024, 5120, 2048).kernel == L.KERNEL_MFMA_W8A8          # K / 2560 = 0
    assert L.w8a8_pick_config(2048, 3840, 17408).to_tuple()[:2] == (L.KERNEL_MFMA_W8A8_TILE, 2)  # 15 x 8
    for M, N, K in ((1536, 5120, 8192), (1024, 5120, 17408), (512, 5120, 17408)):
        c = L.w8a8_pick_config(M, N, K)
        tiles = -(-N // 256) * -(-M // 256)
        ws = lib.qf_w8a8_workspace_bytes(M, N, K, 1, ctypes.byref(c))
        assert ws == 65536 + tiles * c.split_k * 256 * 1024, (M, N, K)
    # The automatic rule's two exceptions: 4-wavefront workgroups, unsplit, where 8-wavefront ones
    # would be under 128 (TILED only), and a split in two for a long K whose last round of 128-row
    # workgroups would leave the CUs at most a quarter busy.
    assert L.w8a8_pick_config(128, 10240, 5120).to_tuple()[1:5] == (1, 2, 4, 4)
    assert L.w8a8_pick_config(128, 10240, 5120, 0).to_tuple()[1:5] == (2, 2, 8, 4)
    assert L.w8a8_pick_config(256, 5120, 8192).to_tuple()[1:5] == (1, 2, 4, 4)
    assert L.w8a8_pick_config(2304, 3840, 17408).to_tuple()[1:5] == (2, 2, 8, 4)
    assert L.w8a8_pick_config(2048, 3072, 4096).to_tuple()[1:5] == (1, 2, 8, 4)
    fake = 1 << 20
    def call(layout=1, cfg=None, M=40, K=1024, ldq=1024):
        return lib.qf_w8a8_gemm(fake, ldq, fake, fake, 0, layout, fake, fake, 1000, 0, M, 1000, K,
                                ctypes.byref(cfg) if cfg is not None else None, None, 0, None)
    assert call(layout=0) == L.ERR_INVALID_ARG                               # row-major: ldw < K
    assert lib.qf_w8a8_gemm(fake, 1024, fake, fake, 1032, 0, fake, fake, 1000, 0, 40, 1000, 1024, None, None, 0,
                            None) == L.ERR_UNSUPPORTED                        # row-major: ldw % 16
    assert call(layout=2) == L.ERR_INVALID_ARG
    assert call(K=1000, ldq=1000) == L.ERR_UNSUPPORTED                     # K % 64
    assert call(ldq=1024 + 8) == L.ERR_UNSUPPORTED                          # ldq % 16
    assert call(M=0) == L.ERR_INVALID_ARG
    for bad in ((L.KERNEL_MFMA_W8A8, 1, 1, 8, 4, 1, 1, 0), (L.KERNEL_MFMA_W8A8, 1, 2, 8, 8, 1, 1, 0),
                (L.KERNEL_MFMA_W8A8, 1, 2, 16, 4, 1, 1, 0), (L.KERNEL_MFMA_WIDE, 1, 2, 8, 4, 1, 1, 0),
                (L.KERNEL_MFMA_W8A8_TILE, 2, 8, 8, 4, 1, 1, 0), (L.KERNEL_MFMA_W8A8_TILE, 1, 8, 4, 4, 1, 1, 0),
                (L.KERNEL_MFMA_W8A8_TILE, 1, 8, 8, 3, 1, 1, 0), (L.KERNEL_MFMA_W8A8_TILE, 1, 8, 8, 4, 1, 2, 0)):
        assert call(cfg=L.Config.from_seq(bad)) != L.OK, bad
    split = L.Config.from_seq((L.KERNEL_MFMA_W8A8, 2, 2, 8, 4, 1, 1, 1))
    assert call(cfg=split) == L.ERR_WORKSPACE
    # the W8A16 entry point does not take the W8A8 kind
    assert _gemm(x=fake, w=fake, s=fake, y=fake, layout=1, M=40, K=1024, ldx=1024, ldw=1024,
                 cfg=L.Config.from_seq((L.KERNEL_MFMA_W8A8, 1, 2, 8, 4, 1, 1, 0))) == L.ERR_INVALID_ARG
    assert lib.qf_quantize_tokens_int8(None, 64, 1, 64, fake, 64, fake, None) == L.ERR_INVALID_ARG
    assert lib.qf_quantize_tokens_int8(fake, 100, 1, 100, fake, 100, fake, None) == L.ERR_UNSUPPORTED  # K % 64
