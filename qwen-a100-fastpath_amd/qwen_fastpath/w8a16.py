"""Small-M W8A16 GEMM over the int8 weights of a W8A8 checkpoint, on MI355X.

Host side of the op (reference: plugin/qwen_fastpath/w8a16.py).  The weights are the checkpoint's
int8 [N, K] row-major matrix -- the [K, N] column-major view vLLM keeps for its int8 GEMM is the same
memory -- with a per-output-channel fp32 scale.  Activations stay bf16; the kernels widen the int8
weights to bf16 in registers, accumulate in fp32 and apply the scale after the K reduction.  The
compute is hand-written HIP for gfx950 behind a C ABI (include/qf_w8a16.h); this module only
allocates outputs and workspaces through torch and launches on torch's current stream.

Public names mirror the reference module:
  SMALL_M        w8a16.py:12     largest M routed to this op
  pick_config    w8a16.py:58-68  None when the shape is not served (K % 64 != 0)
  w8a16_mm       w8a16.py:71-83  y = (x @ W^T) * s as a new [M, N] tensor of out_dtype
"""
from __future__ import annotations

import ctypes
from typing import NamedTuple

import torch

from . import _lib as L

SMALL_M = L.MAX_M
ROWMAJOR = L.LAYOUT_ROWMAJOR
TILED = L.LAYOUT_TILED


class W8A16Config(NamedTuple):
    """Launch configuration; zero fields are chosen by the library for the call's M (see
    qf_w8a16_pick_config).  kernel: 0 auto, 1 gemv (M <= 4), 2 mfma, 3 mfma with x staged in
    chunks through a two-slot LDS ring (k_waves 1), 4 the wide-M mfma kernel (TILED weights, any M;
    k_waves and split_k 1); w8a8_mm only: 5 the int8 wide-M kernel, 6 the int8 LDS-tiled kernel (256 x
    256 workgroups; waves 8, tiles_per_wave 8, depth 4, split_k 1).  waves = wavefronts per workgroup, of which
    k_waves split K inside the workgroup (MFMA); reduce (MFMA, split_k > 1):
    0 = the last workgroup of each n-block sums the splits, 1 = a second kernel does."""

    kernel: int = 0
    split_k: int = 0
    tiles_per_wave: int = 0
    waves: int = 0
    depth: int = 0
    load_hint: int = 0
    k_waves: int = 0
    reduce: int = 0


AUTO = W8A16Config()


def pick_config(N: int, K: int, layout: int = ROWMAJOR) -> W8A16Config | None:
    """Configuration for an [N, K] weight, or None when this op does not serve the shape (the
    caller falls back), as the reference's pick_config does for K not a multiple of 64
    (w8a16.py:63-68).  Kernel, split-K and tiling depend on M, so they are resolved per call."""
    if N < 1 or K < L.K_ALIGN or K % L.K_ALIGN:
        return None
    if layout not in (ROWMAJOR, TILED):
        return None
    return AUTO


def resolve_config(M: int, N: int, K: int, layout: int = ROWMAJOR) -> W8A16Config | None:
    """The configuration the library picks for this M (None: unsupported)."""
    c = L.pick_config(M, N, K, layout)
    return None if c is None else W8A16Config(*c.to_tuple())


_cfg_cache: dict[tuple, L.Config] = {}


def _config_struct(cfg) -> L.Config:
    key = tuple(int(v) for v in cfg)
    c = _cfg_cache.get(key)
    if c is None:
        c = L.Config.from_seq(key)
        _cfg_cache[key] = c
    return c


def _weight_geometry(w: torch.Tensor, N: int, K: int, layout: int) -> int:
    """Validate the weight tensor and return its row stride (bytes between output channels)."""
    if w.dtype != torch.int8:
        raise TypeError(f"weight must be int8, got {w.dtype}")
    if layout == ROWMAJOR:
        # [K, N] with stride (1, ldw): the reference's w_t (w8a16.py:72)
        if w.dim() != 2 or tuple(w.shape) != (K, N) or (w.stride(0) != 1 and K > 1):
            raise ValueError(f"row-major weight must be a [K, N] = [{K}, {N}] view with stride(0) == 1, "
                             f"got shape {tuple(w.shape)} stride {w.stride()}")
        return w.stride(1) if N > 1 else K
    if layout == TILED:
        if not w.is_contiguous() or w.numel() != tiled_numel(N, K):
            raise ValueError(f"TILED weight must be a contiguous image of {tiled_numel(N, K)} bytes")
        return K
    raise ValueError(f"unknown layout {layout}")


# Workspaces (split-K partials and arrival counters, the fused argmax's per-token slots, the row-split
# argmax table), one per (device, stream): calls issued in order on one stream share it, and calls on
# different streams never do, so they may overlap.  The library's arrival counters at the front of a
# workspace must be zero when a call starts and every call leaves them zero, so:
# * an eager workspace is allocated zeroed, grown by doubling, and reused by every later call on its
#   stream; it is kept for the life of the process (one per stream that ran the op);
# * inside a graph capture, calls get a workspace allocated during that capture (so from the graph's
#   memory pool), whose counters are cleared by a fill kernel recorded into the graph ahead of its first
#   use: each replay starts from zero, whatever ran on the stream before.  This module holds it only while
#   the capture is the latest one on its stream; a later capture there releases it, and the graph keeps
#   the memory as it keeps its other intermediates (graphs that share a memory pool may then reuse it,
#   which torch already requires to be replayed one at a time).  So the held capture memory is at most one
#   capture's largest workspace per capture stream, not one per captured size.
_workspaces: dict[tuple, torch.Tensor] = {}
_capture_ws: dict[tuple, tuple[int, list[torch.Tensor]]] = {}  # (device, stream) -> (capture id, buffers)
_WS_MIN = 8 << 20


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    dev = device.index if device.index is not None else torch.cuda.current_device()
    handle = torch.cuda.current_stream(device).cuda_stream
    if torch.cuda.is_current_stream_capturing():
        cid = L.capture_id(handle)
        entry = _capture_ws.get((dev, handle))
        if entry is None or entry[0] != cid:
            entry = (cid, [])  # a new capture on this stream: the previous capture's buffers are released
            _capture_ws[(dev, handle)] = entry
        bufs = entry[1]
        if not bufs or bufs[-1].numel() < nbytes:
            # a larger buffer for the rest of this capture; the earlier ones stay held until it ends, since
            # launches already recorded use them
            ws = torch.empty(max(nbytes, L.COUNTER_BYTES), dtype=torch.uint8, device=device)
            ws[:L.COUNTER_BYTES].zero_()
            bufs.append(ws)
        return bufs[-1]
    key = (dev, handle)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, _WS_MIN, 0 if ws is None else 2 * ws.numel()), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def _on_gpu(*tensors) -> None:
    """Every tensor handed to the library must live on a GPU: a host pointer reaching a kernel faults the device."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise TypeError(f"expected a GPU tensor, got one on {t.device}")


def _launch(x: torch.Tensor, w: torch.Tensor, w_scale: torch.Tensor, layout: int, out_dtype: torch.dtype,
            config) -> torch.Tensor:
    lib = L.load()
    _on_gpu(x, w, w_scale)
    if x.dim() != 2 or x.dtype != torch.bfloat16:
        raise TypeError(f"x must be a 2-D bf16 tensor, got {x.dtype} {tuple(x.shape)}")
    if w_scale.dtype != torch.float32:
        raise TypeError(f"w_scale must be fp32, got {w_scale.dtype}")
    M, K = x.shape
    N = w_scale.numel()
    ldw = _weight_geometry(w, N, K, layout)
    if M == 0:  # no tokens: an empty result, as the reference's masked grid gives
        if out_dtype not in (torch.bfloat16, torch.float32):
            raise TypeError(f"out_dtype must be bf16 or fp32, got {out_dtype}")
        return x.new_empty((0, N), dtype=out_dtype)
    if x.stride(1) != 1 and K > 1:
        x = x.contiguous()
    ldx = x.stride(0) if M > 1 else K
    if x.data_ptr() % 16 or ldx % 8:
        x = x.clone(memory_format=torch.contiguous_format)
        ldx = K
    s = w_scale.reshape(-1)
    if not s.is_contiguous() or s.data_ptr() % 16:
        s = s.clone(memory_format=torch.contiguous_format)
    if out_dtype == torch.bfloat16:
        dt = L.DTYPE_BF16
    elif out_dtype == torch.float32:
        dt = L.DTYPE_F32
    else:
        raise TypeError(f"out_dtype must be bf16 or fp32, got {out_dtype}")
    y = torch.empty((M, N), dtype=out_dtype, device=x.device)
    c = _config_struct(config)
    ws_bytes = int(lib.qf_w8a16_workspace_bytes(M, N, K, layout, ctypes.byref(c)))
    stream = torch.cuda.current_stream(x.device).cuda_stream
    ws = _workspace(x.device, ws_bytes) if ws_bytes else None
    rc = lib.qf_w8a16_gemm(x.data_ptr(), ldx, w.data_ptr(), ldw, layout, s.data_ptr(), y.data_ptr(), N, dt,
                           M, N, K, ctypes.byref(c), ws.data_ptr() if ws is not None else None,
                           ws.numel() if ws is not None else 0, stream)
    L.check(rc, f"qf_w8a16_gemm(M={M}, N={N}, K={K}, layout={layout})")
    return y


@torch.library.custom_op("qwen_fastpath::w8a16_mm", mutates_args=(), device_types="cuda")
def _w8a16_mm_op(x: torch.Tensor, w: torch.Tensor, w_scale: torch.Tensor, layout: int, out_dtype: torch.dtype,
                 config: list[int]) -> torch.Tensor:
    return _launch(x, w, w_scale, layout, out_dtype, config)


@_w8a16_mm_op.register_fake
def _w8a16_mm_fake(x, w, w_scale, layout, out_dtype, config):
    return x.new_empty((x.shape[0], w_scale.numel()), dtype=out_dtype)


def w8a16_mm(x: torch.Tensor, w_t: torch.Tensor, w_scale: torch.Tensor, cfg, out_dtype: torch.dtype,
             layout: int = ROWMAJOR) -> torch.Tensor:
    """y[M, N] = (x @ W^T) * w_scale in out_dtype (reference: w8a16.py:71-83).

    x [M, K] bf16 (row stride arbitrary, unit column stride); w_t [K, N] int8 with stride (1, K) --
    the checkpoint's [N, K] row-major matrix -- or, with layout=TILED, the image made by to_tiled();
    w_scale [N] fp32.  Runs on torch's current stream; graph-capturable (no host synchronisation,
    allocations through torch's caching allocator only)."""
    cfg = AUTO if cfg is None else cfg
    return torch.ops.qwen_fastpath.w8a16_mm(x, w_t, w_scale, int(layout), out_dtype, [int(v) for v in cfg])


def w8a16_mm_rmsnorm(x: torch.Tensor, w_t: torch.Tensor, w_scale: torch.Tensor, cfg, out_dtype: torch.dtype,
                     layout: int = TILED, eps: float = 2.0 ** -23) -> torch.Tensor:
    """w8a16_mm of the rows of x scaled to unit RMS, w8a16_mm(rms_norm_rows(x, eps), ...) bit for bit, in one
    launch where the configuration stages whole rows (qf_w8a16_gemm_rmsnorm); where it does not (a K split,
    row-major weights), the same two calls."""
    _on_gpu(x, w_t, w_scale)
    lib = L.load()
    if x.dim() != 2 or x.dtype != torch.bfloat16 or w_scale.dtype != torch.float32:
        raise TypeError("x must be 2-D bf16 and w_scale fp32")
    M, K = x.shape
    N = w_scale.numel()
    ldw = _weight_geometry(w_t, N, K, layout)
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"out_dtype must be bf16 or fp32, got {out_dtype}")
    if M == 0:
        return x.new_empty((0, N), dtype=out_dtype)
    if x.stride(1) != 1 or x.data_ptr() % 16 or (M > 1 and x.stride(0) % 8):
        x = x.contiguous()
    ldx = x.stride(0) if M > 1 else K
    c = _config_struct(AUTO if cfg is None else cfg)
    ws_bytes = int(lib.qf_w8a16_workspace_bytes(M, N, K, layout, ctypes.byref(c)))
    y = torch.empty((M, N), dtype=out_dtype, device=x.device)
    ws = _workspace(x.device, ws_bytes) if ws_bytes else None
    rc = lib.qf_w8a16_gemm_rmsnorm(x.data_ptr(), ldx, float(eps), w_t.data_ptr(), ldw, layout, w_scale.data_ptr(),
                                   y.data_ptr(), N, L.DTYPE_BF16 if out_dtype == torch.bfloat16 else L.DTYPE_F32,
                                   M, N, K, ctypes.byref(c), ws.data_ptr() if ws is not None else None,
                                   ws.numel() if ws is not None else 0, torch.cuda.current_stream(x.device).cuda_stream)
    if rc == L.ERR_UNSUPPORTED:
        return w8a16_mm(rms_norm_rows(x, eps), w_t, w_scale, cfg, out_dtype, layout)
    L.check(rc, f"qf_w8a16_gemm_rmsnorm(M={M}, N={N}, K={K}, layout={layout})")
    return y


def w8a16_mm_argmax(x: torch.Tensor, w: torch.Tensor, w_scale: torch.Tensor, n_valid: int, index_offset: int = 0,
                    cfg=None, layout: int = ROWMAJOR, with_logits: bool = False):
    """The draft head's argmax fused into the GEMM (the logits of w8a16_mm, then
    index_offset + argmax over the first n_valid columns of the bf16 logits, NaN highest, first index on
    ties: patches.py:160-166,178-185).  Returns the int64 ids [M] -- and the bf16 logits [M, N] when
    with_logits -- or None when the fused path does not serve this configuration (the caller then uses
    w8a16_mm and top_tokens)."""
    _on_gpu(x, w, w_scale)
    lib = L.load()
    if x.dim() != 2 or x.dtype != torch.bfloat16 or w_scale.dtype != torch.float32:
        raise TypeError("x must be 2-D bf16 and w_scale fp32")
    M, K = x.shape
    N = w_scale.numel()
    if not 1 <= n_valid <= N:
        raise ValueError(f"n_valid must be in [1, {N}], got {n_valid}")
    ldw = _weight_geometry(w, N, K, layout)
    c = _config_struct(AUTO if cfg is None else cfg)
    ws_bytes = int(lib.qf_w8a16_argmax_workspace_bytes(M, N, K, layout, ctypes.byref(c)))
    if ws_bytes == 0:
        return None
    if x.stride(1) != 1 or x.data_ptr() % 16 or (M > 1 and x.stride(0) % 8):
        x = x.clone(memory_format=torch.contiguous_format)
    ldx = x.stride(0) if M > 1 else K
    s = w_scale.reshape(-1)
    if not s.is_contiguous() or s.data_ptr() % 16:
        s = s.clone(memory_format=torch.contiguous_format)
    ids = torch.empty((M,), dtype=torch.int64, device=x.device)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device) if with_logits else None
    ws = _workspace(x.device, ws_bytes)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    rc = lib.qf_w8a16_gemm_argmax(x.data_ptr(), ldx, w.data_ptr(), ldw, layout, s.data_ptr(),
                                  y.data_ptr() if y is not None else None, N, L.DTYPE_BF16, M, N, K, int(n_valid),
                                  int(index_offset), ids.data_ptr(), ctypes.byref(c), ws.data_ptr(), ws.numel(),
                                  stream)
    L.check(rc, f"qf_w8a16_gemm_argmax(M={M}, N={N}, K={K}, layout={layout})")
    return (ids, y) if with_logits else ids


# ------------------------------------------------------------------------------------------------
# weight layout
# ------------------------------------------------------------------------------------------------

def tiled_numel(N: int, K: int) -> int:
    return (N + 15) // 16 * 16 * K


def to_tiled(w_t: torch.Tensor) -> torch.Tensor:
    """Pre-permuted image of a [K, N] stride-(1, K) int8 weight: 1 KiB tiles of 16 output channels
    x 64 k, tile (t, s) at byte ((t * K/64) + s) * 1024, lane l of the tile holding channel
    16 t + l % 16, k = 64 s + 16 (l // 16) .. +15.  Every 64-lane 16-byte load of the kernel then
    reads one contiguous KiB."""
    _on_gpu(w_t)
    K, N = w_t.shape
    ldw = _weight_geometry(w_t, N, K, ROWMAJOR)
    out = torch.empty(tiled_numel(N, K), dtype=torch.int8, device=w_t.device)
    stream = torch.cuda.current_stream(w_t.device).cuda_stream
    L.check(L.load().qf_w8a16_repack(w_t.data_ptr(), ldw, out.data_ptr(), N, K, stream), "qf_w8a16_repack")
    return out


def from_tiled(w_tiled: torch.Tensor, N: int, K: int) -> torch.Tensor:
    """Inverse of to_tiled: returns the [K, N] stride-(1, K) view of a fresh [N, K] matrix."""
    _on_gpu(w_tiled)
    out = torch.empty((N, K), dtype=torch.int8, device=w_tiled.device)
    stream = torch.cuda.current_stream(w_tiled.device).cuda_stream
    L.check(L.load().qf_w8a16_unpack(w_tiled.data_ptr(), out.data_ptr(), K, N, K, stream), "qf_w8a16_unpack")
    return out.t()


# ------------------------------------------------------------------------------------------------
# M beyond the decode widths (prefill) on weights this library laid out
# ------------------------------------------------------------------------------------------------

# Output channels widened per library GEMM of w8a16_mm_prefill: the whole weight up to
# PREFILL_WHOLE_MAX_N channels, PREFILL_CHUNK_ROWS at a time above (hipBLASLt's own tiling picks:
# qkv 10240 x 5120 at M = 1024 takes 136 us in one GEMM against 159 us in 8192 + 2048, while
# gate_up 34816 x 5120 takes 478 us in 8192-row chunks against 529 us whole).
PREFILL_CHUNK_ROWS = 8192
PREFILL_WHOLE_MAX_N = 12288


def dequant_bf16(w: torch.Tensor, N: int, K: int, layout: int = ROWMAJOR, n0: int = 0, rows: int | None = None,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """Exact bf16 copy [rows, K] of weight rows [n0, n0 + rows) (no scale), from a [K, N] stride-(1, K)
    view or from the TILED image."""
    _on_gpu(w, out)
    rows = N - n0 if rows is None else rows
    ldw = _weight_geometry(w, N, K, layout)
    if out is None:
        out = torch.empty((rows, K), dtype=torch.bfloat16, device=w.device)
    if out.dtype != torch.bfloat16 or out.dim() != 2 or out.shape[0] < rows or out.shape[1] < K or out.stride(1) != 1:
        raise ValueError("out must be a bf16 [>= rows, >= K] matrix with unit column stride")
    stream = torch.cuda.current_stream(w.device).cuda_stream
    L.check(L.load().qf_w8a16_dequant_bf16(w.data_ptr(), ldw, layout, N, K, n0, rows, out.data_ptr(), out.stride(0),
                                          stream), "qf_w8a16_dequant_bf16")
    return out


def scale_cast_bf16(acc: torch.Tensor, w_scale: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out[m, n] = bf16(acc[m, n] * w_scale[n]) in one pass (qf_scale_cast_bf16): acc fp32 [M, N] and
    out bf16 [M, N], both with unit column stride; bit-identical to (acc * w_scale).to(torch.bfloat16)."""
    _on_gpu(acc, w_scale, out)
    M, N = acc.shape
    if acc.dtype != torch.float32 or out.dtype != torch.bfloat16 or w_scale.dtype != torch.float32:
        raise TypeError("acc and w_scale must be fp32, out bf16")
    if tuple(out.shape) != (M, N) or w_scale.numel() != N or acc.stride(1) != 1 or out.stride(1) != 1:
        raise ValueError("acc [M, N], out [M, N] with unit column strides and w_scale [N] expected")
    s = w_scale.reshape(-1)
    if not s.is_contiguous():
        s = s.contiguous()
    stream = torch.cuda.current_stream(acc.device).cuda_stream
    L.check(L.load().qf_scale_cast_bf16(acc.data_ptr(), acc.stride(0) if M > 1 else N, s.data_ptr(), M, N,
                                        out.data_ptr(), out.stride(0) if M > 1 else N, stream),
            "qf_scale_cast_bf16")
    return out


def rms_norm_rows(x: torch.Tensor, eps: float = 2.0 ** -23, out: torch.Tensor | None = None) -> torch.Tensor:
    """Each row of a bf16 [M, N] tensor scaled to unit RMS in one launch (qf_rms_norm_rows_bf16):
    bf16(x * (1 / sqrt(mean(x^2) + eps))), within one bf16 ulp of torch.nn.functional.rms_norm(x, (N,), eps=eps)
    (whose default eps for a bf16 input is float32's epsilon, 2^-23, the default here too).  The glue between
    the layers of the 64-layer decode-step benchmark; N % 8 == 0."""
    _on_gpu(x, out)
    if x.dim() != 2 or x.dtype != torch.bfloat16:
        raise TypeError("x must be a 2-D bf16 tensor")
    M, N = x.shape
    if x.stride(1) != 1 or x.data_ptr() % 16 or (M > 1 and x.stride(0) % 8):
        x = x.contiguous()
    if out is None:
        y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    else:
        y = out
        if (y.dtype != torch.bfloat16 or y.dim() != 2 or tuple(y.shape) != (M, N) or y.device != x.device
                or y.stride(1) != 1 or y.data_ptr() % 16 or (M > 1 and y.stride(0) % 8)):
            raise ValueError(f"out must be a bf16 [{M}, {N}] tensor on {x.device} with unit column stride, 16-byte "
                             f"aligned rows and a row stride that is a multiple of 8")
    if M == 0:
        return y
    stream = torch.cuda.current_stream(x.device).cuda_stream
    L.check(L.load().qf_rms_norm_rows_bf16(x.data_ptr(), x.stride(0) if M > 1 else N, M, N, float(eps), y.data_ptr(),
                                           y.stride(0) if M > 1 else N, stream), "qf_rms_norm_rows_bf16")
    return y


def quantize_tokens_int8(x: torch.Tensor, tiled: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Dynamic symmetric per-token int8 quantisation (qf_quantize_tokens_int8): s_a[m] = amax|x[m]| /
    127 (as the fp32 reciprocal product), xq = clamp(round_half_even(x / s_a), -128, 127), zero rows -> 0.
    The arithmetic of vLLM's scaled_int8_quant(x, symmetric=True) at the reference's fallback
    (plugin/qwen_fastpath/patches.py:99).  x bf16 [M, K], K % 64 == 0.  Returns (xq int8 [M, K], s_a fp32 [M]);
    with tiled=True xq is instead the token-tiled image (qf_quantize_tokens_int8_tiled), a flat int8 tensor
    of ceil(M/16) * 16 * K bytes (the layout w8a8_mm hands the LDS-tiled kernel)."""
    _on_gpu(x)
    if x.dim() != 2 or x.dtype != torch.bfloat16:
        raise TypeError("x must be a 2-D bf16 tensor")
    M, K = x.shape
    if x.stride(1) != 1 or x.data_ptr() % 16 or (M > 1 and x.stride(0) % 8):
        x = x.clone(memory_format=torch.contiguous_format)
    if tiled:
        xq = torch.empty(((M + 15) // 16 * 16 * K,), dtype=torch.int8, device=x.device)
    else:
        xq = torch.empty((M, K), dtype=torch.int8, device=x.device)
    s_a = torch.empty((M,), dtype=torch.float32, device=x.device)
    if M == 0:
        return xq, s_a
    stream = torch.cuda.current_stream(x.device).cuda_stream
    ldx = x.stride(0) if M > 1 else K
    if tiled:
        L.check(L.load().qf_quantize_tokens_int8_tiled(x.data_ptr(), ldx, M, K, xq.data_ptr(), s_a.data_ptr(), stream),
                "qf_quantize_tokens_int8_tiled")
    else:
        L.check(L.load().qf_quantize_tokens_int8(x.data_ptr(), ldx, M, K, xq.data_ptr(), K, s_a.data_ptr(), stream),
                "qf_quantize_tokens_int8")
    return xq, s_a


def w8a8_mm(x: torch.Tensor, w: torch.Tensor, w_scale: torch.Tensor, out_dtype: torch.dtype, cfg=None,
            layout: int = TILED, x_tiled: bool | None = None) -> torch.Tensor:
    """y = ((xq @ W^T) * s_a) * w_scale with per-token int8 activations (quantize_tokens_int8), exact
    int32 sums on the int8 MFMA: the arithmetic of the reference's M > 16 fallback, scaled_int8_quant +
    cutlass_scaled_mm (plugin/qwen_fastpath/patches.py:99-100).  w is the TILED image or the [K, N]
    stride-(1, K) view of the checkpoint's row-major weight (layout=ROWMAJOR).  Any M.  x_tiled selects
    the activations' layout between the two launches (qf_quantize_tokens_int8_tiled + qf_w8a8_gemm_xt, or
    the row-major pair); None picks the tiled one when the call runs the LDS-tiled kernel.  The result is
    the same either way."""
    _on_gpu(x, w, w_scale)
    lib = L.load()
    if w_scale.dtype != torch.float32:
        raise TypeError(f"w_scale must be fp32, got {w_scale.dtype}")
    M, K = x.shape
    N = w_scale.numel()
    ldw = _weight_geometry(w, N, K, layout)
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"out_dtype must be bf16 or fp32, got {out_dtype}")
    if M == 0:
        return x.new_empty((0, N), dtype=out_dtype)
    c = _config_struct(AUTO if cfg is None else cfg)
    if x_tiled is None:
        kernel = c.kernel
        if kernel == 0:
            picked = L.w8a8_pick_config(M, N, K, layout)
            kernel = picked.kernel if picked is not None else 0
        x_tiled = kernel == L.KERNEL_MFMA_W8A8_TILE
    xq, s_a = quantize_tokens_int8(x, tiled=x_tiled)
    s = w_scale.reshape(-1)
    if not s.is_contiguous() or s.data_ptr() % 16:
        s = s.clone(memory_format=torch.contiguous_format)
    if out_dtype == torch.bfloat16:
        dt = L.DTYPE_BF16
    elif out_dtype == torch.float32:
        dt = L.DTYPE_F32
    else:
        raise TypeError(f"out_dtype must be bf16 or fp32, got {out_dtype}")
    y = torch.empty((M, N), dtype=out_dtype, device=x.device)
    ws_bytes = int(lib.qf_w8a8_workspace_bytes(M, N, K, layout, ctypes.byref(c)))
    ws = _workspace(x.device, ws_bytes) if ws_bytes else None
    stream = torch.cuda.current_stream(x.device).cuda_stream
    ws_ptr, ws_n = (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)
    if x_tiled:
        rc = lib.qf_w8a8_gemm_xt(xq.data_ptr(), s_a.data_ptr(), w.data_ptr(), ldw, layout, s.data_ptr(), y.data_ptr(),
                                 N, dt, M, N, K, ctypes.byref(c), ws_ptr, ws_n, stream)
    else:
        rc = lib.qf_w8a8_gemm(xq.data_ptr(), K, s_a.data_ptr(), w.data_ptr(), ldw, layout, s.data_ptr(), y.data_ptr(),
                              N, dt, M, N, K, ctypes.byref(c), ws_ptr, ws_n, stream)
    L.check(rc, f"qf_w8a8_gemm{'_xt' if x_tiled else ''}(M={M}, N={N}, K={K}, layout={layout})")
    return y


def w8a16_mm_prefill(x: torch.Tensor, w: torch.Tensor, w_scale: torch.Tensor, out_dtype: torch.dtype,
                     layout: int = TILED, chunk_rows: int | None = None) -> torch.Tensor:
    """y[M, N] = (x @ W^T) * w_scale for any M, the same product as w8a16_mm: the int8 weights are
    widened to bf16 exactly, chunk_rows output channels at a time (default: all of them up to
    PREFILL_WHOLE_MAX_N, else PREFILL_CHUNK_ROWS), multiplied by a library bf16 GEMM
    with fp32 accumulation (hipBLASLt through torch.mm), and scaled after the K reduction, then
    rounded to out_dtype (bf16: one qf_scale_cast_bf16 pass per chunk).  This serves M above the
    wide-M kernel's range on weights kept in the TILED layout; the reference sends M > 16 to CUTLASS
    W8A8 on the checkpoint layout (plugin/qwen_fastpath/patches.py:99-100)."""
    if x.dim() != 2 or x.dtype != torch.bfloat16:
        raise TypeError("x must be a 2-D bf16 tensor")
    M, K = x.shape
    N = w_scale.numel()
    s = w_scale.reshape(-1).float().contiguous()
    y = torch.empty((M, N), dtype=out_dtype, device=x.device)
    if chunk_rows is None:
        chunk_rows = N if N <= PREFILL_WHOLE_MAX_N else PREFILL_CHUNK_ROWS
    rows = min(chunk_rows, N)
    wb = torch.empty((rows, K), dtype=torch.bfloat16, device=x.device)
    for n0 in range(0, N, rows):
        r = min(rows, N - n0)
        dequant_bf16(w, N, K, layout, n0, r, wb)
        y32 = torch.mm(x, wb[:r].t(), out_dtype=torch.float32)
        if out_dtype == torch.bfloat16:
            scale_cast_bf16(y32, s[n0:n0 + r], y[:, n0:n0 + r])
        else:
            y[:, n0:n0 + r] = (y32 * s[n0:n0 + r]).to(out_dtype)
    return y
