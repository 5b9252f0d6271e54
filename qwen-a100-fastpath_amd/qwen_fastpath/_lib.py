"""ctypes binding of libqf_w8a16.so, the C ABI declared in include/qf_w8a16.h.

The library is built in-tree (qwen-a100-fastpath_amd/csrc/Makefile) next to this file.  There is no
fallback implementation: if the library is missing, every GPU entry point raises.
"""
from __future__ import annotations

import ctypes
import os

LIB_NAME = "libqf_w8a16.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 1

# qf_status
OK = 0
ERR_INVALID_ARG = 1
ERR_UNSUPPORTED = 2
ERR_WORKSPACE = 3
ERR_HIP = 4

# qf_layout / qf_dtype / qf_kernel
LAYOUT_ROWMAJOR = 0
LAYOUT_TILED = 1
DTYPE_BF16 = 0
DTYPE_F32 = 1
KERNEL_AUTO = 0
KERNEL_GEMV = 1
KERNEL_MFMA = 2
KERNEL_MFMA_XRING = 3
KERNEL_MFMA_WIDE = 4
KERNEL_MFMA_W8A8 = 5
KERNEL_MFMA_W8A8_TILE = 6
KERNEL_MFMA_STREAM = 7

MAX_M = 16
K_ALIGN = 64
COUNTER_BYTES = 65536  # QF_W8A16_COUNTER_BYTES: arrival counters at the front of a workspace
SCRATCH_BYTES = 4 << 20  # QF_W8A16_SCRATCH_BYTES: static scratch of qf_w8a16_gemm_noalloc, per device

# Every symbol include/qf_w8a16.h declares.
EXPORTS = (
    "qf_abi_version",
    "qf_status_string",
    "qf_w8a16_pick_config",
    "qf_w8a16_workspace_bytes",
    "qf_w8a16_gemm",
    "qf_w8a16_gemm_noalloc",
    "qf_w8a16_tiled_bytes",
    "qf_w8a16_repack",
    "qf_w8a16_unpack",
    "qf_w8a16_dequant_bf16",
    "qf_scale_cast_bf16",
    "qf_rms_norm_rows_bf16",
    "qf_w8a16_gemm_rmsnorm",
    "qf_quantize_rows_int8",
    "qf_argmax_rows_bf16",
    "qf_argmax_rows_workspace_bytes",
    "qf_argmax_rows_bf16_ws",
    "qf_w8a16_gemm_argmax",
    "qf_w8a16_argmax_workspace_bytes",
    "qf_stream_capture_info",
    "qf_read_probe",
    "qf_quantize_tokens_int8",
    "qf_w8a8_gemm",
    "qf_tokens_tiled_bytes",
    "qf_quantize_tokens_int8_tiled",
    "qf_w8a8_gemm_xt",
    "qf_w8a8_pick_config",
    "qf_w8a8_workspace_bytes",
    "qf_w8a8_launch_plan",
    "qf_read_probe_stream",
    "qf_empty_kernel",
    "qf_device_cus",
)


class Config(ctypes.Structure):
    """struct qf_w8a16_config."""

    _fields_ = [
        ("kernel", ctypes.c_int32),
        ("split_k", ctypes.c_int32),
        ("tiles_per_wave", ctypes.c_int32),
        ("waves", ctypes.c_int32),
        ("depth", ctypes.c_int32),
        ("load_hint", ctypes.c_int32),
        ("k_waves", ctypes.c_int32),
        ("reduce", ctypes.c_int32),
    ]

    FIELDS = ("kernel", "split_k", "tiles_per_wave", "waves", "depth", "load_hint", "k_waves", "reduce")

    @classmethod
    def from_seq(cls, seq) -> "Config":
        c = cls()
        for name, v in zip(cls.FIELDS, seq):
            setattr(c, name, int(v))
        return c

    def to_tuple(self):
        return tuple(int(getattr(self, f)) for f in self.FIELDS)


class QFError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: {status_string(status)} (status {status})")


_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the library once.  Raises ImportError (never falls back) when it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `make -C qwen-a100-fastpath_amd/csrc` "
            "(or __graft_entry__.build()); the W8A16 op has no non-HIP implementation")
    # torch first: its HIP runtime (soname libamdhip64.so.7) must be the one this library binds to.
    import torch  # noqa: F401
    L = ctypes.CDLL(LIB_PATH)
    p, i64, i32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t
    L.qf_abi_version.argtypes = []
    L.qf_abi_version.restype = i32
    L.qf_status_string.argtypes = [i32]
    L.qf_status_string.restype = ctypes.c_char_p
    L.qf_w8a16_pick_config.argtypes = [i32, i32, i32, i32, ctypes.POINTER(Config)]
    L.qf_w8a16_pick_config.restype = i32
    L.qf_w8a16_workspace_bytes.argtypes = [i32, i32, i32, i32, ctypes.POINTER(Config)]
    L.qf_w8a16_workspace_bytes.restype = sz
    L.qf_w8a16_gemm.argtypes = [p, i64, p, i64, i32, p, p, i64, i32, i32, i32, i32,
                                ctypes.POINTER(Config), p, sz, p]
    L.qf_w8a16_gemm.restype = i32
    L.qf_w8a16_gemm_noalloc.argtypes = [p, i64, p, i64, i32, p, p, i64, i32, i32, i32, i32, ctypes.POINTER(Config), p]
    L.qf_w8a16_gemm_noalloc.restype = i32
    L.qf_w8a16_tiled_bytes.argtypes = [i32, i32]
    L.qf_w8a16_tiled_bytes.restype = sz
    L.qf_w8a16_repack.argtypes = [p, i64, p, i32, i32, p]
    L.qf_w8a16_repack.restype = i32
    L.qf_w8a16_unpack.argtypes = [p, p, i64, i32, i32, p]
    L.qf_w8a16_unpack.restype = i32
    L.qf_w8a16_dequant_bf16.argtypes = [p, i64, i32, i32, i32, i32, i32, p, i64, p]
    L.qf_w8a16_dequant_bf16.restype = i32
    L.qf_scale_cast_bf16.argtypes = [p, i64, p, i32, i32, p, i64, p]
    L.qf_scale_cast_bf16.restype = i32
    L.qf_rms_norm_rows_bf16.argtypes = [p, i64, i32, i32, ctypes.c_float, p, i64, p]
    L.qf_rms_norm_rows_bf16.restype = i32
    L.qf_w8a16_gemm_rmsnorm.argtypes = [p, i64, ctypes.c_float, p, i64, i32, p, p, i64, i32, i32, i32, i32,
                                        ctypes.POINTER(Config), p, sz, p]
    L.qf_w8a16_gemm_rmsnorm.restype = i32
    L.qf_quantize_rows_int8.argtypes = [p, i64, p, p, i32, i32, p]
    L.qf_quantize_rows_int8.restype = i32
    L.qf_argmax_rows_bf16.argtypes = [p, i64, i32, i32, i32, i64, p, p]
    L.qf_argmax_rows_bf16.restype = i32
    L.qf_argmax_rows_workspace_bytes.argtypes = []
    L.qf_argmax_rows_workspace_bytes.restype = sz
    L.qf_argmax_rows_bf16_ws.argtypes = [p, i64, i32, i32, i32, i64, p, p, sz, p]
    L.qf_argmax_rows_bf16_ws.restype = i32
    L.qf_stream_capture_info.argtypes = [p, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_ulonglong)]
    L.qf_stream_capture_info.restype = i32
    L.qf_w8a16_gemm_argmax.argtypes = [p, i64, p, i64, i32, p, p, i64, i32, i32, i32, i32, i32, i64, p,
                                       ctypes.POINTER(Config), p, sz, p]
    L.qf_w8a16_gemm_argmax.restype = i32
    L.qf_w8a16_argmax_workspace_bytes.argtypes = [i32, i32, i32, i32, ctypes.POINTER(Config)]
    L.qf_w8a16_argmax_workspace_bytes.restype = sz
    L.qf_quantize_tokens_int8.argtypes = [p, i64, i32, i32, p, i64, p, p]
    L.qf_quantize_tokens_int8.restype = i32
    L.qf_w8a8_gemm.argtypes = [p, i64, p, p, i64, i32, p, p, i64, i32, i32, i32, i32, ctypes.POINTER(Config), p, sz, p]
    L.qf_w8a8_gemm.restype = i32
    L.qf_tokens_tiled_bytes.argtypes = [i32, i32]
    L.qf_tokens_tiled_bytes.restype = sz
    L.qf_quantize_tokens_int8_tiled.argtypes = [p, i64, i32, i32, p, p, p]
    L.qf_quantize_tokens_int8_tiled.restype = i32
    L.qf_w8a8_gemm_xt.argtypes = [p, p, p, i64, i32, p, p, i64, i32, i32, i32, i32, ctypes.POINTER(Config), p, sz, p]
    L.qf_w8a8_gemm_xt.restype = i32
    L.qf_w8a8_pick_config.argtypes = [i32, i32, i32, i32, ctypes.POINTER(Config)]
    L.qf_w8a8_pick_config.restype = i32
    L.qf_w8a8_workspace_bytes.argtypes = [i32, i32, i32, i32, ctypes.POINTER(Config)]
    L.qf_w8a8_workspace_bytes.restype = sz
    L.qf_w8a8_launch_plan.argtypes = [i32, i32, i32, i32, ctypes.POINTER(Config), ctypes.POINTER(i64),
                                      ctypes.POINTER(ctypes.c_int)]
    L.qf_w8a8_launch_plan.restype = i32
    L.qf_read_probe.argtypes = [p, sz, p, i32, p]
    L.qf_read_probe.restype = i32
    L.qf_read_probe_stream.argtypes = [p, sz, p, i32, i32, p]
    L.qf_read_probe_stream.restype = i32
    L.qf_empty_kernel.argtypes = [p]
    L.qf_empty_kernel.restype = i32
    L.qf_device_cus.argtypes = []
    L.qf_device_cus.restype = i32
    v = L.qf_abi_version()
    if v != ABI_VERSION:
        raise ImportError(f"{LIB_PATH}: ABI version {v}, expected {ABI_VERSION}")
    _lib = L
    return L


def status_string(status: int) -> str:
    try:
        return load().qf_status_string(status).decode()
    except ImportError:
        return f"status {status}"


def check(status: int, what: str) -> None:
    if status != OK:
        raise QFError(status, what)


def pick_config(M: int, N: int, K: int, layout: int = LAYOUT_ROWMAJOR) -> Config | None:
    c = Config()
    rc = load().qf_w8a16_pick_config(M, N, K, layout, ctypes.byref(c))
    if rc == ERR_UNSUPPORTED:
        return None
    check(rc, "qf_w8a16_pick_config")
    return c


def w8a8_pick_config(M: int, N: int, K: int, layout: int = LAYOUT_TILED) -> Config | None:
    c = Config()
    rc = load().qf_w8a8_pick_config(M, N, K, layout, ctypes.byref(c))
    if rc == ERR_UNSUPPORTED:
        return None
    check(rc, "qf_w8a8_pick_config")
    return c


W8A8_LAUNCH_KINDS = ("tile", "tile_256x128", "tile_128x128", "wide", "split_reduce")


def w8a8_launch_plan(M: int, N: int, K: int, layout: int = LAYOUT_TILED, cfg: Config | None = None) -> list[tuple]:
    """The launches qf_w8a8_gemm makes, in stream order: (kind name, workgroups, first channel, channels)."""
    out = (ctypes.c_int64 * 8)()
    count = ctypes.c_int(0)
    check(load().qf_w8a8_launch_plan(M, N, K, layout, ctypes.byref(cfg) if cfg is not None else None, out,
                                     ctypes.byref(count)), "qf_w8a8_launch_plan")
    return [(W8A8_LAUNCH_KINDS[out[4 * i]], int(out[4 * i + 1]), int(out[4 * i + 2]), int(out[4 * i + 3]))
            for i in range(count.value)]


def capture_id(stream_handle: int) -> int:
    """Id of the graph capture `stream_handle` is recording (0 when it is not capturing)."""
    capturing, cid = ctypes.c_int(0), ctypes.c_ulonglong(0)
    check(load().qf_stream_capture_info(stream_handle, ctypes.byref(capturing), ctypes.byref(cid)),
          "qf_stream_capture_info")
    return int(cid.value) if capturing.value else 0


def workspace_bytes(M: int, N: int, K: int, layout: int, cfg: Config | None) -> int:
    return int(load().qf_w8a16_workspace_bytes(M, N, K, layout, ctypes.byref(cfg) if cfg is not None else None))
