"""ctypes binding of ``libmarathon_kvshift.so`` (C ABI: include/marathon_kvshift.h).

The library is built in-tree by :func:`marathon_amd.build.build_library` and loaded
from ``marathon_amd/_lib/``.  There is deliberately no fallback: if the library is
missing, :func:`lib` raises, so a GPU path can never silently run something else.
"""

from __future__ import annotations

import ctypes
import os
import threading

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "_lib")
LIB_NAME = "libmarathon_kvshift.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)

# ---- constants mirrored from the header -----------------------------------------
MKV_OK = 0
MKV_ERR_ARG = 1
MKV_ERR_DTYPE = 2
MKV_ERR_ALIGN = 3
MKV_ERR_UNSUPPORTED = 4
MKV_ERR_HIP = 5

MKV_FLAG_SRC_RANGE = 1
MKV_FLAG_DST_RANGE = 2
MKV_FLAG_SPAN = 4
MKV_FLAG_ALIGN = 8

MKV_BF16 = 0
MKV_F16 = 1
MKV_F32 = 2
MKV_FP8_E4M3 = 3

MKV_ADDR_FLAT = 0
MKV_ADDR_SLOTS = 1
MKV_ADDR_TABLE = 2

MKV_MAX_SPANS = 4096
MKV_MAX_HEAD_SIZE = 512
MKV_DIRECT_MAX_SPANS = 63
MKV_SMALL_MAX_SPANS = 8
MKV_SMALL_MAX_INDEX = 64
MKV_ABI_VERSION = (3 << 16) | 4
MKV_ORDER_NONE = 0
MKV_ORDER_DST_PAGE = 1
MKV_NOALLOC_SCRATCH_BYTES = 16 << 20

ERROR_NAMES = {
    MKV_ERR_ARG: "MKV_ERR_ARG",
    MKV_ERR_DTYPE: "MKV_ERR_DTYPE",
    MKV_ERR_ALIGN: "MKV_ERR_ALIGN",
    MKV_ERR_UNSUPPORTED: "MKV_ERR_UNSUPPORTED",
    MKV_ERR_HIP: "MKV_ERR_HIP",
}

# Every symbol the header declares; tests check the library exports all of them.
EXPORTED = (
    "mkv_scatter_shifted",
    "mkv_shift_spans",
    "mkv_shift_spans_noalloc",
    "mkv_shift_spans_small",
    "mkv_shift_workspace_size",
    "mkv_rope_tables",
    "mkv_last_error",
    "mkv_abi_version",
)


class Span(ctypes.Structure):
    """mkv_span_t (48 bytes)."""

    _fields_ = [
        ("src_pos", ctypes.c_int64),
        ("dst_pos", ctypes.c_int64),
        ("src_index", ctypes.c_int64),
        ("dst_index", ctypes.c_int64),
        ("n_tokens", ctypes.c_int32),
        ("delta", ctypes.c_int32),
        ("src_group", ctypes.c_int32),
        ("dst_group", ctypes.c_int32),
    ]


# numpy twin of mkv_span_t, for building device span tables in bulk
SPAN_DTYPE = np.dtype(
    [
        ("src_pos", "<i8"),
        ("dst_pos", "<i8"),
        ("src_index", "<i8"),
        ("dst_index", "<i8"),
        ("n_tokens", "<i4"),
        ("delta", "<i4"),
        ("src_group", "<i4"),
        ("dst_group", "<i4"),
    ]
)
assert SPAN_DTYPE.itemsize == ctypes.sizeof(Span) == 48


class Side(ctypes.Structure):
    """mkv_side_t (88 bytes)."""

    _fields_ = [
        ("k_base", ctypes.c_void_p),
        ("v_base", ctypes.c_void_p),
        ("index", ctypes.c_void_p),
        ("group_slots", ctypes.c_void_p),
        ("index_len", ctypes.c_int64),
        ("num_slots", ctypes.c_int64),
        ("block_stride", ctypes.c_int64),
        ("head_stride", ctypes.c_int64),
        ("offset_stride", ctypes.c_int64),
        ("block_size", ctypes.c_int32),
        ("mode", ctypes.c_int32),
        ("groups", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class ShiftDesc(ctypes.Structure):
    """mkv_shift_desc_t (288 bytes)."""

    _fields_ = [
        ("spans", ctypes.c_void_p),
        ("inv_freq", ctypes.c_void_p),
        ("k_scale", ctypes.c_void_p),
        ("error_flags", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_int64),
        ("total_tokens", ctypes.c_int64),
        ("n_spans", ctypes.c_int32),
        ("layers", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("head_size", ctypes.c_int32),
        ("rotary", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("src", Side),
        ("dst", Side),
        ("span_starts", ctypes.c_void_p),
        ("span_tables", ctypes.c_void_p),
        ("order", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("token_order", ctypes.c_void_p),
    ]


assert ctypes.sizeof(Side) == 88 and ctypes.sizeof(ShiftDesc) == 288


class KVShiftError(RuntimeError):
    """A non-MKV_OK status from the library."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{ERROR_NAMES.get(code, code)}: {message}")
        self.code = code


_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None


def _bind(cdll: ctypes.CDLL) -> ctypes.CDLL:
    i32, i64, vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p
    f = cdll.mkv_scatter_shifted
    f.restype = ctypes.c_int
    f.argtypes = [vp, i64, i64, vp, i64, i64, i64, i64, vp, i64, i32, i32, i32, i32, vp, vp,
                  i32, vp, vp, vp]
    for name in ("mkv_shift_spans", "mkv_shift_spans_noalloc", "mkv_shift_spans_small"):
        f = getattr(cdll, name)
        f.restype = ctypes.c_int
        f.argtypes = [ctypes.POINTER(ShiftDesc), vp]
    f = cdll.mkv_shift_workspace_size
    f.restype = ctypes.c_int64
    f.argtypes = [i64, i32, i32]
    f = cdll.mkv_rope_tables
    f.restype = ctypes.c_int
    f.argtypes = [vp, i32, vp, i32, vp]
    cdll.mkv_last_error.restype = ctypes.c_char_p
    cdll.mkv_last_error.argtypes = []
    cdll.mkv_abi_version.restype = ctypes.c_int32
    cdll.mkv_abi_version.argtypes = []
    return cdll


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built (no fallback path).

    torch is imported first so that the HIP runtime torch ships is the one the library
    binds to (both carry the soname libamdhip64.so.7).
    """
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with "
                    "`python -c 'import __graft_entry__ as g; g.build()'` "
                    "(marathon_amd has no CPU or fallback path)"
                )
            import torch  # noqa: F401  (bind to torch's HIP runtime)

            cdll = _bind(ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL))
            if cdll.mkv_abi_version() != MKV_ABI_VERSION:
                raise RuntimeError("libmarathon_kvshift ABI version mismatch; rebuild")
            _LIB = cdll
    return _LIB


def check(rc: int) -> None:
    if rc != MKV_OK:
        msg = lib().mkv_last_error().decode(errors="replace")
        raise KVShiftError(rc, msg)


def rope_tables(deltas, inv_freq, rotary: int):
    """``mkv_rope_tables``: the rotation tables of ``deltas`` on the host, fp32
    ``[n_spans, 2, rotary]``, from the routine the device's tables come from.
    ``inv_freq``: fp32 ``[rotary / 2]`` (numpy or a CPU tensor)."""
    import numpy as np

    d = np.ascontiguousarray(np.asarray(deltas), dtype=np.int64)
    if d.size and (d.min() < -2**31 or d.max() >= 2**31):
        raise ValueError("deltas outside int32")
    d = d.astype(np.int32)
    inv = np.ascontiguousarray(np.asarray(inv_freq, dtype=np.float32).reshape(-1))
    out = np.zeros((d.size, 2, rotary), np.float32)
    if rotary == 0 or d.size == 0:
        return out
    if inv.size < rotary // 2:
        raise ValueError(f"inv_freq has {inv.size} entries for rotary {rotary}")
    check(lib().mkv_rope_tables(d.ctypes.data, d.size, inv.ctypes.data, rotary,
                                out.ctypes.data))
    return out
