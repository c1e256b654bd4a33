"""ctypes front of ``oracle/rotate_c.c`` -- TEST INFRASTRUCTURE ONLY.

:func:`rotate_k_bits` computes exactly what :func:`oracle.kvshift_oracle.rotate_k_bits`
computes (same tables, same op order, same rounding), in C and over several threads, so
the full-size GPU tests can hold every K row to the oracle.  The two are pinned
bit-identical by ``tests/test_oracle_c.py``.
"""

from __future__ import annotations

import ctypes
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from . import kvshift_oracle as orc

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_lib", "liborc_rotate.so")
CODES = {"bf16": 0, "f16": 1, "f32": 2, "fp8": 3}

_LIB = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run `make -C oracle` "
                               "(or __graft_entry__.build())")
        cdll = ctypes.CDLL(LIB_PATH)
        vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
        cdll.orc_rotate_k.restype = ctypes.c_int
        cdll.orc_rotate_k.argtypes = [ctypes.c_int, vp, vp, i64, i32, i32, vp, vp, f32]
        cdll.orc_bf16_enc.restype = ctypes.c_uint16
        cdll.orc_bf16_enc.argtypes = [f32]
        cdll.orc_f16_enc.restype = ctypes.c_uint16
        cdll.orc_f16_enc.argtypes = [f32]
        cdll.orc_f16_dec.restype = f32
        cdll.orc_f16_dec.argtypes = [ctypes.c_uint16]
        cdll.orc_e4m3_dec.restype = f32
        cdll.orc_e4m3_dec.argtypes = [ctypes.c_uint8]
        cdll.orc_e4m3_enc_clamped.restype = ctypes.c_uint8
        cdll.orc_e4m3_enc_clamped.argtypes = [f32]
        _LIB = cdll
    return _LIB


def rotate_k_bits(k_bits: np.ndarray, delta: int, inv: np.ndarray, dtype: str,
                  k_scale: float | None = None, threads: int = 8,
                  method: str = "cr") -> np.ndarray:
    """Bit patterns ``[..., head_size]`` of K rotated by ``delta``; see the oracle's
    function of the same name.  ``threads`` workers split the rows."""
    k_bits = np.ascontiguousarray(k_bits, dtype=orc.BITS_DTYPE[dtype])
    rotary = 2 * int(np.asarray(inv).shape[0])
    if delta == 0 or rotary == 0:
        return k_bits.copy()
    head = k_bits.shape[-1]
    rows = k_bits.size // head if head else 0
    c, s = orc.cos_sin(delta, inv, method)
    c = np.ascontiguousarray(c, np.float32)
    s = np.ascontiguousarray(s, np.float32)
    out = np.empty_like(k_bits)
    scale = float(np.float32(k_scale)) if k_scale is not None else 1.0
    L = lib()
    eb = k_bits.itemsize
    step = max(1, -(-rows // max(1, threads)))

    def run(r0: int) -> int:
        n = min(step, rows - r0)
        return L.orc_rotate_k(CODES[dtype], k_bits.ctypes.data + r0 * head * eb,
                              out.ctypes.data + r0 * head * eb, n, head, rotary,
                              c.ctypes.data, s.ctypes.data, scale)

    starts = list(range(0, rows, step))
    if len(starts) <= 1:
        rcs = [run(r0) for r0 in starts]
    else:
        with ThreadPoolExecutor(len(starts)) as ex:  # ctypes releases the GIL
            rcs = list(ex.map(run, starts))
    if any(rcs):
        raise ValueError("orc_rotate_k refused its arguments")
    return out
