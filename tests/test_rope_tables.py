"""The library's host table routine (``mkv_rope_tables``, marathon_amd/csrc/rope_angle.h),
against the oracle, on the CPU.

The plan pass and the small path run the same routine on the device (the GPU test
tests/test_gpu_tables.py reads their tables back through the kernels), so this pins
every path's tables: each entry must be the fp32 rounding of the float64 cosine or sine
of the fp32 angle fl32(delta * inv_freq[f]) (the oracle, shift_kernels.py:73-84), for
every delta in [-32768, 32768] and 200,000 seeded int32 deltas, at theta 1e4 and 1e6,
rotary 128; and the table layout is the span-table one (cos twice, then -sin, +sin).
"""

from __future__ import annotations

import numpy as np
import pytest

from marathon_amd import _lib
from marathon_amd.shift_kernels import inv_freq_for
from oracle import kvshift_oracle as orc


def _oracle(deltas: np.ndarray, inv: np.ndarray):
    ang = deltas.astype(np.float32)[:, None] * inv[None, :]  # fp32 products
    a64 = ang.astype(np.float64)
    return np.cos(a64).astype(np.float32), np.sin(a64).astype(np.float32)


@pytest.mark.parametrize("theta", [1e4, 1e6])
def test_host_tables_match_the_oracle(theta):
    inv = inv_freq_for(128, theta).numpy()
    rng = np.random.default_rng(int(theta) + 3)
    deltas = np.concatenate((np.arange(-32768, 32769),
                             rng.integers(-2**31, 2**31, size=200000))).astype(np.int64)
    half = inv.size
    for lo in range(0, deltas.size, 50000):
        d = deltas[lo:lo + 50000]
        t = _lib.rope_tables(d, inv, 2 * half)
        c, s = _oracle(d, inv)
        assert np.array_equal(t[:, 0, :half].view(np.uint32), c.view(np.uint32))
        assert np.array_equal(t[:, 0, half:].view(np.uint32), c.view(np.uint32))
        assert np.array_equal(t[:, 1, :half].view(np.uint32), (-s).view(np.uint32))
        assert np.array_equal(t[:, 1, half:].view(np.uint32), s.view(np.uint32))


def test_host_tables_agree_with_the_oracles_own_routine():
    inv = inv_freq_for(128, 1e6).numpy()
    for delta in (1, -1, 37, 186, -4096, 131071, 2**24 + 1, -(2**31)):
        c, s = orc.cos_sin(delta, inv)
        t = _lib.rope_tables([delta], inv, 128)[0]
        assert np.array_equal(t[0, :64].view(np.uint32), c.view(np.uint32)), delta
        assert np.array_equal(t[1, 64:].view(np.uint32), s.view(np.uint32)), delta


def test_partial_rotary_and_arguments():
    inv = inv_freq_for(128, 1e4, partial_rotary_factor=0.25).numpy()  # rotary 32
    t = _lib.rope_tables([5, -7], inv, 32)
    assert t.shape == (2, 2, 32)
    c, s = _oracle(np.array([5, -7]), inv)
    assert np.array_equal(t[:, 0, 16:], c) and np.array_equal(t[:, 1, :16], -s)
    lib = _lib.lib()
    d = np.zeros(1, np.int32)
    out = np.zeros(256, np.float32)
    assert lib.mkv_rope_tables(d.ctypes.data, 1, inv.ctypes.data, 31, out.ctypes.data) == \
        _lib.MKV_ERR_ARG  # odd rotary
    assert lib.mkv_rope_tables(d.ctypes.data, -1, inv.ctypes.data, 32, out.ctypes.data) == \
        _lib.MKV_ERR_ARG
    assert lib.mkv_rope_tables(None, 1, inv.ctypes.data, 32, out.ctypes.data) == _lib.MKV_ERR_ARG
    assert lib.mkv_rope_tables(None, 0, None, 32, None) == _lib.MKV_OK  # nothing to do
    with pytest.raises(ValueError, match="int32"):
        _lib.rope_tables([2**31], inv, 32)
