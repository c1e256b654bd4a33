"""The shift kernel's fp8 e4m3fn codec, value by value, on the GPU.

The codec (marathon_amd/csrc/fp8_e4m3.h: gfx950's hardware conversions, the division
by the K scale, the clamp and the NaN rewrite) runs through a small test library
(tests/hip/fp8_codec_probe.hip) on inputs that real shifts reach only by chance:
every exact midpoint between neighbouring codes (ties to even), the fp32 neighbours of
each midpoint, the clamp range, signed zeros, subnormals and NaN.  The expected codes
come from the oracle's nearest-value search (pinned against torch's float8_e4m3fn cast
on the CPU).
"""

from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest
import torch

from oracle import kvshift_oracle as orc

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libfp8_codec_probe.so")


@pytest.fixture(scope="module")
def probe():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(LIB)
    lib.fp8_probe_encode.argtypes = [ctypes.c_void_p, ctypes.c_float, ctypes.c_int,
                                     ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    lib.fp8_probe_decode.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                     ctypes.c_void_p]
    return lib


def _pad4(a: np.ndarray) -> np.ndarray:
    return np.concatenate((a, np.zeros((-a.size) % 4, a.dtype)))


def _encode(probe, gpu, y: np.ndarray, scale: float, quantize: bool) -> np.ndarray:
    y = _pad4(np.asarray(y, np.float32))
    yd = torch.from_numpy(y).to(gpu)
    out = torch.empty(y.size // 4, dtype=torch.int32, device=gpu)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    assert probe.fp8_probe_encode(yd.data_ptr(), scale, int(quantize), out.data_ptr(), y.size,
                                  ctypes.c_void_p(stream)) == 0
    torch.cuda.synchronize(gpu)
    return out.cpu().numpy().view(np.uint8)


def _interesting_values() -> np.ndarray:
    pos = orc.E4M3_TABLE[:127].astype(np.float32)  # 0 .. 448, increasing
    mid = ((pos[:-1].astype(np.float64) + pos[1:]) / 2).astype(np.float32)  # exact in fp32
    near = np.concatenate((np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(1e9))))
    big = np.array([448.0, 448.5, 464.0, 479.9, 480.0, 500.0, 1e6, 3e38, np.inf],
                   np.float32)
    tiny = np.array([0.0, 2.0**-10, 2.0**-11, 2.0**-9 * 1.5, 1e-30, 1e-45], np.float32)
    v = np.concatenate((pos, mid, near, big, tiny))
    return np.concatenate((v, -v, np.array([np.nan, -np.nan], np.float32)))


def test_encode_every_midpoint_and_special_value(probe, gpu):
    print("case fp8 encode: midpoints, neighbours, clamp, specials", flush=True)
    v = _interesting_values()
    got = _encode(probe, gpu, v, 1.0, False)[: v.size]
    want = orc.e4m3_encode(np.clip(v, -orc.E4M3_MAX, orc.E4M3_MAX))
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(float(v[i]), hex(got[i]), hex(want[i])) for i in bad[:8]]


def test_decode_every_code(probe, gpu):
    print("case fp8 decode: all 256 codes", flush=True)
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).to(gpu)
    out = torch.empty(256, dtype=torch.float32, device=gpu)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    assert probe.fp8_probe_decode(codes.data_ptr(), out.data_ptr(), 256,
                                  ctypes.c_void_p(stream)) == 0
    torch.cuda.synchronize(gpu)
    got = out.cpu().numpy()
    want = orc.E4M3_TABLE
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


# workload-like scales, an exact reciprocal (0.125), RN(1/s) above 1/s (3.0), and both
# ends of the range the division is correctly rounded over (2^-90 .. 2^100)
@pytest.mark.parametrize("scale", [0.01, 0.037, 0.081, 0.1, 0.125, 3.0, 2.0 ** -90,
                                   1.7 * 2.0 ** -60, 1.9 * 2.0 ** 99])
def test_requantise_lands_exactly_on_and_around_midpoints(probe, gpu, scale):
    """y chosen so that y / scale sits on, or one fp32 step from, every midpoint: the
    division and the encoder together must give the correctly rounded code."""
    print(f"case fp8 requantise scale={scale}", flush=True)
    s = np.float32(scale)
    target = _interesting_values()
    target = target[np.isfinite(target)]
    with np.errstate(over="ignore"):
        y = (target.astype(np.float64) * np.float64(s)).astype(np.float32)
    # a shift's y is at most 2 * 448 * s in magnitude, never infinite: the quotient is
    # defined for finite y only
    y = y[np.isfinite(y)]
    y = np.concatenate((y, np.nextafter(y, np.float32(-1e9)), np.nextafter(y, np.float32(1e9)),
                        np.random.default_rng(1).standard_normal(20000).astype(np.float32) * 20,
                        np.array([np.nan, 0.0, -0.0], np.float32)))
    got = _encode(probe, gpu, y, float(s), True)[: y.size]
    with np.errstate(invalid="ignore", over="ignore"):
        q = np.clip(y / s, -orc.E4M3_MAX, orc.E4M3_MAX).astype(np.float32)
    want = orc.e4m3_encode(q)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(float(y[i]), hex(got[i]), hex(want[i])) for i in bad[:8]]
    assert got[y.size - 1] == 0x80 and got[y.size - 2] == 0x00  # -0 / s = -0
