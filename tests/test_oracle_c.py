"""Pins the oracle's C restatement (oracle/rotate_c.c, via oracle/fast_rotate.py) to the
numpy oracle, bit for bit: every fp8 code, the fp8 midpoints and their neighbours, a
strided walk over every fp32 magnitude up to 448, tie-heavy bf16/fp16 roundings, and
random rows of every element type at several deltas and rotary widths.  The numpy
oracle is itself pinned in tests/test_oracle.py; the full-size GPU tests use the C one."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import fast_rotate as fast
from oracle import kvshift_oracle as orc

DELTAS = [-3000, -4, 4, 186, 10000, 2**31 - 1, -(2**31)]


def _vec(fn, xs, out_dtype):
    return np.array([fn(x) for x in xs.tolist()], dtype=out_dtype)


def test_fp8_decode_matches_on_every_code():
    L = fast.lib()
    got = np.array([L.orc_e4m3_dec(c) for c in range(256)], np.float32)
    want = orc.E4M3_TABLE
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))  # signed zeros too


def _fp8_encode_inputs():
    pos = orc.E4M3_TABLE[:127].astype(np.float64)
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)  # exact in fp32
    near = np.concatenate([np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9)),
                           mids, pos.astype(np.float32)])
    walk = np.arange(0, np.float32(448.0).view(np.uint32) + 1, 997, dtype=np.uint32).view(np.float32)
    tiny = np.float32([0.0, 2.0**-10, 2.0**-11, 3 * 2.0**-11, 2.0**-9 * 0.75, 1e-30, 448.0])
    a = np.concatenate([near, walk, tiny]).astype(np.float32)
    a = a[(a >= 0) & (a <= 448)]
    return np.concatenate([a, -a])


def test_fp8_encode_matches_on_midpoints_and_a_walk_over_the_range():
    L = fast.lib()
    xs = _fp8_encode_inputs()
    got = _vec(L.orc_e4m3_enc_clamped, xs, np.uint8)
    want = orc.e4m3_encode(xs)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (xs[bad[:5]], got[bad[:5]], want[bad[:5]])


def _tie_heavy(n=60_000, seed=0):
    rng = np.random.default_rng(seed)
    u = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    ties = (u & np.uint32(0xFFFF0000)) | np.uint32(0x8000)
    ties16 = (u & np.uint32(0xFFFFE000)) | np.uint32(0x1000)
    specials = np.float32([0.0, -0.0, np.inf, -np.inf, 65504, 65519.996, 65520, 6.1e-5,
                           5.96e-8, 2.98e-8, 1e-45, 3.4e38]).view(np.uint32)
    return np.concatenate([u, ties, ties16, specials]).view(np.float32)


def test_bf16_and_fp16_rounding_match():
    L = fast.lib()
    xs = _tie_heavy()
    xs = xs[~np.isnan(xs)]
    assert np.array_equal(_vec(L.orc_bf16_enc, xs, np.uint16), orc.f32_to_bf16(xs))
    assert np.array_equal(_vec(L.orc_f16_enc, xs, np.uint16), orc.f32_to_f16(xs))
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    dec = _vec(L.orc_f16_dec, codes, np.float32)
    want = orc.f16_to_f32(codes)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(dec), nan)
    assert np.array_equal(dec[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _rows(dtype, shape, rng, scale=None):
    if dtype == "bf16":
        return orc.f32_to_bf16(rng.standard_normal(shape).astype(np.float32))
    if dtype == "f16":
        return orc.f32_to_f16(rng.standard_normal(shape).astype(np.float32))
    if dtype == "f32":
        return rng.standard_normal(shape).astype(np.float32).view(np.uint32)
    x = (rng.standard_normal(shape) / scale).clip(-448, 448).astype(np.float32)
    return orc.e4m3_encode(x)


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32", "fp8"])
@pytest.mark.parametrize("rotary,head", [(128, 128), (64, 128), (32, 256)])
def test_rotation_matches_the_numpy_oracle(dtype, rotary, head):
    rng = np.random.default_rng(rotary + head)
    inv = orc.inv_freq(rotary, 1e6) if rotary else np.zeros(0, np.float32)
    for delta in DELTAS:
        scale = np.float32(rng.uniform(0.01, 0.1)) if dtype == "fp8" else None
        k = _rows(dtype, (37, 3, head), rng, scale)
        if dtype == "fp8":
            k.reshape(-1)[::97] = 0x7F  # NaN codes, as K and as partner
            k.reshape(-1)[5::101] = 0x80  # -0
        elif dtype in ("bf16", "f16"):
            k.reshape(-1)[::211] = 0x7FC0 if dtype == "bf16" else 0x7E00
        want = orc.rotate_k_bits(k, delta, inv, dtype, scale)
        got = fast.rotate_k_bits(k, delta, inv, dtype, scale, threads=3)
        bad = np.flatnonzero(got.reshape(-1) != want.reshape(-1))
        assert bad.size == 0, (dtype, delta, bad[:5])


def test_delta_zero_and_rotary_zero_copy_the_row():
    rng = np.random.default_rng(1)
    k = _rows("bf16", (5, 8, 128), rng)
    assert np.array_equal(fast.rotate_k_bits(k, 0, orc.inv_freq(128, 1e6), "bf16"), k)
    assert np.array_equal(fast.rotate_k_bits(k, 9, np.zeros(0, np.float32), "bf16"), k)


def test_torch_tables_through_the_c_oracle_equal_the_torch_path():
    """With the reference's own torch tables (method="torch"), the C restatement equals the
    reference's torch op sequence (oracle/torch_path.py) bit for bit."""
    import torch

    from oracle import torch_path

    rng = np.random.default_rng(2)
    inv = orc.inv_freq(128, 1e6)
    k = _rows("bf16", (64, 8, 128), rng)
    v = _rows("bf16", (64, 8, 128), rng)
    for delta in (-566, 37, 186):
        want = fast.rotate_k_bits(k, delta, inv, "bf16", method="torch")
        rows = torch.from_numpy(np.concatenate((k, v), -1).view(np.int16)).view(torch.bfloat16)
        cache = torch.zeros(64, 1, 1, 256, dtype=torch.bfloat16)  # one token per block
        emb = torch_path.rope_emb_tables(delta, torch.from_numpy(inv))
        torch_path.shift_into_paged(rows, cache.expand(64, 8, 1, 256).contiguous(), torch.arange(64),
                                    1, True, emb)
        out = torch.zeros(64, 8, 1, 256, dtype=torch.bfloat16)
        torch_path.shift_into_paged(rows, out, torch.arange(64), 1, True, emb)
        got = out[:, :, 0, :128].contiguous().view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(got, want), delta
