"""Pins the CPU oracle (oracle/kvshift_oracle.py) before anything is checked against it.

Every oracle function is held to something it does not itself compute: the reference's
own test identities and known answers (tests/test_shift_kernels.py, tests/test_kvshift.py,
tests/test_shift_store.py), torch's library casts and fp32 cos/sin, float64 closed
forms, invariants of the rotation, and brute force on tiny inputs.  A planted mistake
(wrong sign, wrong partner, dropped term) must fail at least one of them; the last
tests plant such mistakes and check that they do.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kvshift_oracle as orc
from oracle import torch_path

DELTAS = [-3000, -4, 0, 4, 186, 10000]
# int32 extremes and deltas whose fp32 conversion rounds (beyond 2^24)
EXTREME_DELTAS = [131071, -1048577, 16777219, -33554435, 2**31 - 1, -(2**31)]


def _inv(rotary=128, theta=1e6):
    return orc.inv_freq(rotary, theta)


# ------------------------------------------------------------------ frequencies


@pytest.mark.parametrize("rotary,theta", [(128, 1e6), (64, 1e4), (8, 1e4), (256, 5e5)])
def test_inv_freq_matches_the_closed_form(rotary, theta):
    inv = _inv(rotary, theta)
    exact = 1.0 / theta ** (np.arange(0, rotary, 2, dtype=np.float64) / rotary)
    ulp = np.spacing(np.abs(inv).astype(np.float32)).astype(np.float64)
    assert inv.dtype == np.float32 and inv.shape == (rotary // 2,)
    assert np.all(np.abs(inv.astype(np.float64) - exact) <= 2 * ulp)


def test_angles_are_one_fp32_rounding_of_the_exact_product():
    inv = _inv()
    for delta in DELTAS + [1, -1, 2048, -4096, 12345]:
        got = orc.angles(delta, inv)
        exact = np.float64(delta) * inv.astype(np.float64)  # exact: 24-bit x <=24-bit int
        assert np.array_equal(got, exact.astype(np.float32)), delta
    # beyond 2^24 the delta itself is first rounded to fp32, as torch rounds the Python
    # scalar of ``float(delta) * inv_freq`` to the tensor's fp32 (shift_kernels.py:73)
    for delta in EXTREME_DELTAS:
        d32 = np.float64(np.float32(delta))
        assert d32 == float(torch.tensor(float(delta), dtype=torch.float32))
        got = orc.angles(delta, inv)
        assert np.array_equal(got, (d32 * inv.astype(np.float64)).astype(np.float32)), delta
        want = (float(delta) * torch.from_numpy(inv)).numpy()
        assert np.array_equal(got, want), delta


@pytest.mark.parametrize("delta", DELTAS + [-566, 6759, -2048] + EXTREME_DELTAS)
def test_cos_sin_are_correctly_rounded_and_agree_with_torch(delta):
    inv = _inv()
    c, s = orc.cos_sin(delta, inv, "cr")
    a64 = orc.angles(delta, inv).astype(np.float64)
    # independent float64 evaluation (torch's CPU libm) rounds to the same fp32 values
    tc = torch.from_numpy(a64).cos().numpy().astype(np.float32)
    ts = torch.from_numpy(a64).sin().numpy().astype(np.float32)
    assert np.array_equal(c, tc) and np.array_equal(s, ts)
    # torch's fp32 routines (what the reference's rope_shift uses) are within 1 ulp
    c2, s2 = orc.cos_sin(delta, inv, "torch")
    assert np.all(np.abs(c2 - c) <= np.spacing(np.abs(c))) and np.all(
        np.abs(s2 - s) <= np.spacing(np.abs(s)) + np.float32(1e-45)
    )
    assert np.allclose(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2, 1.0, atol=4e-7)


# --------------------------------------------------------------------- codecs


def _tie_heavy_floats(n=200_000, seed=0):
    rng = np.random.default_rng(seed)
    u = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    ties = (u & np.uint32(0xFFFF0000)) | np.uint32(0x8000)  # exact bf16 ties
    near = ties + np.uint32(1)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 3.4e38, -3.4e38,
                         1.17549435e-38, 65504.0, 65520.0, 6.1e-5, 5.96e-8], np.float32)
    return np.concatenate([u.view(np.float32), ties.view(np.float32), near.view(np.float32),
                           specials])


def test_bf16_rounding_matches_torch():
    x = _tie_heavy_floats()
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = orc.f32_to_bf16(x)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    # NaN payloads are implementation-defined (torch's vectorized CPU cast keeps payload
    # bits, c10's scalar cast returns 0x7FC0); the kernels canonicalise every NaN
    assert np.all(got[nan] == 0x7FC0)
    assert np.all((want[nan] & 0x7F80) == 0x7F80) and np.all(want[nan] & 0x007F)
    # and upcasting is exact
    assert np.array_equal(orc.bf16_to_f32(got[~nan]).view(np.uint32), got[~nan].astype(np.uint32) << 16)


def test_fp16_rounding_matches_torch():
    x = _tie_heavy_floats(seed=1)
    want = torch.from_numpy(x).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    got = orc.f32_to_f16(x)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all(got[nan] == 0x7E00)


def test_e4m3_decode_table_matches_torch_for_all_codes():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    want = codes.view(torch.float8_e4m3fn).to(torch.float32).numpy()
    got = orc.E4M3_TABLE
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert nan.sum() == 2 and got[0x7E] == 448.0 and got[0x01] == 2.0**-9


def test_e4m3_encode_matches_torch_in_range():
    pos = np.unique(np.abs(orc.E4M3_TABLE[np.isfinite(orc.E4M3_TABLE)])).astype(np.float64)
    mids = (pos[1:] + pos[:-1]) / 2
    rng = np.random.default_rng(2)
    x = np.concatenate([pos, -pos, mids, -mids, np.nextafter(mids, 0), np.nextafter(mids, 1e9),
                        rng.uniform(-448, 448, 100_000), rng.uniform(-0.01, 0.01, 100_000),
                        [0.0, -0.0]]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(orc.e4m3_encode(x), want)
    assert orc.e4m3_encode(np.array([np.nan, -np.nan], np.float32)).tolist() == [0x7F, 0x7F]
    # clamp behaviour the kernels rely on: 448 is representable and is the maximum
    assert orc.e4m3_encode(np.array([448.0, -448.0], np.float32)).tolist() == [0x7E, 0xFE]


# ------------------------------------------------------------------- rotation


def test_tables_match_rerotate_keys():
    """tests/test_shift_kernels.py:32-43, restated: both table forms equal rerotate_keys."""
    inv = _inv()
    k = np.random.default_rng(3).standard_normal((2, 8, 5, 128)).astype(np.float32)
    for delta in DELTAS:
        t = orc.rope_tables(delta, 128, inv)
        want = orc.rerotate_keys(k, delta, inv)
        got = k * t["emb_cos"] + np.concatenate((-k[..., 64:], k[..., :64]), -1) * t["emb_sin"]
        assert np.allclose(got, want, atol=1e-6), delta
        fused = k * t["cos"] + k[..., t["partner"].astype(np.int64)] * t["sgn"]
        assert np.allclose(fused, want, atol=1e-6), delta


@pytest.mark.parametrize("head_dim,theta", [(8, 1e4), (128, 1e6)])
@pytest.mark.parametrize("delta", [-7, -1, 0, 1, 13, 64])
def test_rerotate_matches_fresh_rope_at_the_shifted_position(head_dim, theta, delta):
    """tests/test_kvshift.py:48-55 restated against a float64 RoPE."""
    inv = orc.inv_freq(head_dim, theta)
    k = np.random.default_rng(0).standard_normal((1, 2, 11, head_dim))
    pos = np.arange(100, 111)
    at_p = orc.rope_f64(k, pos, inv).astype(np.float32)
    shifted = orc.rerotate_keys(at_p, delta, inv)
    fresh = orc.rope_f64(k, pos + delta, inv)
    assert np.allclose(shifted, fresh, atol=1e-5, rtol=1e-4)


def test_rerotation_is_invertible_composes_and_preserves_pair_norms():
    inv = _inv()
    k = np.random.default_rng(4).standard_normal((3, 8, 128)).astype(np.float32)
    back = orc.rerotate_keys(orc.rerotate_keys(k, 9, inv), -9, inv)
    assert np.allclose(back, k, atol=1e-5)
    two = orc.rerotate_keys(orc.rerotate_keys(k, 300, inv), -77, inv)
    assert np.allclose(two, orc.rerotate_keys(k, 223, inv), atol=1e-4)
    r = orc.rerotate_keys(k, 1234, inv)
    n0 = np.hypot(k[..., :64], k[..., 64:])
    n1 = np.hypot(r[..., :64], r[..., 64:])
    assert np.allclose(n0, n1, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("delta", DELTAS + [-566] + EXTREME_DELTAS)
def test_bf16_rotation_is_the_reference_op_sequence(delta):
    """With torch's own CPU tables, the oracle's bit-level rotation equals the reference
    torch path's bytes exactly (same fp32 ops, same rounding)."""
    g = torch.Generator().manual_seed(11)
    rows = torch.randn(40, 8, 256, generator=g).to(torch.bfloat16)
    kv = torch.zeros(4, 8, 16, 256, dtype=torch.bfloat16)
    slot = torch.randperm(64, generator=g)[:40]
    inv = torch.from_numpy(_inv())
    emb = torch_path.rope_emb_tables(delta, inv) if delta else None
    torch_path.shift_into_paged(rows, kv, slot, 16, True, emb)
    want = kv.view(torch.int16).numpy().view(np.uint16)
    got = np.zeros_like(want)
    src_bits = rows.view(torch.int16).numpy().view(np.uint16)
    orc.scatter_shifted(src_bits, got, slot.numpy(), 16, True, delta, inv.numpy(), "bf16",
                        method="torch")
    assert np.array_equal(got, want)


@pytest.mark.parametrize("rotary", [128, 64, 32])
@pytest.mark.parametrize("delta", [-3000, -566, 4, 186, 10000])
def test_triton_arithmetic_restatement_is_the_rotate_half_rotation(rotary, delta):
    """``torch_path.triton_rows_into_paged`` (the Triton kernel's ``k*cos + k[partner]*sgn``
    through the ``[head_size]`` tables) equals the oracle's ``cat``-based rotate-half
    (kvshift.py:44-46) with the same torch tables, bit for bit, at full and partial
    rotary; at full rotary it also equals the torch path.  A wrong partner table fails."""
    g = torch.Generator().manual_seed(rotary + delta % 101)
    rows = torch.randn(40, 8, 256, generator=g).to(torch.bfloat16)
    slot = torch.randperm(64, generator=g)[:40]
    inv = torch.from_numpy(_inv(rotary))
    t = torch_path.rope_shift_tables(delta, 128, inv, "cpu")
    kv = torch.zeros(4, 8, 16, 256, dtype=torch.bfloat16)
    torch_path.triton_rows_into_paged(rows, kv, slot, 16, True, (t["cos"], t["sgn"], t["partner"]))
    got = kv.view(torch.int16).numpy().view(np.uint16)
    want = np.zeros_like(got)
    orc.scatter_shifted(rows.view(torch.int16).numpy().view(np.uint16), want, slot.numpy(), 16,
                        True, delta, inv.numpy(), "bf16", method="torch")
    assert np.array_equal(got, want)
    if rotary == 128:
        ref = torch.zeros_like(kv)
        torch_path.shift_into_paged(rows, ref, slot, 16, True, (t["emb_cos"], t["emb_sin"]))
        assert torch.equal(ref.view(torch.int16), kv.view(torch.int16))
    wrong = torch.arange(128, dtype=torch.int32)  # identity partner: no rotate-half
    bad = torch.zeros_like(kv)
    torch_path.triton_rows_into_paged(rows, bad, slot, 16, True, (t["cos"], t["sgn"], wrong))
    assert not np.array_equal(bad.view(torch.int16).numpy().view(np.uint16), want)


@pytest.mark.parametrize("hnd", [True, False])
@pytest.mark.parametrize("delta", [0, 1, -1, 17, -17, 566, -566, -1133, 6759])
def test_scatter_lands_what_rerotate_keys_says_qwen3_geometry(delta, hnd):
    """tests/test_shift_kernels.py:93-134, on the oracle's fp32 scatter."""
    rng = np.random.default_rng(2 * abs(delta) + (delta < 0))
    heads, hs, bs, blocks, n = 8, 128, 16, 12, 40
    inv = _inv()
    src = rng.standard_normal((n, heads, 2 * hs)).astype(np.float32)
    shape = (blocks, heads, bs, 2 * hs) if hnd else (blocks, bs, heads, 2 * hs)
    kv = np.zeros(shape, np.uint32)
    slot = rng.permutation(blocks * bs)[:n]
    orc.scatter_shifted(src.view(np.uint32), kv, slot, bs, hnd, delta, inv, "f32")
    want = np.concatenate((orc.rerotate_keys(src[..., :hs], delta, inv), src[..., hs:]), -1)
    blk, off = slot // bs, slot % bs
    got = (kv[blk, :, off] if hnd else kv[blk, off]).view(np.float32)
    assert np.allclose(got, want, atol=1e-4)


def test_the_scatter_check_catches_a_wrong_angle():
    """tests/test_shift_kernels.py:137-155: delta 100 must not pass for 101."""
    rng = np.random.default_rng(5)
    inv = _inv()
    src = rng.standard_normal((40, 8, 256)).astype(np.float32)
    kv = np.zeros((12, 8, 16, 256), np.uint32)
    slot = np.arange(40)
    orc.scatter_shifted(src.view(np.uint32), kv, slot, 16, True, 100, inv, "f32")
    want = np.concatenate((orc.rerotate_keys(src[..., :128], 101, inv), src[..., 128:]), -1)
    got = kv[slot // 16, :, slot % 16].view(np.float32)
    assert not np.allclose(got, want, atol=1e-4)


def test_delta_zero_and_partial_rotary_tail_are_bit_copies():
    rng = np.random.default_rng(6)
    k = rng.integers(0, 2**16, (5, 8, 128), dtype=np.uint16)
    assert np.array_equal(orc.rotate_k_bits(k, 0, _inv(), "bf16"), k)
    part = orc.rotate_k_bits(k, 33, _inv(64), "bf16")  # rotary 64 of 128
    assert np.array_equal(part[..., 64:], k[..., 64:])
    assert not np.array_equal(part[..., :64], k[..., :64])


def test_fp8_rotation_closed_form_with_power_of_two_scale():
    """With scale 2^-4 the dequant and requant scalings are exact, so the fp8 rule
    reduces to encode(clamp(rotate(decode(k))))."""
    rng = np.random.default_rng(7)
    k = rng.integers(0, 256, (6, 8, 128), dtype=np.uint8)
    k[(k & 0x7F) == 0x7F] = 0  # no NaN codes here
    inv = _inv()
    got = orc.rotate_k_bits(k, -777, inv, "fp8", k_scale=np.float32(0.0625))
    ec, es = orc.emb_tables(-777, inv)
    y = orc.rotate_f32(orc.e4m3_decode(k), ec, es)
    want = orc.e4m3_encode(np.clip(y, -448, 448).astype(np.float32))
    assert np.array_equal(got, want)


def test_fp8_requant_error_is_within_half_an_fp8_step():
    rng = np.random.default_rng(8)
    k = rng.integers(0, 256, (6, 8, 128), dtype=np.uint8)
    k[(k & 0x7F) == 0x7F] = 0
    inv = _inv()
    s = np.float32(0.037)
    got = orc.e4m3_decode(orc.rotate_k_bits(k, 1234, inv, "fp8", k_scale=s)).astype(np.float64)
    x = orc.e4m3_decode(k).astype(np.float64) * float(s)
    a = orc.angles(1234, inv).astype(np.float64)
    c, sn = np.cos(np.concatenate((a, a))), np.sin(np.concatenate((a, a)))
    rot = np.concatenate((-x[..., 64:], x[..., :64]), -1)
    exact = np.clip((x * c + rot * sn) / float(s), -448, 448)
    pos = np.unique(np.abs(orc.E4M3_TABLE[np.isfinite(orc.E4M3_TABLE)]))
    step = np.diff(pos)[np.clip(np.searchsorted(pos, np.abs(exact)) - 1, 0, len(pos) - 2)]
    assert np.all(np.abs(got - exact) <= step / 2 + 1e-5 * np.abs(exact) + 1e-9)


# ----------------------------------------------------------------- slots, paging


def test_slots_known_answer():
    """tests/test_shift_store.py:24-27."""
    assert orc.slots([7, 3], 2, 6, 4).tolist() == [7 * 4 + 2, 7 * 4 + 3, 3 * 4 + 0, 3 * 4 + 1]


def test_slots_brute_force():
    rng = np.random.default_rng(9)
    for bs in (1, 4, 16, 24):
        table = rng.permutation(50)
        lo, hi = 5, 5 + 300 // bs * 3
        hi = min(hi, 50 * bs)
        want = []
        for p in range(lo, hi):
            want.append(int(table[p // bs]) * bs + p % bs)
        assert orc.slots(table, lo, hi, bs).tolist() == want


def test_paged_layouts_brute_force():
    """HND puts row (blk, head, off) at kv[blk, head, off]; NHD at kv[blk, off, head]."""
    rng = np.random.default_rng(10)
    rows = rng.integers(0, 2**16, (7, 4, 8), dtype=np.uint16)
    slot = np.array([0, 5, 17, 33, 71, 96, 111])
    for hnd in (True, False):
        kv = np.zeros((7, 4, 16, 8) if hnd else (7, 16, 4, 8), np.uint16)
        kv[orc.paged_rows(kv, slot, 16, "hnd" if hnd else "nhd")] = rows
        for i, s in enumerate(slot):
            for h in range(4):
                cell = kv[s // 16, h, s % 16] if hnd else kv[s // 16, s % 16, h]
                assert np.array_equal(cell, rows[i, h])


def test_shift_spans_equals_per_span_scatters():
    rng = np.random.default_rng(12)
    inv = _inv()
    layers, heads = 2, 4
    src_caches = [[rng.integers(0, 2**16, (20, 16, heads, 256), dtype=np.uint16)
                   for _ in range(layers)]]
    dst_a = [np.zeros((30, heads, 16, 256), np.uint16) for _ in range(layers)]
    dst_b = [x.copy() for x in dst_a]
    src_tab = rng.permutation(20)
    dst_slots = rng.permutation(30 * 16)[:100]
    spans = [orc.Span(5, 0, 60, -31, 0, 0), orc.Span(200, 0, 40, 0, 0, 60)]
    orc.shift_spans(spans, orc.Side(src_caches, "nhd", 16, "table", src_tab),
                    orc.Side([dst_a], "hnd", 16, "slots", dst_slots), inv, "bf16")
    for sp in spans:
        s_slot = orc.slots(src_tab, sp.src_pos, sp.src_pos + sp.n_tokens, 16)
        for layer in range(layers):
            rows = src_caches[0][layer][s_slot // 16, s_slot % 16]
            orc.scatter_shifted(rows, dst_b[layer], dst_slots[sp.dst_index:sp.dst_index + sp.n_tokens],
                                16, True, sp.delta, inv, "bf16")
    for a, b in zip(dst_a, dst_b):
        assert np.array_equal(a, b)


# --------------------------------------------- planted mistakes must be caught


def test_planted_mistakes_fail_the_checks(monkeypatch):
    """A wrong sign or a wrong partner in the oracle's rotation fails the fresh-RoPE
    identity that pins it."""
    inv = orc.inv_freq(8, 1e4)
    k = np.random.default_rng(0).standard_normal((1, 2, 11, 8))
    pos = np.arange(100, 111)
    at_p = orc.rope_f64(k, pos, inv).astype(np.float32)
    fresh = orc.rope_f64(k, pos + 13, inv)

    def wrong_sign(kf, ec, es):
        kf = np.asarray(kf, np.float32)
        h = kf.shape[-1] // 2
        rot = np.concatenate((kf[..., h:], kf[..., :h]), axis=-1)  # sign dropped
        return kf * ec + rot * es

    def wrong_partner(kf, ec, es):
        kf = np.asarray(kf, np.float32)
        rot = np.concatenate((-kf[..., 1:], kf[..., :1]), axis=-1)  # neighbour, not i+h
        return kf * ec + rot * es

    for bad in (wrong_sign, wrong_partner):
        monkeypatch.setattr(orc, "rotate_f32", bad)
        assert not np.allclose(orc.rerotate_keys(at_p, 13, inv), fresh, atol=1e-5, rtol=1e-4)
