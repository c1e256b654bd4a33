"""Full-size shifts (the benchmark configurations) checked through size-independent
properties, on the GPU:

* V is bit-exact for every row of every layer (gathers on the device, compared whole);
* sampled K rows are bit-exact against the oracle;
* destination slots outside every span are untouched;
* shifting by delta and back by -delta returns K within the bf16 double-rounding bound;
* K of keys RoPE'd at position p, shifted by delta, is within 2e-2 (max-abs, where
  |k| < 4) of the same keys RoPE'd fresh at p + delta.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from marathon_amd import workloads as W
from marathon_amd.spans import CacheSet, ShiftPlan, span_array
from oracle import kvshift_oracle as orc
from tests.helpers import bits

pytestmark = pytest.mark.gpu

D = 128


def _src_rows(wl, g, layer, sp):
    """[n, heads, 2D] source rows of span ``sp`` (store block layout, NHD)."""
    cache = wl.src.caches[g][layer]
    pos = torch.arange(int(sp["src_pos"]), int(sp["src_pos"]) + int(sp["n_tokens"]),
                       device=cache.device)
    tab = wl.src_index.to(cache.device, torch.int64)[int(sp["src_index"]):]
    blk = tab[pos // 16]
    return cache[blk, pos % 16]


def _dst_slots(wl, sp):
    n = int(sp["n_tokens"])
    if wl.dst_mode == "slots":
        return wl.dst_index[int(sp["dst_index"]):int(sp["dst_index"]) + n].to(torch.int64)
    pos = torch.arange(int(sp["dst_pos"]), int(sp["dst_pos"]) + n)
    tab = wl.dst_index.to(torch.int64)[int(sp["dst_index"]):]
    return tab[pos // 16] * 16 + pos % 16


def _dst_rows(wl, layer, slot):
    cache = wl.dst.caches[0][layer]
    slot = slot.to(cache.device)
    return cache[slot // 16, :, slot % 16]  # HND


def _check_full(wl, dtype_name, samples=192, seed=0, snapshot=True):
    """snapshot=False: the destination started all-zero (saves a copy of a large cache)."""
    dev = wl.dst.first.device
    snapshot = [c.clone() for c in wl.dst.caches[0]] if snapshot else None
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    wl.plan().launch(error_flags=flags)
    torch.cuda.synchronize(dev)
    assert int(flags.item()) == 0
    spans = wl.spans
    written = [torch.zeros(c.shape[0] * 16, dtype=torch.bool, device=dev) for c in wl.dst.caches[0]]
    for sp in spans:
        g = int(sp["src_group"])
        slot = _dst_slots(wl, sp)
        for layer in range(wl.layers):
            src = _src_rows(wl, g, layer, sp)
            got = _dst_rows(wl, layer, slot)
            assert torch.equal(got[..., D:].contiguous().view(torch.uint8),
                               src[..., D:].contiguous().view(torch.uint8)), (
                f"V differs: span {sp} layer {layer}")
            if int(sp["delta"]) == 0:
                assert torch.equal(got.contiguous().view(torch.uint8),
                                   src.contiguous().view(torch.uint8))
            written[layer][slot.to(dev)] = True
    # untouched slots keep their bytes
    for layer, c in enumerate(wl.dst.caches[0]):
        keep = ~written[layer].view(-1, 16)  # [blocks, 16]
        a = c.permute(0, 2, 1, 3)[keep].contiguous().view(torch.uint8)  # rows [m, heads, 2D]
        if snapshot is None:
            assert not bool(a.any())
        else:
            b = snapshot[layer].permute(0, 2, 1, 3)[keep].contiguous().view(torch.uint8)
            assert torch.equal(a, b)
    del snapshot
    # sampled K rows against the oracle
    rng = np.random.default_rng(seed)
    inv = wl.inv_freq.numpy()
    for _ in range(samples):
        sp = spans[int(rng.integers(len(spans)))]
        i = int(rng.integers(int(sp["n_tokens"])))
        layer = int(rng.integers(wl.layers))
        one = sp.copy()
        one["src_pos"] = int(sp["src_pos"]) + i
        one["dst_pos"] = int(sp["dst_pos"]) + i
        one["n_tokens"] = 1
        if wl.dst_mode == "slots":
            one["dst_index"] = int(sp["dst_index"]) + i
        src = bits(_src_rows(wl, int(sp["src_group"]), layer, one))
        got = bits(_dst_rows(wl, layer, _dst_slots(wl, one)))
        scale = None if wl.k_scale is None else np.float32(wl.k_scale[layer])
        want = orc.rotate_k_bits(src[..., :D], int(sp["delta"]), inv, dtype_name, scale)
        assert np.array_equal(got[..., :D], want), f"K differs: span {sp} token {i} layer {layer}"


def test_qwen3_8b_single_span_full_size(gpu):
    print("case Qwen3-8B single span full size (36 layers, 15,872 tokens)", flush=True)
    wl = W.qwen3_8b_single_span(gpu, dst_fill="random")
    _check_full(wl, "bf16")
    del wl
    torch.cuda.empty_cache()


def test_qwen3_14b_multispan_full_size(gpu):
    print("case Qwen3-14B multi-span full size (40 layers, 8 spans)", flush=True)
    wl = W.qwen3_14b_multispan(gpu, dst_fill="random")
    assert wl.tokens > 20000 and len(wl.spans) == 8
    _check_full(wl, "bf16")
    del wl
    torch.cuda.empty_cache()


def test_qwen3_14b_multispan_fp8_full_size(gpu):
    print("case Qwen3-14B multi-span fp8 full size", flush=True)
    wl = W.qwen3_14b_multispan_fp8(gpu)
    _check_full(wl, "fp8")
    del wl
    torch.cuda.empty_cache()


def test_batched_sessions_full_size(gpu):
    print("case batched sessions full size (32 sessions x 36 layers)", flush=True)
    wl = W.batched_sessions(gpu)
    assert wl.src.groups == 32 and len(wl.spans) > 32
    _check_full(wl, "bf16", samples=128, snapshot=False)
    del wl
    torch.cuda.empty_cache()


def test_round_trip_at_full_size(gpu):
    """Shift by delta, then back by -delta: K returns within the double-rounding bound,
    V exactly."""
    print("case round trip (Qwen3-14B multi-span layout, 40 layers)", flush=True)
    wl = W.qwen3_14b_multispan(gpu)
    wl.plan().launch()
    back = [torch.zeros_like(c) for c in wl.src.caches[0]]
    # the way back: read the destination cache through the same slots, write a fresh
    # store in block layout through the source block table, rotate by -delta
    rows = [(0, int(sp["src_pos"]), int(sp["dst_index"]), int(sp["src_index"]),
             int(sp["n_tokens"]), -int(sp["delta"]), 0, 0) for sp in wl.spans]
    plan = ShiftPlan(span_array(rows), CacheSet([wl.dst.caches[0]], "hnd", 16),
                     CacheSet([back], "nhd", 16), inv_freq=wl.inv_freq, src_mode="slots",
                     src_index=wl.dst_index, dst_mode="table", dst_index=wl.src_index)
    plan.launch()
    torch.cuda.synchronize(gpu)
    tab = wl.src_index.to(gpu, torch.int64)
    for sp in wl.spans:
        pos = torch.arange(int(sp["src_pos"]), int(sp["src_pos"]) + int(sp["n_tokens"]),
                           device=gpu)
        for layer in range(0, wl.layers, 7):
            orig = _src_rows(wl, 0, layer, sp).float()
            got = back[layer][tab[pos // 16], pos % 16].float()
            assert torch.equal(got[..., D:], orig[..., D:])
            k0 = orig[..., :D]
            pair = torch.maximum(k0.abs(), torch.roll(k0, D // 2, -1).abs())
            bound = 2.0**-8 * (3 * pair + got[..., :D].abs()) + 1e-6
            assert bool(((got[..., :D] - k0).abs() <= bound).all()), f"span {sp} layer {layer}"
    del wl, back, plan
    torch.cuda.empty_cache()


def test_fresh_rope_bar(gpu):
    """Keys RoPE'd at p (bf16), shifted by delta, against the same keys RoPE'd at p + delta
    in float64: max-abs <= 2e-2 where |k| < 4, and the double-rounding bound elsewhere."""
    print("case fresh RoPE (8 spans, 2 layers)", flush=True)
    lay = W.qwen3_14b_multispan_layout()
    inv = W.inv_freq_for(D, 1e6)
    heads = 8
    g = torch.Generator(device=gpu)
    g.manual_seed(123)
    raw = torch.randn(lay.src_history, heads, D, dtype=torch.float64, device=gpu, generator=g)
    inv64 = inv.to(gpu, torch.float64)

    def rope(x, pos):
        ang = pos.to(torch.float64)[:, None] * inv64[None, :]
        emb = torch.cat((ang, ang), -1)[:, None, :]
        rot = torch.cat((-x[..., D // 2:], x[..., : D // 2]), -1)
        return x * emb.cos() + rot * emb.sin()

    pos_all = torch.arange(lay.src_history, device=gpu)
    k_old = rope(raw, pos_all).to(torch.bfloat16)
    v = torch.randn(lay.src_history, heads, D, device=gpu, generator=g).to(torch.bfloat16)
    store = torch.cat((k_old, v), -1).contiguous()  # flat store [hist, heads, 2D]
    blocks = -(-lay.dst_history // 16) + 4
    kv = torch.zeros(blocks, heads, 16, 2 * D, dtype=torch.bfloat16, device=gpu)
    rows, slot_parts, off = [], [], 0
    for s, d, n, dl in zip(lay.src_start, lay.dst_start, lay.length, lay.delta):
        rows.append((int(s), 0, 0, off, int(n), int(dl), 0, 0))
        slot_parts.append(torch.arange(int(d), int(d) + int(n)))
        off += int(n)
    slots = torch.cat(slot_parts)
    plan = ShiftPlan(span_array(rows), CacheSet([[store]], "flat"), CacheSet([[kv]], "hnd", 16),
                     inv_freq=inv, src_mode="flat", dst_mode="slots", dst_index=slots)
    plan.launch()
    torch.cuda.synchronize(gpu)
    worst_small = 0.0
    for s, d, n, dl in zip(lay.src_start, lay.dst_start, lay.length, lay.delta):
        src_pos = torch.arange(int(s), int(s) + int(n), device=gpu)
        fresh = rope(raw[src_pos], src_pos + int(dl))
        sl = torch.arange(int(d), int(d) + int(n), device=gpu)
        got = kv[sl // 16, :, sl % 16][..., :D].to(torch.float64)
        kin = k_old[src_pos].to(torch.float64)
        err = (got - fresh).abs()
        pair = torch.maximum(kin.abs(), torch.roll(kin, D // 2, -1).abs())
        small = (pair < 4) & (fresh.abs() < 4)
        worst_small = max(worst_small, float(err[small].max()))
        bound = 2.0**-8 * (2 * pair + fresh.abs()) + 1e-6
        assert bool((err <= bound).all())
    assert worst_small <= 2e-2, worst_small
