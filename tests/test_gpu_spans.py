"""Batched shifts on the GPU (one launch over a span table) against the oracle.

Reduced-size versions of the Qwen3-14B multi-span, its fp8 variant and the batched
session workloads, every byte of every destination cache compared with the oracle's
``shift_spans``; and the connector-shaped loader reading straight out of a store.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from marathon_amd import ShiftStore, slots
from marathon_amd import workloads as W
from marathon_amd.connector import Load, ShiftLoader
from marathon_amd.spans import span_array
from oracle import kvshift_oracle as orc
from tests.helpers import bits, dname, inv_freq, oracle_side, oracle_spans, randn

pytestmark = pytest.mark.gpu


def _check_workload(wl, dev, dtype_name="bf16"):
    """Every destination byte against the oracle, through the two-launch path and,
    where eligible, the direct path (each run from the same starting caches)."""
    before = [[t.clone() for t in row] for row in wl.dst.caches]
    src_o = oracle_side(wl.src, wl.src_mode, wl.src_index)
    dst_o = oracle_side(wl.dst, wl.dst_mode, wl.dst_index)
    k_scale = None if wl.k_scale is None else wl.k_scale.numpy()
    orc.shift_spans(oracle_spans(wl.spans), src_o, dst_o, wl.inv_freq.numpy(), dtype_name,
                    k_scale)
    for direct in (False, True):
        plan = wl.plan(direct=direct)
        if direct and not plan.direct:
            continue
        for row, saved in zip(wl.dst.caches, before):
            for t, b in zip(row, saved):
                t.copy_(b)
        flags = torch.zeros(1, dtype=torch.int32, device=dev)
        plan.launch(error_flags=flags)
        torch.cuda.synchronize(dev)
        assert int(flags.item()) == 0, f"direct={plan.direct}"
        for g, row in enumerate(wl.dst.caches):
            for layer, t in enumerate(row):
                got = bits(t)
                want = dst_o.caches[g][layer]
                bad = int((got != want).sum())
                assert bad == 0, (f"direct={plan.direct} group {g} layer {layer}: "
                                  f"{bad} elements differ")


@pytest.mark.parametrize("history,layers", [(2048, 3), (4099, 2)])
def test_multispan_matches_oracle(gpu, history, layers):
    print(f"case multispan history={history} layers={layers}", flush=True)
    wl = W.qwen3_14b_multispan(gpu, layers=layers, history=history, dst_fill="random")
    lay = wl.meta["layout"]
    assert np.any(lay.delta == 0) and np.any(lay.delta > 0) and np.any(lay.delta < 0)
    _check_workload(wl, gpu)


def test_fp8_multispan_matches_oracle(gpu):
    print("case fp8 multispan", flush=True)
    wl = W.qwen3_14b_multispan_fp8(gpu, layers=3, history=2048)
    _check_workload(wl, gpu, "fp8")


def test_batched_sessions_match_oracle(gpu):
    print("case batched sessions", flush=True)
    wl = W.batched_sessions(gpu, layers=2, sessions=6, hist_lo=64, hist_hi=700)
    assert wl.src.groups == 6
    _check_workload(wl, gpu)


def test_nhd_destination_and_flat_source(gpu):
    """The reference's own layout pair: flat store rows -> NHD paged cache via slots."""
    print("case flat->nhd", flush=True)
    g = torch.Generator().manual_seed(9)
    layers, heads, d, bs = 3, 8, 128, 16
    bufs = [[torch.randn(500, heads, 2 * d, generator=g).to(torch.bfloat16).to(gpu)
             for _ in range(layers)] for _ in range(2)]
    kv = [torch.randn(40, bs, heads, 2 * d, generator=g).to(torch.bfloat16).to(gpu)
          for _ in range(layers)]
    from marathon_amd.spans import CacheSet, ShiftPlan, span_array

    table0 = torch.randperm(40, generator=g)
    s0 = slots(table0[:20].tolist(), 3, 3 + 150, bs)
    s1 = slots(table0[20:].tolist(), 0, 100, bs)
    spans = span_array([(17, 0, 0, 0, 150, -14, 0, 0), (230, 0, 0, 150, 100, 0, 1, 0)])
    plan = ShiftPlan(spans, CacheSet(bufs, "flat"), CacheSet([kv], "nhd", bs),
                     inv_freq=inv_freq(), src_mode="flat", dst_mode="slots",
                     dst_index=torch.cat((s0, s1)))
    src_o = oracle_side(plan.src, "flat", None)
    dst_o = oracle_side(plan.dst, "slots", torch.cat((s0, s1)))
    orc.shift_spans(oracle_spans(spans), src_o, dst_o, inv_freq().numpy(), "bf16")
    plan.launch()
    torch.cuda.synchronize(gpu)
    for layer in range(layers):
        assert np.array_equal(bits(kv[layer]), dst_o.caches[0][layer])


def test_connector_loader_end_to_end(gpu):
    """Store writes, then one step with two loads from two sessions, one launch."""
    print("case connector loader", flush=True)
    layers, heads, d, bs = 4, 8, 128, 16
    names = [f"model.layers.{i}.self_attn" for i in range(layers)]
    store = ShiftStore(budget_tokens=8192, device=str(gpu), slab=512)
    g = torch.Generator().manual_seed(21)
    hist = {"a": 600, "b": 333}
    for s, n in hist.items():
        assert store.reserve(s, 0, n)
        for name in names:
            store.write(s, name, 0, torch.randn(n, heads, 2 * d, generator=g)
                        .to(torch.bfloat16).to(gpu))
    kv = {name: torch.zeros(64, heads, bs, 2 * d, dtype=torch.bfloat16, device=gpu)
          for name in names}
    loader = ShiftLoader(store, bs, inv_freq())
    loader.register_kv_caches(kv)
    assert loader.hnd is True
    perm = torch.randperm(64, generator=g).tolist()
    la = Load("a", slots(perm[:32], 160, 160 + 304, bs), src_start=160 + 37, delta=-37)
    lb = Load("b", slots(perm[32:], 32, 32 + 256, bs), src_start=32, delta=0)
    loaded = loader.start_load_kv([la, lb])
    torch.cuda.synchronize(gpu)
    assert loaded == (304 + 256) * layers
    assert store.stats()["loaded_token_layers"] == (304 + 256) * layers
    for name in names:
        want = np.zeros_like(bits(kv[name]))
        for ld in (la, lb):
            src_rows = bits(store.read(ld.session, name, ld.src_start, ld.slots.numel()))
            orc.scatter_shifted(src_rows, want, ld.slots.numpy(), bs, True, ld.delta,
                                inv_freq().numpy(), "bf16")
        assert np.array_equal(bits(kv[name]), want), name


def _two_session_plan(gpu, dtype, heads, d, rotary, seed, spans, table, k_scale=None,
                      fill=None, direct=None):
    """Two flat sessions (300 and 200 rows) -> an HND paged cache addressed through a
    block table; returns (plan, dst caches)."""
    from marathon_amd.spans import CacheSet, ShiftPlan, span_array
    from tests.helpers import randn

    g = torch.Generator().manual_seed(seed)
    layers, bs = 2, 16
    sc = 0.05
    bufs = [[randn((n, heads, 2 * d), dtype, g, sc).to(gpu) for _ in range(layers)]
            for n in (300, 200)]
    kv = [(randn((48, heads, bs, 2 * d), dtype, g, sc) if fill is None else fill).to(gpu)
          for _ in range(layers)]
    plan = ShiftPlan(span_array(spans), CacheSet(bufs, "flat"), CacheSet([kv], "hnd", bs),
                     inv_freq=inv_freq(rotary), src_mode="flat", dst_mode="table",
                     dst_index=torch.tensor(table, dtype=torch.int32), k_scale=k_scale,
                     direct=direct)
    return plan, kv


@pytest.mark.parametrize("dtype,heads,d,rotary", [
    (torch.float16, 6, 128, 128),
    (torch.float32, 5, 128, 64),
    (torch.bfloat16, 3, 64, 64),
    (torch.bfloat16, 5, 256, 128),
    (torch.float8_e4m3fn, 5, 128, 128),
    (torch.bfloat16, 2, 512, 512),       # a K row fills a whole wave
    (torch.float32, 4, 256, 256),        # fp32: a K row fills a whole wave
    (torch.bfloat16, 64, 128, 128),      # one token is 8 passes of a workgroup
    (torch.float8_e4m3fn, 8, 64, 64),    # fp8: 16 rows per wave span two tokens
    (torch.float8_e4m3fn, 3, 256, 128),  # fp8: ragged heads, partial rotary
    (torch.float8_e4m3fn, 8, 128, 64),   # fp8, whole tokens per pass (span table in LDS),
    (torch.float8_e4m3fn, 8, 256, 128),  # partial rotary
])
def test_batched_other_geometries_match_oracle(gpu, dtype, heads, d, rotary):
    """Non-uniform head counts (a wave pass spans tokens), partial rotary, fp16 / fp32 /
    fp8, a table-addressed destination: every destination byte against the oracle."""
    print(f"case batched geometry {dtype} heads={heads} d={d} rotary={rotary}", flush=True)
    table = torch.randperm(48, generator=torch.Generator().manual_seed(3)).tolist()
    spans = [(5, 3, 0, 0, 120, -41, 0, 0),    # session 0, positions 3..123
             (150, 130, 0, 0, 140, 1999, 0, 0),
             (0, 300, 0, 0, 190, 0, 1, 0),     # session 1, delta 0: a plain copy
             (17, 520, 0, 0, 180, -7, 1, 0)]
    k_scale = torch.tensor([0.037, 0.081]) if dtype == torch.float8_e4m3fn else None
    plan, kv = _two_session_plan(gpu, dtype, heads, d, rotary, 11, spans, table, k_scale)
    src_o = oracle_side(plan.src, "flat", None)
    dst_o = oracle_side(plan.dst, "table", torch.tensor(table, dtype=torch.int32))
    orc.shift_spans(oracle_spans(span_array(spans)), src_o, dst_o, inv_freq(rotary).numpy(),
                    dname(dtype), None if k_scale is None else k_scale.numpy())
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    plan.launch(error_flags=flags)
    torch.cuda.synchronize(gpu)
    assert int(flags.item()) == 0
    for layer, t in enumerate(kv):
        assert np.array_equal(bits(t), dst_o.caches[0][layer]), f"layer {layer}"


@pytest.mark.parametrize("dtype,heads,d,rotary", [
    (torch.bfloat16, 1, 128, 128),       # 4 tokens per wave pass
    (torch.bfloat16, 2, 128, 128),       # 2 tokens per pass
    (torch.bfloat16, 1, 64, 64),         # 8 tokens per pass
    (torch.bfloat16, 4, 64, 32),         # 2 tokens per pass, partial rotary
    (torch.float16, 1, 128, 128),
    (torch.float32, 1, 128, 128),        # fp32: 2 tokens per pass
    (torch.float8_e4m3fn, 1, 128, 128),  # fp8: 8 tokens per pass
    (torch.float8_e4m3fn, 2, 128, 128),  # fp8: 4 tokens per pass
    (torch.float8_e4m3fn, 4, 128, 64),   # fp8: 2 tokens per pass, partial rotary
])
def test_batched_multi_token_passes_match_oracle(gpu, dtype, heads, d, rotary):
    """Head counts that divide a wave's rows: a wave pass covers several whole tokens.
    Span boundaries fall at odd tokens, so passes straddle spans of different deltas and
    the two sessions (base-address rows of different groups, the per-lane fallback);
    every destination byte against the oracle."""
    print(f"case batched multi-token {dtype} heads={heads} d={d} rotary={rotary}", flush=True)
    table = torch.randperm(48, generator=torch.Generator().manual_seed(4)).tolist()
    spans = [(5, 3, 0, 0, 121, -41, 0, 0),
             (150, 130, 0, 0, 138, 1999, 0, 0),  # session 1 starts at token 259
             (0, 300, 0, 0, 191, 0, 1, 0),     # session 1, delta 0: a plain copy
             (17, 520, 0, 0, 179, -7, 1, 0)]
    k_scale = torch.tensor([0.044, 0.072]) if dtype == torch.float8_e4m3fn else None
    plan, kv = _two_session_plan(gpu, dtype, heads, d, rotary, 13, spans, table, k_scale)
    src_o = oracle_side(plan.src, "flat", None)
    dst_o = oracle_side(plan.dst, "table", torch.tensor(table, dtype=torch.int32))
    orc.shift_spans(oracle_spans(span_array(spans)), src_o, dst_o, inv_freq(rotary).numpy(),
                    dname(dtype), None if k_scale is None else k_scale.numpy())
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    plan.launch(error_flags=flags)
    torch.cuda.synchronize(gpu)
    assert int(flags.item()) == 0
    for layer, t in enumerate(kv):
        assert np.array_equal(bits(t), dst_o.caches[0][layer]), f"layer {layer}"


@pytest.mark.parametrize("plane_axis", [0, 1])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_split_k_and_v_planes_match_oracle(gpu, dtype, plane_axis):
    """K and V in separate tensors: a fused flat store (two sessions) into the split
    planes of one cache, ``[2, blocks, bs, heads, D]`` (plane_axis 0) or ``[blocks, 2,
    bs, heads, D]`` (plane_axis 1, strided views), then those planes back into split
    flat stores.  Against the oracle on the same rows fused."""
    from marathon_amd.spans import CacheSet, ShiftPlan
    from tests.helpers import randn

    print(f"case split K/V planes {dtype} axis={plane_axis}", flush=True)
    g = torch.Generator().manual_seed(31 + plane_axis)
    layers, heads, d, bs, nblk = 2, 4, 128, 16, 40
    sc = 0.05
    bufs = [[randn((n, heads, 2 * d), dtype, g, sc) for _ in range(layers)] for n in (300, 200)]
    shape = (2, nblk, bs, heads, d) if plane_axis == 0 else (nblk, 2, bs, heads, d)
    kvs = [randn(shape, dtype, g, sc) for _ in range(layers)]

    def planes(t):
        return (t[0], t[1]) if plane_axis == 0 else (t[:, 0], t[:, 1])

    table = torch.randperm(nblk, generator=torch.Generator().manual_seed(7)).tolist()
    spans = [(5, 3, 0, 0, 121, -41, 0, 0), (150, 130, 0, 0, 138, 1999, 0, 0),
             (0, 300, 0, 0, 191, 0, 1, 0), (17, 520, 0, 0, 79, -7, 1, 0)]
    k_scale = torch.tensor([0.031, 0.066]) if dtype == torch.float8_e4m3fn else None
    kvs_dev = [t.to(gpu) for t in kvs]
    dst = CacheSet([[planes(t)[0] for t in kvs_dev]], "nhd", bs,
                   v_caches=[[planes(t)[1] for t in kvs_dev]])
    src = CacheSet([[b.to(gpu) for b in row] for row in bufs], "flat")
    tab = torch.tensor(table, dtype=torch.int32)
    plan = ShiftPlan(span_array(spans), src, dst, inv_freq=inv_freq(128), src_mode="flat",
                     dst_mode="table", dst_index=tab, k_scale=k_scale)
    # the oracle works on fused rows: the same planes, concatenated
    fused = [torch.cat(planes(t), dim=-1) for t in kvs]
    src_o = oracle_side(src, "flat", None)
    dst_o = orc.Side([[bits(t) for t in fused]], "nhd", bs, "table", tab.numpy())
    orc.shift_spans(oracle_spans(span_array(spans)), src_o, dst_o, inv_freq(128).numpy(),
                    dname(dtype), None if k_scale is None else k_scale.numpy())
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    plan.launch(error_flags=flags)
    torch.cuda.synchronize(gpu)
    assert int(flags.item()) == 0
    for layer, t in enumerate(kvs_dev):
        k, v = planes(t)
        want = dst_o.caches[0][layer]
        assert np.array_equal(bits(k), want[..., :d]), f"K layer {layer}"
        assert np.array_equal(bits(v), want[..., d:]), f"V layer {layer}"

    # and back: the planes (paged, split) into split flat stores, delta 0
    back_k = [torch.zeros(700, heads, d, dtype=dtype, device=gpu) for _ in range(layers)]
    back_v = [torch.zeros(700, heads, d, dtype=dtype, device=gpu) for _ in range(layers)]
    save = ShiftPlan(span_array([(0, 0, 0, 0, 600, 0, 0, 0)]), dst, CacheSet(
        [back_k], "flat", v_caches=[back_v]), inv_freq=None, src_mode="table", src_index=tab,
        dst_mode="flat")
    save.launch(error_flags=flags)
    torch.cuda.synchronize(gpu)
    assert int(flags.item()) == 0
    pos = torch.arange(600)
    slot = tab.long()[pos // bs] * bs + pos % bs
    for layer, t in enumerate(kvs_dev):
        k, v = planes(t)
        assert torch.equal(back_k[layer][:600], k[slot // bs, slot % bs])
        assert torch.equal(back_v[layer][:600], v[slot // bs, slot % bs])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_batched_extreme_deltas_match_oracle(gpu, dtype):
    """The plan kernel evaluates each span's cos/sin on the device: int32 extremes and
    deltas beyond 2^24, against the oracle byte for byte."""
    print(f"case batched extreme deltas {dtype}", flush=True)
    table = torch.randperm(48, generator=torch.Generator().manual_seed(6)).tolist()
    spans = [(5, 3, 0, 0, 70, 2**31 - 1, 0, 0),
             (90, 80, 0, 0, 61, -(2**31), 0, 0),
             (0, 300, 0, 0, 45, 16777219, 1, 0),
             (50, 400, 0, 0, 77, -1048577, 1, 0),
             (130, 520, 0, 0, 33, 131071, 1, 0)]
    k_scale = torch.tensor([0.05, 0.021]) if dtype == torch.float8_e4m3fn else None
    plan, kv = _two_session_plan(gpu, dtype, 8, 128, 128, 21, spans, table, k_scale)
    src_o = oracle_side(plan.src, "flat", None)
    dst_o = oracle_side(plan.dst, "table", torch.tensor(table, dtype=torch.int32))
    orc.shift_spans(oracle_spans(span_array(spans)), src_o, dst_o, inv_freq(128).numpy(),
                    dname(dtype), None if k_scale is None else k_scale.numpy())
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    plan.launch(error_flags=flags)
    torch.cuda.synchronize(gpu)
    assert int(flags.item()) == 0
    for layer, t in enumerate(kv):
        assert np.array_equal(bits(t), dst_o.caches[0][layer]), f"layer {layer}"


@pytest.mark.parametrize("direct", [False, None])
@pytest.mark.parametrize("heads", [8, 2, 1])
def test_out_of_range_rows_are_flagged_and_skipped(gpu, heads, direct):
    """Bad indices on either side never write: a -1 and a too-large block id in the
    destination table, source positions past a session's rows, and a span naming a
    group that does not exist.  Each raises its flag; every other row lands exactly as
    in a plan that leaves the bad rows out.  8 heads: one token per wave pass; 2 and 1:
    several tokens per pass, good and bad ones side by side."""
    from marathon_amd import _lib

    print(f"case out-of-range rows heads={heads} direct={direct}", flush=True)
    table = torch.randperm(48, generator=torch.Generator().manual_seed(5)).tolist()
    bad_table = list(table)
    bad_table[2] = -1  # positions 32..47
    bad_table[4] = 10**6  # positions 64..79
    spans_bad = [(0, 20, 0, 0, 80, 33, 0, 0),       # dst 20..100 crosses blocks 2 and 4
                 (190, 400, 0, 0, 20, -5, 1, 0),    # src 190..210, session 1 has 200 rows
                 (0, 600, 0, 0, 30, 0, 7, 0)]       # group 7 does not exist
    spans_ok = [(0, 20, 0, 0, 12, 33, 0, 0),        # 20..32
                (28, 48, 0, 0, 16, 33, 0, 0),       # 48..64
                (60, 80, 0, 0, 20, 33, 0, 0),       # 80..100
                (190, 400, 0, 0, 10, -5, 1, 0)]     # src 190..200
    fill = torch.full((48, heads, 16, 256), 3.0).to(torch.bfloat16)
    plan_b, kv_b = _two_session_plan(gpu, torch.bfloat16, heads, 128, 128, 4, spans_bad,
                                     bad_table, fill=fill, direct=direct)
    plan_g, kv_g = _two_session_plan(gpu, torch.bfloat16, heads, 128, 128, 4, spans_ok, table,
                                     fill=fill, direct=direct)
    fb = torch.zeros(1, dtype=torch.int32, device=gpu)
    fg = torch.zeros(1, dtype=torch.int32, device=gpu)
    plan_b.launch(error_flags=fb)
    plan_g.launch(error_flags=fg)
    torch.cuda.synchronize(gpu)
    assert int(fg.item()) == 0
    want = _lib.MKV_FLAG_SRC_RANGE | _lib.MKV_FLAG_DST_RANGE | _lib.MKV_FLAG_SPAN
    assert int(fb.item()) == want
    for a, b in zip(kv_b, kv_g):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("heads", [8, 1])
def test_single_span_out_of_range_slot_is_flagged_and_skipped(gpu, heads):
    from marathon_amd import _lib, rope_shift, scatter_shifted

    print(f"case single-span out-of-range slot heads={heads}", flush=True)
    g = torch.Generator().manual_seed(8)
    src = torch.randn(40, heads, 256, generator=g).to(torch.bfloat16).to(gpu)
    kv = torch.zeros(4, heads, 16, 256, dtype=torch.bfloat16, device=gpu)
    kv_ok = kv.clone()
    sl = torch.arange(40, dtype=torch.int64)
    sl[7] = 64  # the cache holds 64 slots
    sl[30] = -3
    keep = torch.tensor([i not in (7, 30) for i in range(40)])
    shift = rope_shift(123, 128, inv_freq(), gpu)
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    scatter_shifted(src, kv, sl.to(gpu), 16, True, shift, error_flags=flags)
    scatter_shifted(src[keep.to(gpu)].contiguous(), kv_ok, sl[keep].to(gpu), 16, True, shift)
    torch.cuda.synchronize(gpu)
    assert int(flags.item()) == _lib.MKV_FLAG_DST_RANGE
    assert torch.equal(kv.view(torch.int16), kv_ok.view(torch.int16))


@pytest.mark.parametrize("direct", [False, True])
def test_plan_launched_on_another_stream(gpu, direct):
    """A plan built on the current stream (its tables copied there) and launched at once
    on a side stream, with no host synchronisation in between: the launch first makes
    the side stream wait for the build stream and for the caches' base-address tables,
    and keeps the plan's buffers alive on that stream.  Every destination byte against
    the oracle, then a second launch on the same side stream."""
    print(f"case plan launched on a side stream direct={direct}", flush=True)
    wl = W.qwen3_14b_multispan(gpu, layers=2, history=1024, dst_fill="random")
    src_o = oracle_side(wl.src, wl.src_mode, wl.src_index)
    dst_o = oracle_side(wl.dst, wl.dst_mode, wl.dst_index)
    orc.shift_spans(oracle_spans(wl.spans), src_o, dst_o, wl.inv_freq.numpy(), "bf16")
    torch.cuda.synchronize(gpu)
    side = torch.cuda.Stream(device=gpu)
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    torch.cuda.synchronize(gpu)
    # the caches and flags are complete (synchronised above); the plan's tables are
    # copied on the current stream, and only the launch's stream wait orders that copy
    # before the side-stream launch
    plan = wl.plan(direct=direct)
    assert plan.direct is direct
    plan.launch(side.cuda_stream, error_flags=flags)
    plan.launch(side.cuda_stream, error_flags=flags)  # a second launch: same bytes
    side.synchronize()
    assert int(flags.item()) == 0
    for layer, t in enumerate(wl.dst.caches[0]):
        assert np.array_equal(bits(t), dst_o.caches[0][layer]), f"layer {layer}"


@pytest.mark.parametrize("direct", [False, True])
def test_plan_launch_replays_from_a_hip_graph(gpu, direct):
    """A captured launch replays exactly like an eager one: three replays, with eager
    work between them (new source values, a cleared destination, an eager launch that
    gives the expected bytes), each replay checked byte for byte.  Both kernel paths:
    plan pass + shift, and the direct single launch."""
    print(f"case graph capture of a batched plan direct={direct}", flush=True)
    wl = W.qwen3_14b_multispan(gpu, layers=2, history=1024, dst_fill="zeros")
    plan = wl.plan(direct=direct)
    assert plan.direct is direct
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    plan.launch(error_flags=flags)  # warm-up, eager
    torch.cuda.synchronize(gpu)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.launch(error_flags=flags)
    for i in range(3):
        for c in wl.src.caches[0] + (wl.src.v_caches[0] if wl.src.split else []):
            c.mul_(-1.0 if i % 2 == 0 else 0.5)  # exact in bf16: a sign flip, a halving
        for c in wl.dst.caches[0]:
            c.zero_()
        plan.launch(error_flags=flags)
        torch.cuda.synchronize(gpu)
        want = [c.clone() for c in wl.dst.caches[0]]
        for c in wl.dst.caches[0]:
            c.zero_()
        torch.cuda.synchronize(gpu)
        graph.replay()
        torch.cuda.synchronize(gpu)
        for layer, (a, b) in enumerate(zip(wl.dst.caches[0], want)):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), (i, layer)
        assert bool(want[0].view(torch.int16).any())
    assert int(flags.item()) == 0


def test_connector_loader_fp8_with_layer_scales(gpu):
    """The loader on an fp8 paged cache: each layer's K scale reaches the kernel, K is
    dequantised, rotated and requantised exactly as the oracle's fp8 rule, V is copied."""
    print("case connector loader fp8", flush=True)
    layers, heads, d, bs = 3, 8, 128, 16
    names = [f"layers.{i}" for i in range(layers)]
    scales = {name: s for name, s in zip(names, (0.013, 0.05, 0.094))}
    store = ShiftStore(budget_tokens=4096, device=str(gpu), slab=512)
    g = torch.Generator().manual_seed(33)
    assert store.reserve("s", 0, 400)
    for name in names:
        x = (torch.randn(400, heads, 2 * d, generator=g) / scales[name]).clamp(-448, 448)
        store.write("s", name, 0, x.to(torch.float8_e4m3fn).to(gpu))
    kv = {name: torch.zeros(40, heads, bs, 2 * d, dtype=torch.float8_e4m3fn, device=gpu)
          for name in names}
    loader = ShiftLoader(store, bs, inv_freq(), k_scales=scales)
    loader.register_kv_caches(kv)
    perm = torch.randperm(40, generator=g).tolist()
    ld = Load("s", slots(perm, 21, 21 + 333, bs), src_start=50, delta=-29)
    assert loader.start_load_kv([ld]) == 333 * layers
    torch.cuda.synchronize(gpu)
    for name in names:
        want = np.zeros_like(bits(kv[name]))
        src_rows = bits(store.read("s", name, 50, 333))
        orc.scatter_shifted(src_rows, want, ld.slots.numpy(), bs, True, -29,
                            inv_freq().numpy(), "fp8", np.float32(scales[name]))
        assert np.array_equal(bits(kv[name]), want), name


def test_load_read_back_check(gpu):
    """The reference's MARATHON_VERIFY_LOAD read-back (vllm_shift_connector.py:444-480),
    on a block-store bf16 load with partial rotary and on a flat-store fp8 load with
    per-layer K scales: one entry per (load, layer), V exact, K within half an element
    step of torch's fp32 rotation (bf16: 2^-9 of the largest value, checked at 2^-8;
    e4m3: 2^-4, checked at 0.07)."""
    from marathon_amd import BlockShiftStore
    from marathon_amd.connector import Load as L

    print("case load read-back check", flush=True)
    layers, heads, d, bs = 2, 8, 128, 16
    names = [f"layers.{i}" for i in range(layers)]
    g = torch.Generator().manual_seed(71)
    # bf16, block store, rotary 64 of 128
    store = BlockShiftStore(budget_tokens=2048, device=str(gpu), block_size=bs)
    assert store.reserve("s", 0, 500)
    for name in names:
        store.write_target("s", name, 0, 500, (heads, 2 * d), torch.bfloat16,
                           gpu).copy_(torch.randn(store.pool_blocks, 2, bs, heads, d,
                                                  generator=g).to(torch.bfloat16))
    kv = {name: torch.zeros(48, heads, bs, 2 * d, dtype=torch.bfloat16, device=gpu)
          for name in names}
    loader = ShiftLoader(store, bs, inv_freq(64), verify=True)
    loader.register_kv_caches(kv)
    table = torch.randperm(48, generator=g).numpy().astype(np.int32)
    loads = [L.from_blocks("s", table, 40, 300, -17), L.from_blocks("s", table, 310, 470, 0)]
    loader.start_load_kv(loads)
    torch.cuda.synchronize(gpu)
    log = loader.verify_log
    assert len(log) == len(loads) * layers
    for e in log:
        assert e["v_exact"], e
        assert e["max_rel"] <= 2.0**-8, e
    assert any(e["max_abs"] > 0 for e in log if e["delta"] != 0)  # a rotation happened
    assert all(e["max_abs"] == 0 for e in log if e["delta"] == 0)  # delta 0: a copy

    # fp8, flat store, per-layer scales
    scales = {name: s for name, s in zip(names, (0.02, 0.07))}
    fstore = ShiftStore(budget_tokens=2048, device=str(gpu), slab=512)
    assert fstore.reserve("f", 0, 300)
    for name in names:
        x = (torch.randn(300, heads, 2 * d, generator=g) / scales[name]).clamp(-448, 448)
        fstore.write("f", name, 0, x.to(torch.float8_e4m3fn).to(gpu))
    fkv = {name: torch.zeros(32, heads, bs, 2 * d, dtype=torch.float8_e4m3fn, device=gpu)
           for name in names}
    floader = ShiftLoader(fstore, bs, inv_freq(), k_scales=scales, verify=True)
    floader.register_kv_caches(fkv)
    perm = torch.randperm(32, generator=g).tolist()
    floader.start_load_kv([L("f", slots(perm, 5, 5 + 250, bs), src_start=30, delta=211)])
    torch.cuda.synchronize(gpu)
    assert len(floader.verify_log) == layers
    for e in floader.verify_log:
        assert e["v_exact"], e
        assert 0 < e["max_rel"] <= 0.07, e


def test_more_spans_than_one_launch_takes(gpu):
    """5,000 short spans (some empty), past the 4,096-span launch limit: the plan splits
    them into launches that share one workspace in stream order; every destination byte
    against the oracle."""
    from marathon_amd import _lib
    from marathon_amd.spans import CacheSet, ShiftPlan

    print("case 5,000 spans in two launches", flush=True)
    rng = np.random.default_rng(17)
    g = torch.Generator().manual_seed(17)
    layers, heads, d, bs, n_spans = 2, 8, 128, 16, 5000
    lens = rng.integers(0, 4, n_spans)
    hist = [4096, 3000]
    bufs = [[torch.randn(h, heads, 2 * d, generator=g).to(torch.bfloat16).to(gpu)
             for _ in range(layers)] for h in hist]
    total = int(lens.sum())
    blocks = -(-total // bs) + 4
    kv = [torch.randn(blocks, heads, bs, 2 * d, generator=g).to(torch.bfloat16).to(gpu)
          for _ in range(layers)]
    dst_slots = torch.from_numpy(rng.permutation(blocks * bs)[:total].astype(np.int64))
    rows, off = [], 0
    for i, n in enumerate(lens):
        grp = int(rng.integers(2))
        src = int(rng.integers(0, hist[grp] - 4))
        rows.append((src, 0, 0, off, int(n), int(rng.integers(-3000, 3000)), grp, 0))
        off += int(n)
    assert n_spans > _lib.MKV_MAX_SPANS
    plan = ShiftPlan(span_array(rows), CacheSet(bufs, "flat"), CacheSet([kv], "hnd", bs),
                     inv_freq=inv_freq(), src_mode="flat", dst_mode="slots",
                     dst_index=dst_slots)
    assert len(plan.descs) == 2
    src_o = oracle_side(plan.src, "flat", None)
    dst_o = oracle_side(plan.dst, "slots", dst_slots)
    orc.shift_spans(oracle_spans(span_array(rows)), src_o, dst_o, inv_freq().numpy(), "bf16")
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    plan.launch(error_flags=flags)
    torch.cuda.synchronize(gpu)
    assert int(flags.item()) == 0
    for layer in range(layers):
        assert np.array_equal(bits(kv[layer]), dst_o.caches[0][layer]), f"layer {layer}"


def test_direct_path_flags_a_prefix_that_disagrees_with_the_spans(gpu):
    """The direct path trusts no caller prefix: a prefix whose steps differ from the
    spans' token counts raises MKV_FLAG_SPAN, and the tokens it does map still land on
    their own rows (every row bounds-checked), so nothing outside the spans' rows is
    written."""
    import ctypes

    from marathon_amd import _lib
    from marathon_amd.shift_kernels import current_stream

    print("case direct path with a bad prefix", flush=True)
    wl = W.qwen3_14b_multispan(gpu, layers=2, history=1024, dst_fill="random")
    plan = wl.plan(direct=True)
    assert plan.direct
    counts = [int(c) for c in wl.spans["n_tokens"]]
    good = np.concatenate(([0], np.cumsum(counts))).astype(np.int64)
    bad = good.copy()
    bad[1] -= 5  # span 0's last 5 tokens are never mapped; span 1 starts 5 early
    dst_o = oracle_side(wl.dst, wl.dst_mode, wl.dst_index)
    src_o = oracle_side(wl.src, wl.src_mode, wl.src_index)
    torch.cuda.synchronize(gpu)
    before = [bits(t) for t in wl.dst.caches[0]]
    orc.shift_spans(oracle_spans(wl.spans), src_o, dst_o, wl.inv_freq.numpy(), "bf16")
    starts = torch.from_numpy(bad).to(gpu)
    d = plan.descs[0]
    d.span_starts = starts.data_ptr()
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    d.error_flags = flags.data_ptr()
    _lib.check(_lib.lib().mkv_shift_spans(ctypes.byref(d), ctypes.c_void_p(current_stream(gpu))))
    torch.cuda.synchronize(gpu)
    assert int(flags.item()) & _lib.MKV_FLAG_SPAN
    # every destination row is either untouched or the oracle's (no stray writes)
    for layer, t in enumerate(wl.dst.caches[0]):
        def tokens(a):  # HND [blocks, heads, 16, 2D] -> one row per (block, offset)
            return a.transpose(0, 2, 1, 3)

        got = tokens(bits(t))
        ok = (got == tokens(before[layer])).all(axis=(-1, -2)) | (
            got == tokens(dst_o.caches[0][layer])).all(axis=(-1, -2))
        assert bool(ok.all()), f"layer {layer}: a row is neither untouched nor the oracle's"


def test_page_order_over_a_destination_wider_than_256_pages(gpu):
    """A 590 MB destination cache (9,000 HND blocks of 64 KB): the page order's buckets
    widen to 4 MB so the extent fits 256 of them.  Sorted and span-ordered plans write
    the oracle's bytes."""
    from marathon_amd.spans import CacheSet, ShiftPlan

    print("case page order over a 590 MB destination", flush=True)
    rng = np.random.default_rng(23)
    g = torch.Generator().manual_seed(23)
    heads, d, bs, blocks, n = 8, 128, 16, 9000, 3000
    src = [torch.randn(4096, heads, 2 * d, generator=g).to(torch.bfloat16).to(gpu)]
    kv = [torch.zeros(blocks, heads, bs, 2 * d, dtype=torch.bfloat16, device=gpu)]
    assert kv[0].numel() * 2 > 512 << 20
    dst_slots = torch.from_numpy(rng.permutation(blocks * bs)[:n].astype(np.int64))
    rows = [(0, 0, 0, 0, 1000, 77, 0, 0), (1500, 0, 0, 1000, 2000, -901, 0, 0)]
    src_o = oracle_side(CacheSet([src], "flat"), "flat", None)
    dst_o = oracle_side(CacheSet([kv], "hnd", bs), "slots", dst_slots)
    orc.shift_spans(oracle_spans(span_array(rows)), src_o, dst_o, inv_freq().numpy(), "bf16")
    for order in ("none", "dst_page", "dst_page_device"):
        kv[0].zero_()
        plan = ShiftPlan(span_array(rows), CacheSet([src], "flat"), CacheSet([kv], "hnd", bs),
                         inv_freq=inv_freq(), src_mode="flat", dst_mode="slots",
                         dst_index=dst_slots, direct=False, order=order)
        flags = torch.zeros(1, dtype=torch.int32, device=gpu)
        plan.launch(error_flags=flags)
        torch.cuda.synchronize(gpu)
        assert int(flags.item()) == 0
        assert np.array_equal(bits(kv[0]), dst_o.caches[0][0]), order


@pytest.mark.parametrize("dtype,d,layers", [
    (torch.bfloat16, 128, 6), (torch.bfloat16, 128, 9), (torch.float32, 128, 6),
    (torch.float8_e4m3fn, 128, 9), (torch.float16, 64, 5), (torch.bfloat16, 256, 7),
    (torch.float32, 256, 4)])
def test_direct_path_above_the_wide_threshold(gpu, dtype, d, layers):
    """A direct shift of more than 2,560 (token, layer) rows: 2- and 4-byte elements move
    four layers per workgroup, so 5, 6, 7 and 9 layers leave a partial last group (fp8
    stays at one layer per workgroup).  Every destination byte against the oracle."""
    from marathon_amd.spans import CacheSet, ShiftPlan

    eb = torch.empty(0, dtype=dtype).element_size()
    heads = max(1, 64 // (d * eb // 16))  # the smallest head count the direct path takes
    print(f"case wide direct shift {dtype} d={d} heads={heads} layers={layers}", flush=True)
    rng = np.random.default_rng(layers)
    g = torch.Generator().manual_seed(layers)
    bs, hist, blocks = 16, 1200, 120
    k_scale = None
    if dtype == torch.float8_e4m3fn:
        k_scale = torch.from_numpy(rng.uniform(0.01, 0.1, layers).astype(np.float32))
    src = [randn((hist, heads, 2 * d), dtype, g,
                 1.0 if k_scale is None else float(k_scale[i])).to(gpu) for i in range(layers)]
    kv = [torch.zeros(blocks, heads, bs, 2 * d, dtype=dtype, device=gpu) for _ in range(layers)]
    n = 700
    dst_slots = torch.from_numpy(rng.permutation(blocks * bs)[:n].astype(np.int64))
    rows = [(0, 0, 0, 0, 300, 45, 0, 0), (500, 0, 0, 300, 250, -2000, 0, 0),
            (900, 0, 0, 550, 150, 0, 0, 0)]
    assert n * layers > 2560
    src_set, dst_set = CacheSet([src], "flat"), CacheSet([kv], "hnd", bs)
    inv = inv_freq(d)
    plan = ShiftPlan(span_array(rows), src_set, dst_set, inv_freq=inv, src_mode="flat",
                     dst_mode="slots", dst_index=dst_slots, k_scale=k_scale, direct=True)
    assert plan.direct
    src_o = oracle_side(src_set, "flat", None)
    dst_o = oracle_side(dst_set, "slots", dst_slots)
    orc.shift_spans(oracle_spans(span_array(rows)), src_o, dst_o, inv.numpy(),
                    dname(dtype), None if k_scale is None else k_scale.numpy())
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    plan.launch(error_flags=flags)
    torch.cuda.synchronize(gpu)
    assert int(flags.item()) == 0
    for layer in range(layers):
        assert np.array_equal(bits(kv[layer]), dst_o.caches[0][layer]), f"layer {layer}"


def test_caller_token_order(gpu):
    """``mkv_shift_desc_t.token_order``: the plan pass resolves record i from token
    token_order[i].  A reversed order writes the oracle's bytes; an entry out of range
    raises MKV_FLAG_SPAN and leaves that record empty (its token is not moved, and every
    other row is still the oracle's or untouched)."""
    import ctypes

    from marathon_amd import _lib, workloads as W
    from marathon_amd.shift_kernels import current_stream

    print("case caller token order", flush=True)
    wl = W.qwen3_14b_multispan(gpu, layers=2, history=2048, dst_fill="random")
    src_o = oracle_side(wl.src, wl.src_mode, wl.src_index)
    dst_o = oracle_side(wl.dst, wl.dst_mode, wl.dst_index)
    orc.shift_spans(oracle_spans(wl.spans), src_o, dst_o, wl.inv_freq.numpy(), "bf16")
    before = [bits(t) for t in wl.dst.caches[0]]
    plan = wl.plan(direct=False, order="none")
    torch.cuda.synchronize(gpu)
    (d,) = plan.descs
    n = int(d.total_tokens)
    L = _lib.lib()
    stream = ctypes.c_void_p(current_stream(gpu))
    for name, order in (("reversed", np.arange(n - 1, -1, -1)),
                        ("one entry out of range", np.r_[np.arange(n - 1), n + 5])):
        for t, b in zip(wl.dst.caches[0], before):
            t.copy_(torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).to(gpu))
        order_dev = torch.from_numpy(order.astype(np.int32)).to(gpu)
        flags = torch.zeros(1, dtype=torch.int32, device=gpu)
        d.token_order = order_dev.data_ptr()
        d.error_flags = flags.data_ptr()
        _lib.check(L.mkv_shift_spans(ctypes.byref(d), stream))
        torch.cuda.synchronize(gpu)
        if name == "reversed":
            assert int(flags.item()) == 0
            for layer, t in enumerate(wl.dst.caches[0]):
                assert np.array_equal(bits(t), dst_o.caches[0][layer]), f"{name} layer {layer}"
        else:
            assert int(flags.item()) & _lib.MKV_FLAG_SPAN
            for layer, t in enumerate(wl.dst.caches[0]):
                got = bits(t).transpose(0, 2, 1, 3)  # one row per (block, offset)
                ok = (got == before[layer].transpose(0, 2, 1, 3)).all(axis=(-1, -2)) | (
                    got == dst_o.caches[0][layer].transpose(0, 2, 1, 3)).all(axis=(-1, -2))
                assert bool(ok.all()), f"{name} layer {layer}"
                # the last token (never named) was not moved: its row kept its old bytes
                last = int(wl.dst_index[-1])
                assert np.array_equal(bits(t)[last // 16, :, last % 16],
                                      before[layer][last // 16, :, last % 16])
    d.token_order = None
