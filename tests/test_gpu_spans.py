"""Batched shifts on the GPU (one launch over a span table) against the oracle.

Reduced-size versions of the multi-span (config 3), fp8 (config 4) and batched-session
(config 5) workloads, every byte of every destination cache compared with the oracle's
``shift_spans``; and the connector-shaped loader reading straight out of a store.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from marathon_amd import ShiftStore, slots
from marathon_amd import workloads as W
from marathon_amd.connector import Load, ShiftLoader
from oracle import kvshift_oracle as orc
from tests.helpers import bits, inv_freq, oracle_side, oracle_spans

pytestmark = pytest.mark.gpu


def _check_workload(wl, dev, dtype_name="bf16"):
    src_o = oracle_side(wl.src, wl.src_mode, wl.src_index)
    dst_o = oracle_side(wl.dst, wl.dst_mode, wl.dst_index)
    k_scale = None if wl.k_scale is None else wl.k_scale.numpy()
    orc.shift_spans(oracle_spans(wl.spans), src_o, dst_o, wl.inv_freq.numpy(), dtype_name,
                    k_scale)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    wl.plan().launch(error_flags=flags)
    torch.cuda.synchronize(dev)
    assert int(flags.item()) == 0
    for g, row in enumerate(wl.dst.caches):
        for layer, t in enumerate(row):
            got = bits(t)
            want = dst_o.caches[g][layer]
            bad = int((got != want).sum())
            assert bad == 0, f"group {g} layer {layer}: {bad} elements differ"


@pytest.mark.parametrize("history,layers", [(2048, 3), (4099, 2)])
def test_multispan_matches_oracle(gpu, history, layers):
    print(f"case multispan history={history} layers={layers}", flush=True)
    wl = W.config3(gpu, layers=layers, history=history, dst_fill="random")
    lay = wl.meta["layout"]
    assert np.any(lay.delta == 0) and np.any(lay.delta > 0) and np.any(lay.delta < 0)
    _check_workload(wl, gpu)


def test_fp8_multispan_matches_oracle(gpu):
    print("case fp8 multispan", flush=True)
    wl = W.config4(gpu, layers=3, history=2048)
    _check_workload(wl, gpu, "fp8")


def test_batched_sessions_match_oracle(gpu):
    print("case batched sessions", flush=True)
    wl = W.config5(gpu, layers=2, sessions=6, hist_lo=64, hist_hi=700)
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
