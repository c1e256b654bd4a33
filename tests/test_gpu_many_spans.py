"""Span-count limits on the GPU, against the oracle byte for byte.

* More spans than one descriptor takes (``MKV_MAX_SPANS``, 4,096): ``ShiftPlan`` splits
  them into several plan + shift launches on one workspace, in stream order.
* The direct path's limit (``MKV_DIRECT_MAX_SPANS``, 63 spans) and one span past it,
  where ``ShiftPlan`` must fall back to the two-launch path.
* Empty spans among the others (their prefix entries repeat), and a shift with no
  tokens at all.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from marathon_amd import _lib
from marathon_amd import workloads as W
from marathon_amd.spans import CacheSet, ShiftPlan, span_array
from oracle import kvshift_oracle as orc
from tests.helpers import bits, inv_freq, oracle_side, oracle_spans

pytestmark = pytest.mark.gpu

HEADS, D, BS, LAYERS = 8, 128, 16, 2


def _many_spans(gpu, n_spans: int, seed: int, max_len: int, empty_every: int = 0):
    """n_spans short spans (1..max_len tokens, deltas of both signs and 0) from a store
    of K/V-plane blocks through a shuffled table into an HND cache through slots, with
    disjoint destinations; every ``empty_every``-th span has no tokens."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(1, max_len + 1, n_spans)
    if empty_every:
        lens[::empty_every] = 0
    total = int(lens.sum())
    src_hist = total + 64
    src_blocks = -(-src_hist // BS)
    dst_hist = total + n_spans * 3 + 64
    dst_blocks = -(-dst_hist // BS) + 4
    gen = torch.Generator(device=gpu)
    gen.manual_seed(seed)
    src = W.store_cache_set([[W.store_blocks(src_blocks, HEADS, torch.bfloat16, gen, gpu)
                              for _ in range(LAYERS)]])
    dst = CacheSet([[torch.randn(dst_blocks, HEADS, BS, 2 * D, device=gpu, generator=gen)
                     .to(torch.bfloat16) for _ in range(LAYERS)]], "hnd", BS)
    src_table = rng.permutation(src_blocks).astype(np.int32)
    dst_table = rng.permutation(dst_blocks).astype(np.int64)
    rows, slots_parts, d_pos, d_off = [], [], 0, 0
    for n in lens.tolist():
        s_pos = int(rng.integers(0, src_hist - n + 1))
        d_pos += int(rng.integers(0, 4))
        delta = int(rng.choice([0, int(rng.integers(-3000, 3001))]))
        pos = np.arange(d_pos, d_pos + n)
        slots_parts.append(dst_table[pos // BS] * BS + pos % BS)
        rows.append((s_pos, 0, 0, d_off, n, delta, 0, 0))
        d_pos += n
        d_off += n
    spans = span_array(rows)
    src_index = torch.from_numpy(src_table)
    dst_index = torch.from_numpy(np.concatenate(slots_parts))
    return spans, src, dst, src_index, dst_index


def _check(gpu, spans, src, dst, src_index, dst_index, **plan_kw):
    src_o = oracle_side(src, "table", src_index)
    dst_o = oracle_side(dst, "slots", dst_index)
    orc.shift_spans(oracle_spans(spans), src_o, dst_o, inv_freq().numpy(), "bf16")
    plan = ShiftPlan(spans, src, dst, inv_freq=inv_freq(), src_mode="table",
                     src_index=src_index, dst_mode="slots", dst_index=dst_index, **plan_kw)
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    plan.launch(error_flags=flags)
    torch.cuda.synchronize(gpu)
    assert int(flags.item()) == 0
    for layer in range(LAYERS):
        got = bits(dst.caches[0][layer])
        bad = int((got != dst_o.caches[0][layer]).sum())
        assert bad == 0, f"layer {layer}: {bad} elements differ"
    return plan


@pytest.mark.parametrize("order", ["none", "dst_page", "dst_page_device"])
def test_more_spans_than_one_descriptor_takes(gpu, order):
    n = _lib.MKV_MAX_SPANS + 905
    print(f"case {n} spans in one plan (several launches), order={order}", flush=True)
    plan = _check(gpu, *_many_spans(gpu, n, seed=11, max_len=6), direct=False, order=order)
    assert len(plan.descs) == 2 and not plan.direct


@pytest.mark.parametrize("n_spans,direct", [(_lib.MKV_DIRECT_MAX_SPANS, True),
                                            (_lib.MKV_DIRECT_MAX_SPANS + 1, False)])
def test_direct_path_span_limit(gpu, n_spans, direct):
    print(f"case {n_spans} spans, direct path asked for", flush=True)
    plan = _check(gpu, *_many_spans(gpu, n_spans, seed=12 + n_spans, max_len=9), direct=True)
    assert plan.direct is direct


@pytest.mark.parametrize("direct", [False, True])
def test_empty_spans_among_the_others(gpu, direct):
    print(f"case 40 spans, every third empty, direct={direct}", flush=True)
    plan = _check(gpu, *_many_spans(gpu, 40, seed=21, max_len=30, empty_every=3),
                  direct=direct)
    assert plan.direct is direct


def test_a_shift_with_no_tokens_changes_nothing(gpu):
    print("case spans with no tokens only, and no spans", flush=True)
    spans, src, dst, src_index, dst_index = _many_spans(gpu, 5, seed=22, max_len=4,
                                                        empty_every=1)
    before = [t.clone() for t in dst.caches[0]]
    for rows in (spans, span_array([])):
        for direct in (False, True):
            plan = ShiftPlan(rows, src, dst, inv_freq=inv_freq(), src_mode="table",
                             src_index=src_index, dst_mode="slots",
                             dst_index=dst_index[:0], direct=direct)
            flags = torch.zeros(1, dtype=torch.int32, device=gpu)
            plan.launch(error_flags=flags)
            torch.cuda.synchronize(gpu)
            assert int(flags.item()) == 0
    for t, t0 in zip(dst.caches[0], before):
        assert torch.equal(t.view(torch.int16), t0.view(torch.int16))
