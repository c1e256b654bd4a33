"""Seeded random batched shifts against the oracle, byte for byte.

Each case draws:
* a geometry: element type, head size, heads, rotary width, one to five layers, block
  size;
* a source side: flat session stores, or paged NHD / HND caches through block tables,
  in one to three groups;
* a destination side: a paged NHD or HND cache through a slot mapping or a block table,
  or flat session stores, in one or two groups;
* for each side, fused rows (K then V) or split K and V planes, either as strided views
  of one tensor that holds both planes (``[blocks, 2, ...]``) or as two tensors;
* one to six spans of up to 240 tokens, with disjoint destinations and deltas of both
  signs, zero and large (the largest cases pass the direct path's four-layer threshold).
Every destination byte of every layer must equal the oracle's, and no error flag may be
raised.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from marathon_amd.spans import CacheSet, ShiftPlan, span_array
from oracle import kvshift_oracle as orc
from tests.helpers import bits, dname, inv_freq, oracle_side, oracle_spans, randn

pytestmark = pytest.mark.gpu

# more seeds for a longer sweep: MKV_RANDOM_CASES=2000 python -m pytest tests/test_gpu_random.py
_EXTRA = int(__import__("os").environ.get("MKV_RANDOM_CASES", "0"))

DTYPES = [torch.bfloat16, torch.float16, torch.float32, torch.float8_e4m3fn]
EB = {torch.bfloat16: 2, torch.float16: 2, torch.float32: 4, torch.float8_e4m3fn: 1}


def _case(seed: int):
    rng = np.random.default_rng(seed)
    dtype = DTYPES[seed % len(DTYPES)]
    eb = EB[dtype]
    d = int(rng.choice([64, 128, 256]))
    per_chunk = 16 // eb
    rot_choices = [r for r in (0, d // 2, d) if r % (2 * per_chunk) == 0]
    rotary = int(rng.choice(rot_choices))
    heads = int(rng.choice([1, 2, 3, 4, 5, 6, 8, 12, 16]))
    layers = int(rng.integers(1, 6))
    bs = int(rng.choice([16, 16, 32]))
    src_layout = str(rng.choice(["flat", "nhd", "hnd"]))
    dst_layout = str(rng.choice(["nhd", "hnd", "flat"]))
    dst_mode = "flat" if dst_layout == "flat" else str(rng.choice(["slots", "table"]))
    src_groups = int(rng.integers(1, 4))
    dst_groups = int(rng.integers(1, 3)) if dst_mode != "slots" else 1
    # the K/V split of each side from a generator of its own, so that the other draws
    # stay those of the cases before the split was drawn: 0 fused, 1 planes in one
    # tensor, 2 planes in two tensors
    split_rng = np.random.default_rng(10**6 + seed)
    src_split, dst_split = (int(x) for x in split_rng.integers(0, 3, 2))
    return dict(seed=seed, dtype=dtype, d=d, rotary=rotary, heads=heads, layers=layers,
                bs=bs, src_layout=src_layout, dst_layout=dst_layout, dst_mode=dst_mode,
                src_groups=src_groups, dst_groups=dst_groups, src_split=src_split,
                dst_split=dst_split, rng=rng)


def _paged_shape(blocks, layout, bs, heads, d):
    return (blocks, heads, bs, 2 * d) if layout == "hnd" else (blocks, bs, heads, 2 * d)


def _cache_set(caches, layout, bs, split, gpu) -> CacheSet:
    """A CacheSet on ``gpu`` holding the fused-row CPU tensors ``caches[group][layer]``:
    as they are (split 0), or as K and V planes -- strided views of one tensor with the
    two planes on axis 1 (split 1), or two tensors (split 2)."""
    bs = 1 if layout == "flat" else bs
    rows = [[t.to(gpu) for t in row] for row in caches]
    if split == 0:
        return CacheSet(rows, layout, bs)
    k_rows, v_rows = [], []
    for row in rows:
        ks, vs = [], []
        for t in row:
            d = t.shape[-1] // 2
            if split == 1:
                both = torch.stack((t[..., :d], t[..., d:]), dim=1).contiguous()
                ks.append(both[:, 0])
                vs.append(both[:, 1])
            else:
                ks.append(t[..., :d].contiguous())
                vs.append(t[..., d:].contiguous())
        k_rows.append(ks)
        v_rows.append(vs)
    return CacheSet(k_rows, layout, bs, v_caches=v_rows)


def _restore(cs: CacheSet, start) -> None:
    """Set every (group, layer) cache back to the fused rows ``start[group][layer]``."""
    for g in range(cs.groups):
        for layer in range(cs.layers):
            t0 = start[g][layer]
            if cs.split:
                d = t0.shape[-1] // 2
                cs.caches[g][layer].copy_(t0[..., :d])
                cs.v_caches[g][layer].copy_(t0[..., d:])
            else:
                cs.caches[g][layer].copy_(t0)


def _build(c, gpu):
    rng, dtype, d, heads, layers, bs = c["rng"], c["dtype"], c["d"], c["heads"], c["layers"], c["bs"]
    gen = torch.Generator().manual_seed(c["seed"])
    fp8 = dtype == torch.float8_e4m3fn
    sc = 0.05

    # source: per group, a flat store of `rows` positions or a paged cache through a table
    src_rows = [int(rng.integers(64, 400)) for _ in range(c["src_groups"])]
    src_caches, src_tabs, src_tab_off = [], [], []
    if c["src_layout"] == "flat":
        for g in range(c["src_groups"]):
            src_caches.append([randn((src_rows[g], heads, 2 * d), dtype, gen, sc)
                               for _ in range(layers)])
    else:
        # one block count for every group (a CacheSet's groups share trailing shapes;
        # the block count may differ, but equal sizes keep the case simple)
        nb = max(-(-r // bs) for r in src_rows) + 2
        off = 0
        for g in range(c["src_groups"]):
            src_caches.append([randn(_paged_shape(nb, c["src_layout"], bs, heads, d), dtype,
                                     gen, sc) for _ in range(layers)])
            src_tabs.append(rng.permutation(nb)[: -(-src_rows[g] // bs)].astype(np.int32))
            src_tab_off.append(off)
            off += src_tabs[-1].size

    # spans: disjoint destination ranges in each destination group's position space
    n_spans = int(rng.integers(1, 7))
    dst_pos_space = [0] * c["dst_groups"]
    raw = []
    for _ in range(n_spans):
        g = int(rng.integers(c["src_groups"]))
        n = int(rng.integers(1, min(240, src_rows[g]) + 1))
        sp = int(rng.integers(0, src_rows[g] - n + 1))
        dg = int(rng.integers(c["dst_groups"]))
        dp = dst_pos_space[dg] + int(rng.integers(0, 40))
        dst_pos_space[dg] = dp + n
        delta = int(rng.choice([0, int(rng.integers(-64, 65)), int(rng.integers(-40000, 40001)),
                                int(rng.integers(-(2**31), 2**31))]))
        raw.append((sp, dp, n, delta, g, dg))

    dst_blocks = max(-(-p // bs) for p in dst_pos_space) + 3
    dst_caches = []
    for g in range(c["dst_groups"]):
        if c["dst_layout"] == "flat":  # a session store: slot = position
            shape = (dst_pos_space[g] + int(rng.integers(1, 30)), heads, 2 * d)
        else:
            shape = _paged_shape(dst_blocks, c["dst_layout"], bs, heads, d)
        dst_caches.append([randn(shape, dtype, gen, sc) for _ in range(layers)])
    dst_tabs = [rng.permutation(dst_blocks).astype(np.int64) for _ in range(c["dst_groups"])]

    rows, dst_index_parts, d_off = [], [], 0
    for sp, dp, n, delta, g, dg in raw:
        s_idx = src_tab_off[g] if c["src_layout"] != "flat" else 0
        if c["dst_mode"] == "slots":
            pos = np.arange(dp, dp + n)
            dst_index_parts.append(dst_tabs[dg][pos // bs] * bs + pos % bs)
            rows.append((sp, 0, s_idx, d_off, n, delta, g, dg))
            d_off += n
        elif c["dst_mode"] == "flat":
            rows.append((sp, dp, s_idx, 0, n, delta, g, dg))
        else:
            rows.append((sp, dp, s_idx, dg * dst_blocks, n, delta, g, dg))
    if c["dst_mode"] == "slots":
        dst_index = torch.from_numpy(np.concatenate(dst_index_parts).astype(np.int64))
    elif c["dst_mode"] == "flat":
        dst_index = None
    else:
        dst_index = torch.from_numpy(np.concatenate(dst_tabs).astype(np.int32))
    src_index = (None if c["src_layout"] == "flat"
                 else torch.from_numpy(np.concatenate(src_tabs).astype(np.int32)))
    spans = span_array(rows)
    k_scale = (torch.from_numpy(rng.uniform(0.01, 0.1, layers).astype(np.float32)) if fp8
               else None)
    inv = inv_freq(c["rotary"]) if c["rotary"] else None

    src_cs = _cache_set(src_caches, c["src_layout"], bs, c["src_split"], gpu)
    dst_cs = _cache_set(dst_caches, c["dst_layout"], bs, c["dst_split"], gpu)
    plans = [ShiftPlan(spans, src_cs, dst_cs, inv_freq=inv,
                       src_mode="flat" if c["src_layout"] == "flat" else "table",
                       src_index=src_index, dst_mode=c["dst_mode"], dst_index=dst_index,
                       k_scale=k_scale, direct=direct, order=order)
             for direct, order in ((False, "none"), (False, "dst_page"),
                                   (False, "dst_page_device"), (True, None))]
    src_o = oracle_side(src_cs, "flat" if c["src_layout"] == "flat" else "table", src_index)
    dst_o = oracle_side(dst_cs, c["dst_mode"], dst_index)
    return plans, dst_cs, spans, src_o, dst_o, inv, k_scale


@pytest.mark.parametrize("seed", range(max(48, _EXTRA)))
def test_random_batched_shift_matches_oracle(gpu, seed):
    """Each case runs four times from the same starting caches: the two-launch path
    (plan pass and workspace) in span order, in destination-page order sorted on the host
    (``token_order``) and sorted on the device, and the direct single-launch path, where
    the case is eligible for it (up to 63 spans, power-of-two blocks, heads a multiple of
    a wave's rows)."""
    c = _case(seed)
    desc = {k: (str(v) if k == "dtype" else v) for k, v in c.items() if k != "rng"}
    print(f"case random {desc}", flush=True)
    plans, dst_cs, spans, src_o, dst_o, inv, k_scale = _build(c, gpu)
    inv_np = np.zeros(0, np.float32) if inv is None else inv.numpy()
    orc.shift_spans(oracle_spans(spans), src_o, dst_o, inv_np, dname(c["dtype"]),
                    None if k_scale is None else k_scale.numpy())
    start = [[dst_cs.fused(g, layer).clone() for layer in range(dst_cs.layers)]
             for g in range(dst_cs.groups)]
    for plan in plans:
        _restore(dst_cs, start)
        flags = torch.zeros(1, dtype=torch.int32, device=gpu)
        plan.launch(error_flags=flags)
        torch.cuda.synchronize(gpu)
        assert int(flags.item()) == 0, plan.direct
        for g in range(dst_cs.groups):
            for layer in range(dst_cs.layers):
                assert np.array_equal(bits(dst_cs.fused(g, layer)), dst_o.caches[g][layer]), (
                    f"group {g} layer {layer} direct={plan.direct} order={plan.order}")


@pytest.mark.parametrize("seed", range(max(24, _EXTRA // 2)))
def test_random_single_span_matches_oracle(gpu, seed):
    """The per-layer entry point (``scatter_shifted``, the reference's signature) over
    random geometries: any element type, head size, rotary width, head count, layout and
    block size (16, 32 or 24, not a power of two); the source a view into a larger store
    buffer; distinct random destination slots; deltas of every magnitude."""
    from marathon_amd import rope_shift, scatter_shifted

    rng = np.random.default_rng(1000 + seed)
    dtype = DTYPES[seed % len(DTYPES)]
    d = int(rng.choice([64, 128, 256]))
    per_chunk = 16 // EB[dtype]
    rotary = int(rng.choice([r for r in (d // 2, d) if r % (2 * per_chunk) == 0]))
    heads = int(rng.choice([1, 2, 3, 4, 5, 8, 16]))
    bs = int(rng.choice([16, 32, 24]))
    hnd = bool(rng.integers(2))
    n = int(rng.integers(1, 300))
    delta = int(rng.choice([0, int(rng.integers(-64, 65)), int(rng.integers(-40000, 40001)),
                            int(rng.integers(-(2**31), 2**31))]))
    print(f"case random single span seed={seed} {dtype} d={d} rotary={rotary} heads={heads} "
          f"bs={bs} hnd={hnd} n={n} delta={delta}", flush=True)
    gen = torch.Generator().manual_seed(seed)
    sc = 0.05
    start = int(rng.integers(0, 50))
    buf = randn((start + n + int(rng.integers(0, 20)), heads, 2 * d), dtype, gen, sc)
    nblocks = -(-n // bs) + int(rng.integers(1, 8))
    shape = (nblocks, heads, bs, 2 * d) if hnd else (nblocks, bs, heads, 2 * d)
    kv = randn(shape, dtype, gen, sc)
    slots = torch.from_numpy(rng.permutation(nblocks * bs)[:n].astype(np.int64))
    fp8 = dtype == torch.float8_e4m3fn
    inv = inv_freq(rotary)
    kv_dev = kv.to(gpu)
    buf_dev = buf.to(gpu)
    scatter_shifted(buf_dev[start:start + n], kv_dev, slots.to(gpu), bs, hnd,
                    rope_shift(delta, d, inv, gpu), **({"k_scale": sc} if fp8 else {}))
    torch.cuda.synchronize(gpu)
    want = bits(kv)
    orc.scatter_shifted(bits(buf[start:start + n]), want, slots.numpy(), bs, hnd, delta,
                        inv.numpy(), dname(dtype), **({"k_scale": np.float32(sc)} if fp8 else {}))
    got = bits(kv_dev)
    assert np.array_equal(got, want), f"{int((got != want).sum())} elements differ"
