"""Caches of more than 4 GiB per layer, with rows past byte offset 2^32 on both sides.

On one 288 GB MI355X a serving engine gives each layer's paged cache several GB (40
layers sharing 250 GB hold about 6 GB each), so every row offset the kernels form must be
64-bit.  Each case puts spans on blocks above and below the 4 GiB mark of the source and
destination caches (bf16 blocks of 64 KB: block 65,536 starts at byte 2^32; fp8 blocks
of 32 KB: block 131,072), runs one path of the library, checks every written row against
the oracle, and counts the untouched elements of every destination cache -- filled
beforehand with a NaN pattern that no shifted row holds -- to show that nothing else was
written.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from marathon_amd import rope_shift, scatter_shifted
from marathon_amd.spans import CacheSet, ShiftPlan, SmallShifts, span_array
from oracle import kvshift_oracle as orc
from tests.helpers import TORCH_BITS, inv_freq

pytestmark = pytest.mark.gpu

HEADS, D, BS = 8, 128, 16
LAYERS = 2
SENTINEL = {torch.bfloat16: 0x7FC1, torch.float8_e4m3fn: 0x7F}  # NaN codes


def _blocks_past_4gib(dtype) -> int:
    """Blocks per layer so that the last 1,024 start beyond byte 2^32."""
    block_bytes = BS * HEADS * 2 * D * torch.empty(0, dtype=dtype).element_size()
    return (1 << 32) // block_bytes + 1024


def _tables(rng, nblocks: int, need: int) -> np.ndarray:
    """`need` distinct block ids, half from the last 1,024 blocks (past 4 GiB), half from
    the first 1,024, in random order."""
    hi = rng.choice(np.arange(nblocks - 1024, nblocks), need - need // 2, replace=False)
    lo = rng.choice(np.arange(1024), need // 2, replace=False)
    return rng.permutation(np.concatenate([hi, lo])).astype(np.int32)


# (src_pos, dst_pos, n_tokens, delta): unaligned, one span of each sign of delta
SPANS = [(5, 42, 300, 37), (400, 380, 200, -20), (650, 650, 110, 0)]
SRC_BLOCKS = 48  # source positions < 768
DST_BLOCKS = 48  # destination positions < 768


class Big:
    """Source NHD block store and destination HND cache of LAYERS layers, each more
    than 4 GiB, with block tables that mix blocks below and above 2^32 bytes."""

    def __init__(self, dev, dtype, layers: int, seed: int):
        self.dev, self.dtype, self.layers = dev, dtype, layers
        self.nblocks = _blocks_past_4gib(dtype)
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        self.src = [self._random((self.nblocks, BS, HEADS, 2 * D), gen)
                    for _ in range(layers)]
        self.dst = [torch.empty(self.nblocks, HEADS, BS, 2 * D, dtype=dtype, device=dev)
                    for _ in range(layers)]
        rng = np.random.default_rng(seed)
        self.src_table = _tables(rng, self.nblocks, SRC_BLOCKS)
        self.dst_table = _tables(rng, self.nblocks, DST_BLOCKS)
        self.k_scale = (torch.from_numpy(rng.uniform(0.01, 0.1, layers).astype(np.float32))
                        if dtype == torch.float8_e4m3fn else None)

    def _random(self, shape, gen) -> torch.Tensor:
        """Random finite values, filled in slices of 2^28 elements (no float32 copy of a
        whole 4 GiB cache)."""
        out = torch.empty(shape, dtype=self.dtype, device=self.dev)
        flat = out.view(-1)
        step = 1 << 28
        for a in range(0, flat.numel(), step):
            x = torch.randn(min(step, flat.numel() - a), device=self.dev, generator=gen)
            if self.dtype == torch.float8_e4m3fn:
                x = (x * 8).clamp(-448, 448)
            flat[a:a + x.numel()] = x.to(self.dtype)
        return out

    def reset(self) -> None:
        iv = TORCH_BITS[self.dtype][0]
        for t in self.dst:
            t.view(iv).fill_(SENTINEL[self.dtype])

    def src_rows(self, spans=SPANS):
        """Per span: source (block, offset) of every token in the block store."""
        return [(self.src_table[np.arange(s, s + n) // BS], np.arange(s, s + n) % BS)
                for s, _, n, _ in spans]

    def dst_rows(self, spans=SPANS):
        """Per span: destination (block, offset) of every token."""
        return [(self.dst_table[np.arange(d, d + n) // BS], np.arange(d, d + n) % BS)
                for _, d, n, _ in spans]

    def check(self, spans=SPANS, src_rows=None) -> None:
        """Every written row against the oracle; every other element still the sentinel.

        ``src_rows(layer, span_index)``: the source rows of a span ([n, heads, 2D]) when
        the source is not the block store."""
        torch.cuda.synchronize(self.dev)
        iv, nv, name = TORCH_BITS[self.dtype]
        inv = inv_freq().numpy()
        on = lambda a: torch.from_numpy(a).long().to(self.dev)  # noqa: E731
        for layer in range(self.layers):
            written = 0
            for i, (db, do) in enumerate(self.dst_rows(spans)):
                if src_rows is None:
                    sb, so = self.src_rows(spans)[i]
                    src = self.src[layer][on(sb), on(so)]
                else:
                    src = src_rows(layer, i)
                got = self.dst[layer][on(db), :, on(do)]  # HND row of each token
                sbits = src.cpu().view(iv).numpy().view(nv)
                gbits = got.cpu().view(iv).numpy().view(nv)
                scale = None if self.k_scale is None else float(self.k_scale[layer])
                delta = spans[i][3]
                want_k = orc.rotate_k_bits(sbits[..., :D], delta, inv, name, scale)
                assert np.array_equal(gbits[..., :D], want_k), f"K layer {layer} span {i}"
                assert np.array_equal(gbits[..., D:], sbits[..., D:]), f"V layer {layer} span {i}"
                written += sbits.size
            kept = int((self.dst[layer].view(iv) == SENTINEL[self.dtype]).sum())
            assert self.dst[layer].numel() - kept == written, (
                f"layer {layer}: {self.dst[layer].numel() - kept} elements changed, "
                f"{written} written")

    def cache_sets(self):
        return CacheSet([self.src], "nhd", BS), CacheSet([self.dst], "hnd", BS)


@pytest.fixture(scope="module")
def big_bf16(gpu):
    b = Big(gpu, torch.bfloat16, LAYERS, seed=41)
    yield b
    del b
    torch.cuda.empty_cache()


def _table_plan(b: Big, **kw) -> ShiftPlan:
    spans = span_array([(s, d, 0, 0, n, delta, 0, 0) for s, d, n, delta in SPANS])
    src, dst = b.cache_sets()
    return ShiftPlan(spans, src, dst, inv_freq=inv_freq(), src_mode="table",
                     src_index=torch.from_numpy(b.src_table), dst_mode="table",
                     dst_index=torch.from_numpy(b.dst_table), k_scale=b.k_scale, **kw)


@pytest.mark.parametrize("path", ["two-launch", "direct", "dst_page order"])
def test_block_tables_past_4gib(gpu, big_bf16, path):
    print(f"case >4GiB caches, block tables, {path}", flush=True)
    b = big_bf16
    b.reset()
    kw = {"direct": path == "direct"}
    if path == "dst_page order":
        kw["order"] = "dst_page"
    plan = _table_plan(b, **kw)
    assert plan.direct == (path == "direct")
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    plan.launch(error_flags=flags)
    b.check()
    assert int(flags.item()) == 0


@pytest.mark.parametrize("direct", [False, True])
def test_slots_into_a_cache_past_4gib(gpu, big_bf16, direct):
    print(f"case >4GiB caches, destination slots, direct={direct}", flush=True)
    b = big_bf16
    b.reset()
    dst_slots = np.concatenate([db.astype(np.int64) * BS + do for db, do in b.dst_rows()])
    idx = np.cumsum([0] + [n for _, _, n, _ in SPANS])
    spans = span_array([(s, d, 0, int(idx[i]), n, delta, 0, 0)
                        for i, (s, d, n, delta) in enumerate(SPANS)])
    src, dst = b.cache_sets()
    plan = ShiftPlan(spans, src, dst, inv_freq=inv_freq(), src_mode="table",
                     src_index=torch.from_numpy(b.src_table), dst_mode="slots",
                     dst_index=torch.from_numpy(dst_slots), direct=direct)
    assert plan.direct == direct
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    plan.launch(error_flags=flags)
    b.check()
    assert int(flags.item()) == 0


def test_small_shift_past_4gib(gpu, big_bf16):
    """The small path: spans and table windows in the launch's own arguments."""
    print("case >4GiB caches, small path", flush=True)
    b = big_bf16
    b.reset()
    src, dst = b.cache_sets()
    runner = SmallShifts(src, dst, inv_freq=inv_freq(), src_mode="table", dst_mode="table")
    rows = [(s, d, 0, 0, n, delta, 0, 0) for s, d, n, delta in SPANS]
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    runner.run(rows, b.src_table, b.dst_table, error_flags=flags)
    assert runner._last == (True,), "expected the launch-argument path"
    b.check()
    assert int(flags.item()) == 0


@pytest.mark.parametrize("direct", [False, True])
def test_flat_source_past_4gib(gpu, big_bf16, direct):
    """A flat store whose rows past 2^32 bytes are read (token 1,048,576 starts there)."""
    print(f"case >4GiB flat source, direct={direct}", flush=True)
    b = big_bf16
    b.reset()
    row_bytes = HEADS * 2 * D * 2
    first = (1 << 32) // row_bytes - 400  # spans straddle the 4 GiB mark
    n_flat = first + 1024
    gen = torch.Generator(device=gpu)
    gen.manual_seed(5)
    flat = []
    for _ in range(LAYERS):
        t = torch.empty(n_flat, HEADS, 2 * D, dtype=torch.bfloat16, device=gpu)
        t[first:] = torch.randn(n_flat - first, HEADS, 2 * D, device=gpu,
                                generator=gen).to(torch.bfloat16)
        flat.append(t)
    spans_flat = [(first + s, d, n, delta) for s, d, n, delta in SPANS]
    spans = span_array([(s, d, 0, 0, n, delta, 0, 0) for s, d, n, delta in spans_flat])
    _, dst = b.cache_sets()
    plan = ShiftPlan(spans, CacheSet([flat], "flat"), dst, inv_freq=inv_freq(),
                     src_mode="flat", dst_mode="table", dst_index=torch.from_numpy(b.dst_table),
                     direct=direct)
    assert plan.direct == direct
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    plan.launch(error_flags=flags)
    b.check(spans_flat, src_rows=lambda layer, i: flat[layer][
        spans_flat[i][0]:spans_flat[i][0] + spans_flat[i][2]])
    assert int(flags.item()) == 0
    del flat, plan
    torch.cuda.empty_cache()


def test_per_layer_scatter_past_4gib(gpu, big_bf16):
    """The reference's per-layer call (scatter_shifted) with slots past 2^32 bytes."""
    print("case >4GiB caches, scatter_shifted", flush=True)
    b = big_bf16
    b.reset()
    src_rows = {}
    for layer in range(LAYERS):
        for i, ((sb, so), (db, do)) in enumerate(zip(b.src_rows(), b.dst_rows())):
            src = b.src[layer][torch.from_numpy(sb).long().to(gpu),
                               torch.from_numpy(so).long().to(gpu)].contiguous()
            src_rows[layer, i] = src
            slots_t = torch.from_numpy(db.astype(np.int64) * BS + do).to(gpu)
            delta = SPANS[i][3]
            shift = rope_shift(delta, D, inv_freq(), gpu) if delta else None
            scatter_shifted(src, b.dst[layer], slots_t, BS, True, shift)
    b.check(src_rows=lambda layer, i: src_rows[layer, i])


@pytest.mark.parametrize("direct", [False, True])
def test_fp8_block_tables_past_4gib(gpu, direct):
    print(f"case >4GiB fp8 caches, block tables, direct={direct}", flush=True)
    b = Big(gpu, torch.float8_e4m3fn, 1, seed=43)
    try:
        b.reset()
        plan = _table_plan(b, direct=direct)
        assert plan.direct == direct
        flags = torch.zeros(1, dtype=torch.int32, device=gpu)
        plan.launch(error_flags=flags)
        b.check()
        assert int(flags.item()) == 0
    finally:
        del b
        torch.cuda.empty_cache()
