"""Seeded synthetic shift workloads: the benchmark and parity workloads.

Shared geometry (Qwen3 KV): 8 KV heads, head_dim 128, full NeoX rotary, theta 1e6,
block_size 16.  Synthetic data (there is no checkpoint to load): K/V ~ N(0, 1) drawn
on the device from seeded generators.

1. Qwen3-0.6B-shaped, CPU: 28 layers, a flat store of 4,096 tokens, one span shifted
   by +37 into 259 destination blocks drawn from a seeded permutation of 512.
2. Qwen3-8B-shaped single span: 36 layers, history 16,384, span [512, 16384) ->
   [0, 15872) (delta -512), shuffled source and destination block tables.
3. Qwen3-14B-shaped multi-span: 40 layers, history 30,720, 8 spans of 256..8192
   tokens, deltas in [-2048, 2048] of both signs and one 0, no span boundary on a
   multiple of 16, disjoint and order-preserving, shuffled block tables.
4. The Qwen3-14B multi-span layout in fp8 e4m3fn with per-layer fp32 scales in
   [0.01, 0.1].
5. 32 sessions x 36 layers, histories in [2048, 32768], 1..6 spans per session,
   deltas in [-4096, 4096], one span table, one shared paged destination.

The source is the session store in block layout (read through a block table), as
:class:`~marathon_amd.block_store.BlockShiftStore` holds it for the element type
(``store_layout``): bf16 blocks as a K plane then a V plane, ``[blocks, 2, 16, heads,
D]``; fp8 blocks as rows of K then V per head, ``[blocks, 16, heads, 2D]``.
``src_layout`` picks either for any type.  The destination is an HND paged cache written through a slot mapping (workloads 2-4) or
through per-request block tables (workload 5).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from .block_store import store_layout
from .shift_kernels import inv_freq_for
from .shift_store import slots as slot_map
from .spans import CacheSet, ShiftPlan

HEADS, HEAD_SIZE, BLOCK, THETA = 8, 128, 16, 1e6


# ------------------------------------------------------------------ span layouts


@dataclass
class SpanLayout:
    src_start: np.ndarray
    dst_start: np.ndarray
    length: np.ndarray
    delta: np.ndarray
    src_history: int
    dst_history: int

    @property
    def tokens(self) -> int:
        return int(self.length.sum())


def multispan_layout(
    rng: np.random.Generator,
    history: int,
    n_spans: int,
    len_lo: int,
    len_hi: int,
    delta_lo: int,
    delta_hi: int,
    *,
    need_zero: bool,
    need_mixed: bool,
    unaligned: bool,
    max_tries: int = 200000,
) -> SpanLayout:
    """Disjoint, order-preserving spans of an edited history, by seeded rejection.

    Source spans are laid out with at least one token between them; deltas are a
    random walk anchored at one span (delta 0 when ``need_zero``), each step bounded so
    the destination spans stay disjoint and in order.  ``unaligned`` rejects any span
    whose length, source start or destination start is a multiple of 16.
    """
    for _ in range(max_tries):
        lens = rng.integers(len_lo, len_hi + 1, n_spans)
        if unaligned:
            lens = np.where(lens % 16 == 0, np.where(lens < len_hi, lens + 1, lens - 1), lens)
        free = history - int(lens.sum())
        if free < n_spans + 1:
            continue
        cuts = np.sort(rng.choice(free - 1, n_spans, replace=False) + 1)
        gaps = np.diff(np.concatenate(([0], cuts, [free])))  # n_spans + 1 gaps, >= 1
        src = gaps[0] + np.concatenate(([0], np.cumsum(lens[:-1] + gaps[1:-1])))
        if unaligned and np.any(src % 16 == 0):
            continue
        z = int(rng.integers(n_spans))
        d = np.zeros(n_spans, np.int64)
        d[z] = 0 if need_zero else int(rng.integers(delta_lo, delta_hi + 1))
        ok = True
        for k in range(z + 1, n_spans):  # dst gap k stays >= 1
            lo = max(delta_lo, int(d[k - 1]) + 1 - int(gaps[k]))
            if lo > delta_hi:
                ok = False
                break
            d[k] = rng.integers(lo, delta_hi + 1)
        for k in range(z - 1, -1, -1):
            hi = min(delta_hi, int(d[k + 1]) - 1 + int(gaps[k + 1]))
            lo = max(delta_lo, -int(src[0])) if k == 0 else delta_lo
            if lo > hi:
                ok = False
                break
            d[k] = rng.integers(lo, hi + 1)
        if not ok:
            continue
        if need_zero and not np.any(d == 0):
            continue
        if need_mixed and not (np.any(d > 0) and np.any(d < 0)):
            continue
        dst = src + d
        if dst.min() < 0 or np.any(dst[1:] < (dst + lens)[:-1]):
            continue
        if unaligned and np.any(dst % 16 == 0):
            continue
        dst_hist = int(max(history, int((dst + lens).max()) + int(gaps[-1])))
        return SpanLayout(src.astype(np.int64), dst.astype(np.int64), lens.astype(np.int64),
                          d, history, dst_hist)
    raise RuntimeError("no span layout found; constraints too tight")


def qwen3_14b_multispan_layout(seed: int = 3, history: int = 30720) -> SpanLayout:
    rng = np.random.default_rng(seed)
    lo, hi = (256, 8192) if history >= 30720 else (max(17, history // 120), max(33, history // 4))
    return multispan_layout(rng, history, 8, lo, hi, -2048, 2048, need_zero=True,
                            need_mixed=True, unaligned=True)


# ------------------------------------------------------------- device workloads


@dataclass
class Workload:
    """A device-resident shift: caches, span table, index arrays -- ready to plan."""

    name: str
    spans: np.ndarray
    src: CacheSet
    dst: CacheSet
    src_mode: str
    src_index: torch.Tensor | None
    dst_mode: str
    dst_index: torch.Tensor | None
    inv_freq: torch.Tensor
    k_scale: torch.Tensor | None = None
    v_scale: torch.Tensor | None = None
    meta: dict = field(default_factory=dict)

    def plan(self, direct: bool | None = None, order: str | None = None) -> ShiftPlan:
        return ShiftPlan(
            self.spans,
            self.src,
            self.dst,
            inv_freq=self.inv_freq,
            src_mode=self.src_mode,
            src_index=self.src_index,
            dst_mode=self.dst_mode,
            dst_index=self.dst_index,
            k_scale=self.k_scale,
            direct=direct,
            order=order,
        )

    @property
    def tokens(self) -> int:
        return int(self.spans["n_tokens"].sum())

    @property
    def layers(self) -> int:
        return self.dst.layers

    @property
    def algorithmic_bytes(self) -> int:
        eb = self.dst.first.element_size()
        return 2 * self.tokens * self.layers * self.dst.heads * 2 * self.dst.head_size * eb


def fp8_layer_scales(seed: int, layers: int) -> tuple[np.ndarray, np.ndarray]:
    """Per-layer fp32 K and V scales of an fp8 workload, uniform in [0.01, 0.1]."""
    srng = np.random.default_rng(seed)
    k = srng.uniform(0.01, 0.1, layers).astype(np.float32)
    v = srng.uniform(0.01, 0.1, layers).astype(np.float32)
    return k, v


def _randn_cache(shape, dtype, gen, device, scale=None) -> torch.Tensor:
    if dtype == torch.float8_e4m3fn:
        x = torch.randn(shape, dtype=torch.float32, device=device, generator=gen)
        x = (x / float(scale)).clamp_(-448.0, 448.0)
        return x.to(torch.float8_e4m3fn)
    return torch.randn(shape, dtype=dtype, device=device, generator=gen)


def _paged(blocks, layout, heads=HEADS):
    return (blocks, heads, BLOCK, 2 * HEAD_SIZE) if layout == "hnd" else (blocks, BLOCK, heads, 2 * HEAD_SIZE)


#: Block layouts of a session store: ``"planes"`` -- a K plane then a V plane per
#: block, ``[blocks, 2, 16, heads, D]`` (the block store's pool); ``"fused"`` -- rows of
#: K then V per head, ``[blocks, 16, heads, 2D]``.
STORE_LAYOUTS = ("planes", "fused")


def store_blocks(blocks: int, heads: int, dtype, gen, device, k_scale=None, v_scale=None,
                 layout: str = "planes", block: int = BLOCK) -> torch.Tensor:
    """One layer of a session store: ``blocks`` blocks of ``block`` tokens of N(0, 1) K
    and V (fp8: divided by the layer's K and V scales) in ``layout``."""
    if layout not in STORE_LAYOUTS:
        raise ValueError(f"store layout {layout!r}")
    plane = (blocks, block, heads, HEAD_SIZE)
    if dtype != torch.float8_e4m3fn:
        if layout == "planes":
            return _randn_cache((blocks, 2, block, heads, HEAD_SIZE), dtype, gen, device)
        return _randn_cache((blocks, block, heads, 2 * HEAD_SIZE), dtype, gen, device)
    k = _randn_cache(plane, dtype, gen, device, k_scale)
    v = _randn_cache(plane, dtype, gen, device, v_scale)
    return torch.stack((k, v), dim=1) if layout == "planes" else torch.cat((k, v), dim=-1)


def store_cache_set(groups: list, layout: str = "planes", block: int = BLOCK) -> CacheSet:
    """A :class:`CacheSet` over ``groups[group][layer]`` tensors from :func:`store_blocks`."""
    if layout == "planes":
        return CacheSet([[t[:, 0] for t in row] for row in groups], "nhd", block,
                        v_caches=[[t[:, 1] for t in row] for row in groups])
    return CacheSet(groups, "nhd", block)


def single_session_workload(
    name: str,
    layout: SpanLayout,
    layers: int,
    device,
    *,
    seed: int,
    dtype=torch.bfloat16,
    scale_seed: int | None = None,
    spare_blocks: int = 64,
    dst_fill: str = "zeros",
    heads: int = HEADS,
    src_layout: str | None = None,
    src_block: int = BLOCK,
) -> Workload:
    """One session's store (blocks in ``src_layout``, via a shuffled table) -> one HND
    paged cache via a slot mapping: the single-span and multi-span workloads, bf16 or
    fp8.  ``heads`` below 8 is one GPU's share of the KV heads under tensor
    parallelism.  ``src_layout``: ``"planes"`` or ``"fused"`` (default: the block store's
    layout for ``dtype``).  ``src_block``: tokens per store block (the store's own
    choice; the destination keeps vLLM's 16)."""
    src_layout = src_layout or store_layout(dtype)
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    src_blocks = -(-layout.src_history // src_block)
    dst_need = -(-layout.dst_history // BLOCK)
    dst_pool = dst_need + spare_blocks
    src_table = rng.permutation(src_blocks).astype(np.int32)
    dst_table = rng.permutation(dst_pool)[:dst_need].astype(np.int64)
    k_scale = v_scale = None
    if dtype == torch.float8_e4m3fn:
        k, v = fp8_layer_scales(scale_seed if scale_seed is not None else seed, layers)
        k_scale, v_scale = torch.from_numpy(k), torch.from_numpy(v)
    src_caches, dst_caches = [], []
    for layer in range(layers):
        fp8 = dtype == torch.float8_e4m3fn
        src_caches.append(store_blocks(src_blocks, heads, dtype, gen, device,
                                       k_scale[layer] if fp8 else None,
                                       v_scale[layer] if fp8 else None, src_layout,
                                       src_block))
        if dst_fill == "random" and dtype != torch.float8_e4m3fn:
            dst_caches.append(_randn_cache(_paged(dst_pool, "hnd", heads), dtype, gen, device))
        else:
            dst_caches.append(torch.zeros(_paged(dst_pool, "hnd", heads), dtype=dtype,
                                          device=device))
    dst_slots, rows, off = [], [], 0
    for s, d, n, dl in zip(layout.src_start, layout.dst_start, layout.length, layout.delta):
        dst_slots.append(slot_map(dst_table, int(d), int(d + n), BLOCK))
        rows.append((int(s), int(d), 0, off, int(n), int(dl), 0, 0))
        off += int(n)
    spans = np.array(rows, dtype=_lib.SPAN_DTYPE)
    return Workload(
        name,
        spans,
        store_cache_set([src_caches], src_layout, src_block),
        CacheSet([dst_caches], "hnd", BLOCK),
        "table",
        torch.from_numpy(src_table),
        "slots",
        torch.cat(dst_slots),
        inv_freq_for(HEAD_SIZE, THETA),
        k_scale,
        v_scale,
        {"src_table": src_table, "dst_table": dst_table, "layout": layout},
    )


def qwen3_8b_single_span(device, layers: int = 36, history: int = 16384, seed: int = 2, **kw) -> Workload:
    cut = 512 * history // 16384
    lay = SpanLayout(np.array([cut]), np.array([0]), np.array([history - cut]),
                     np.array([-cut]), history, history - cut)
    return single_session_workload("qwen3-8b single span", lay, layers, device, seed=seed, **kw)


def qwen3_14b_multispan(device, layers: int = 40, history: int = 30720, seed: int = 3, **kw) -> Workload:
    lay = qwen3_14b_multispan_layout(seed, history)
    return single_session_workload("qwen3-14b multi-span", lay, layers, device, seed=seed, **kw)


def qwen3_14b_multispan_fp8(device, layers: int = 40, history: int = 30720, **kw) -> Workload:
    lay = qwen3_14b_multispan_layout(3, history)
    return single_session_workload("qwen3-14b multi-span fp8", lay, layers, device, seed=4,
                                   dtype=torch.float8_e4m3fn, scale_seed=4, **kw)


def batched_sessions_layouts(seed: int = 5, sessions: int = 32, hist_lo: int = 2048,
                    hist_hi: int = 32768) -> list:
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(sessions):
        h = int(rng.integers(hist_lo, hist_hi + 1))
        n = int(rng.integers(1, 7))
        len_hi = max(2, int(0.9 * h / n))
        lay = multispan_layout(rng, h, n, max(1, len_hi // 8), len_hi, -4096, 4096,
                               need_zero=False, need_mixed=False, unaligned=False)
        out.append(lay)
    return out


def batched_sessions(device, layers: int = 36, seed: int = 5, sessions: int = 32, hist_lo: int = 2048,
            hist_hi: int = 32768, dtype=torch.bfloat16, heads: int = HEADS) -> Workload:
    """32 sessions, each its own store (group), one shared HND destination pool; both
    sides addressed through block tables, so the slot math runs on the device.  fp8:
    per-layer K and V scales shared by the sessions."""
    lays = batched_sessions_layouts(seed, sessions, hist_lo, hist_hi)
    rng = np.random.default_rng(seed + 1000)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    dst_need = [-(-lay.dst_history // BLOCK) for lay in lays]
    pool = int(sum(dst_need)) + 64
    perm = rng.permutation(pool).astype(np.int32)
    fp8 = dtype == torch.float8_e4m3fn
    k_scale = v_scale = None
    if fp8:
        k, v = fp8_layer_scales(seed, layers)
        k_scale, v_scale = torch.from_numpy(k), torch.from_numpy(v)
    src_tables, dst_tables, src_caches, rows = [], [], [], []
    s_off = d_off = 0
    for g, lay in enumerate(lays):
        nb = -(-lay.src_history // BLOCK)
        src_tables.append(rng.permutation(nb).astype(np.int32))
        dst_tables.append(perm[d_off : d_off + dst_need[g]])
        src_caches.append([store_blocks(nb, heads, dtype, gen, device,
                                        k_scale[layer] if fp8 else None,
                                        v_scale[layer] if fp8 else None,
                                        layout=store_layout(dtype))
                           for layer in range(layers)])
        for s, d, n, dl in zip(lay.src_start, lay.dst_start, lay.length, lay.delta):
            rows.append((int(s), int(d), s_off, d_off, int(n), int(dl), g, 0))
        s_off += nb
        d_off += dst_need[g]
    dst_caches = [torch.zeros(_paged(pool, "hnd", heads), dtype=dtype, device=device)
                  for _ in range(layers)]
    return Workload(
        "batched restore",
        np.array(rows, dtype=_lib.SPAN_DTYPE),
        store_cache_set(src_caches, store_layout(dtype)),
        CacheSet([dst_caches], "hnd", BLOCK),
        "table",
        torch.from_numpy(np.concatenate(src_tables)),
        "table",
        torch.from_numpy(np.concatenate(dst_tables)),
        inv_freq_for(HEAD_SIZE, THETA),
        k_scale,
        v_scale,
        meta={"layouts": lays, "src_tables": src_tables, "dst_tables": dst_tables},
    )


# ------------------------------------------------------ the CPU reference workload


def qwen3_0_6b_cpu_shift(layers: int = 28, n: int = 4096, delta: int = 37, seed: int = 1):
    """Flat store rows per layer and an HND paged cache per layer, on the CPU."""
    gen = torch.Generator().manual_seed(seed)
    src = [torch.randn(n, HEADS, 2 * HEAD_SIZE, dtype=torch.bfloat16, generator=gen)
           for _ in range(layers)]
    pool = 512
    need = -(-(n + delta) // BLOCK)
    table = torch.randperm(pool, generator=gen)[:need]
    kv = [torch.zeros(pool, HEADS, BLOCK, 2 * HEAD_SIZE, dtype=torch.bfloat16)
          for _ in range(layers)]
    slots = slot_map(table.tolist(), delta, delta + n, BLOCK)
    return {"src": src, "kv": kv, "slots": slots, "delta": delta,
            "inv_freq": inv_freq_for(HEAD_SIZE, THETA), "table": table}
