"""Worker-side load path of the shift connector, one HIP launch per engine step.

The reference's ``MarathonShiftConnector`` (src/marathon/vllm_shift_connector.py) runs,
for every load of a step and every layer, ``ShiftStore.read`` and one
``scatter_shifted`` launch (:481-534, loop at :505-518): 40 launches per load on
Qwen3-14B, plus per-layer Python.  :class:`ShiftLoader` keeps the same inputs -- the
``_Load`` list (:135-140), the registered paged caches (:393-412) and the session store
-- and issues the whole step as one batched launch (:class:`marathon_amd.spans.ShiftPlan`):
every load x every layer, sources read straight out of each session's store buffer.

Also here, as host logic: the layout detection of ``register_kv_caches`` (:393-402) and
the multi-segment block alignment of ``_accept_multi`` (:225-245).
"""

from __future__ import annotations

import logging
import time
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .shift_store import ShiftStore
from .spans import CacheSet, ShiftPlan

logger = logging.getLogger("marathon_amd.shift")


@dataclass
class Save:
    """One save of a step (vllm_shift_connector.py:143-151): the positions this step
    computed, ``slots`` in the paged cache, stored from ``dst_start``."""

    session: str
    slots: torch.Tensor  # int64 [T]
    dst_start: int


@dataclass
class Load:
    """One load of a step (vllm_shift_connector.py:135-140)."""

    session: str
    slots: torch.Tensor  # int64 [T]: destination slots of positions [lo, hi)
    src_start: int  # first source position in the session's store
    delta: int


def detect_hnd(shape, block_size: int) -> bool:
    """HND ``[blocks, heads, bs, 2D]`` vs NHD ``[blocks, bs, heads, 2D]``; an ambiguous
    shape is NHD, vLLM's default (vllm_shift_connector.py:396-402)."""
    assert len(shape) == 4, f"expected fused 4-D KV layout, got {tuple(shape)}"
    hnd = shape[2] == block_size and shape[1] != block_size
    if shape[1] == block_size and shape[2] == block_size:
        hnd = False
    return hnd


def accept_multi(loads: list, num_computed: int, num_prompt_tokens: int, block_size: int,
                 covers) -> list:
    """Block-align every segment of a multi-segment load (vllm_shift_connector.py:225-245).

    ``covers(src_start, n)`` is the store's coverage check.  A segment is dropped, never
    guessed at, when alignment leaves less than a block, when it lies inside what the
    engine already holds, or when the store lost its source.
    """
    limit = (num_prompt_tokens - 1) // block_size * block_size
    floor = -(-num_computed // block_size) * block_size
    out = []
    for ld in loads:
        delta = int(ld["delta"])
        lo = max(-(-int(ld["dst_start"]) // block_size) * block_size, floor)
        hi = min(int(ld["dst_end"]), limit) // block_size * block_size
        if hi - lo < block_size:
            continue
        if not covers(lo - delta, hi - lo):
            continue
        out.append({"dst_start": lo, "dst_end": hi, "delta": delta})
    return out


class ShiftLoader:
    """Loads reused spans from a :class:`ShiftStore` into registered paged caches."""

    def __init__(
        self,
        store: ShiftStore,
        block_size: int,
        inv_freq: torch.Tensor,
        *,
        k_scales: dict | None = None,
        timing: bool = False,
    ):
        self.store = store
        self.block_size = int(block_size)
        self.inv_freq = inv_freq.detach().to(torch.float32).cpu()
        self.k_scales = k_scales or {}
        self.timing = timing
        self._kv: dict[str, torch.Tensor] = {}
        self.hnd: bool | None = None
        self.head_size: int | None = None
        self.last_plan: ShiftPlan | None = None

    def register_kv_caches(self, kv_caches: dict) -> None:
        """Record the per-layer paged caches and their layout (:393-412)."""
        self._kv = dict(kv_caches)
        shape = next(iter(self._kv.values())).shape
        self.hnd = detect_hnd(shape, self.block_size)
        self.head_size = shape[3] // 2
        one = next(iter(self._kv.values()))
        if one.is_cuda:
            _lib.lib()  # the kernels are compiled ahead of time: only load the library

    def start_load_kv(self, loads: list) -> int:
        """Issue every load of the step as one launch; returns token-layers loaded.

        Mirrors :481-534: each (load, layer) source is ``store.read`` (so the store's
        counters and LRU order move exactly as in the reference), and a load whose
        source is missing for any layer is logged and ends the step's loading.
        Divergence: the reference has already written the layers before the missing
        one when it stops; here a missed load writes nothing.
        """
        if not loads or not self._kv:
            return 0
        names = list(self._kv)
        groups: dict[str, int] = {}
        rows = []
        slot_parts = []
        offset = 0
        for load in loads:
            n = int(load.slots.numel())
            if n == 0:
                continue
            missing = None
            for name in names:
                if self.store.read(load.session, name, load.src_start, n) is None:
                    missing = name
                    break
            if missing is not None:
                logger.error(
                    "shift: session %s has no stored KV for %s; load skipped", load.session, missing
                )
                break
            g = groups.setdefault(load.session, len(groups))
            rows.append((load.src_start, 0, 0, offset, n, int(load.delta), g, 0))
            slot_parts.append(load.slots.to(torch.int64).reshape(-1))
            offset += n
        if not rows:
            return 0
        src = CacheSet(
            [[self.store.buffer(s, name) for name in names] for s in groups], "flat"
        )
        dst = CacheSet([[self._kv[name] for name in names]], "hnd" if self.hnd else "nhd",
                       self.block_size)
        k_scale = None
        if dst.first.dtype == torch.float8_e4m3fn:
            k_scale = torch.tensor([float(self.k_scales.get(name, 1.0)) for name in names])
        spans = np.array(rows, dtype=_lib.SPAN_DTYPE)
        plan = ShiftPlan(
            spans,
            src,
            dst,
            inv_freq=self.inv_freq,
            src_mode="flat",
            dst_mode="slots",
            dst_index=torch.cat(slot_parts),
            k_scale=k_scale,
        )
        t0 = 0.0
        if self.timing:
            torch.cuda.synchronize(dst.first.device)
            t0 = time.perf_counter()
        plan.launch()
        self.last_plan = plan
        if self.timing:
            torch.cuda.synchronize(dst.first.device)
            ms = (time.perf_counter() - t0) * 1e3
            logger.info(
                "shift: %d loads, %d tokens x %d layers, copy_ms=%.3f (%.1f GB/s)",
                len(rows),
                offset,
                len(names),
                ms,
                plan.algorithmic_bytes / 1e9 / max(ms / 1e3, 1e-12),
            )
        return offset * len(names)


class ShiftSaver:
    """Save path: paged cache -> session store, gathered on the device.

    The reference's ``save_kv_layer`` (vllm_shift_connector.py:539-553) reserves the
    span, gathers ``[T, heads, 2D]`` with advanced indexing (``_gather``, :418-442) and
    copies it into the store buffer (``ShiftStore.write``, shift_store.py:225-236).
    Here the gather kernel reads the paged rows and writes them straight into each
    session's buffer (delta 0: a pure copy), one launch for every save of the call.
    """

    def __init__(self, store: ShiftStore, block_size: int):
        self.store = store
        self.block_size = int(block_size)
        self.last_plan: ShiftPlan | None = None

    def _plan(self, names: list, caches: list, saves: list) -> int:
        first = caches[0]
        hnd = detect_hnd(first.shape, self.block_size)
        row_shape = (first.shape[1] if hnd else first.shape[2], first.shape[3])
        groups: dict[str, int] = {}
        bufs: list[list] = []
        rows, slot_parts, offset = [], [], 0
        for save in saves:
            n = int(save.slots.numel())
            if n == 0:
                continue
            # mirrors the scheduler's reserve for this step; idempotent across layers
            if not self.store.reserve(save.session, save.dst_start, n):
                continue
            targets = [self.store.write_target(save.session, name, save.dst_start, n, row_shape,
                                               first.dtype, first.device) for name in names]
            if any(t is None for t in targets):
                continue
            g = groups.get(save.session)
            if g is None:
                g = groups[save.session] = len(bufs)
                bufs.append(targets)
            else:
                bufs[g] = targets  # a save may have grown (reallocated) the buffers
            rows.append((0, int(save.dst_start), offset, 0, n, 0, 0, g))
            slot_parts.append(save.slots.to(torch.int64).reshape(-1))
            offset += n
        if not rows:
            return 0
        plan = ShiftPlan(
            np.array(rows, dtype=_lib.SPAN_DTYPE),
            CacheSet([caches], "hnd" if hnd else "nhd", self.block_size),
            CacheSet(bufs, "flat"),
            inv_freq=None,
            src_mode="slots",
            src_index=torch.cat(slot_parts),
            dst_mode="flat",
        )
        plan.launch()
        self.last_plan = plan
        return offset * len(names)

    def save_kv_layer(self, layer_name: str, kv_layer: torch.Tensor, saves: list) -> int:
        """One layer, every save of the step (the reference's per-layer hook)."""
        return self._plan([layer_name], [kv_layer], saves)

    def save_all(self, kv_caches: dict, saves: list) -> int:
        """Every layer and every save of the step in one launch (at the end of a step)."""
        names = list(kv_caches)
        return self._plan(names, [kv_caches[n] for n in names], saves)
