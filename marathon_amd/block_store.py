"""Block-layout session store: fixed 16-token blocks of one preallocated pool per layer.

The reference's ``ShiftStore`` (src/marathon/shift_store.py:101-266) keeps each session
in a flat ``[capacity, heads, 2D]`` buffer per layer.  It grows by geometric realloc plus
a copy of everything already stored (``_grow``, :149-175), and it has one validity window
``[base, filled)``: a save at or below ``filled`` truncates everything above it.  That
window is why the generation-0 address book (src/marathon/remap.py) cannot be wired:
under no-resave, the gaps between reused spans are saved at lower indices, and each such
save destroys the bytes the remap addresses higher up (docs/single-request-load.md,
"Design 2"; src/marathon/server.py:267-276 raises for it).

:class:`BlockShiftStore` keeps the reference's API (``reserve`` / ``covers`` / ``write``
/ ``read`` / ``drop`` / ``stats``, the same return values and counters) over a different
memory layout:

* **Pool.** Per layer, one device tensor allocated once on the layer's first save, in
  the block layout the kernels move fastest for its element size (:func:`store_layout`):
  * 2- and 4-byte elements: ``[pool_blocks, 2, block_size, heads, D]``, each block a K
    plane then a V plane, each ``[block_size, heads, D]`` (NHD).  A token's K rows of
    all heads are one contiguous run, and so are its V rows.  On the Qwen3-14B
    multi-span shift (bf16) the kernel reads this layout 3.3% faster than rows that
    interleave K and V per head, and a save writes it about 3% faster.
  * 1-byte elements (fp8): ``[pool_blocks, block_size, heads, 2D]``, rows of K then V
    per head.  For fp8 that layout reads 0.6% faster than planes.

  The HIP kernels read and write the pool through block tables (``MKV_ADDR_TABLE``):
  the planes as split K and V caches, the rows as fused ones (:meth:`kernel_views`).  A
  session owns a block table: logical block ``k`` holds positions ``[k*bs, (k+1)*bs)``.
* **Allocator.** Growth takes blocks from a free list, lowest ids first, so that a
  session's blocks tend to form contiguous runs.  No byte is ever copied to grow.  An
  evicted or dropped session returns its blocks.  Eviction is whole sessions in LRU
  order, never the session being written, as in the reference.
* **Validity, two policies.**
  * ``truncate=True`` (default) is the reference's rule, bit for bit.  The scheduler
    mirror and the worker reach the same decisions as with ``ShiftStore``: a start above
    ``filled`` is refused as a hole, and a start at or below it drops everything above
    the new top.  The blocks above are freed, not copied.
  * ``truncate=False`` gives per-position validity: a sorted set of disjoint intervals.
    A save marks its range valid and touches nothing else, holes are allowed, and
    ``covers`` answers for every position of the range.  Generation-0 reuse
    (no-resave) needs this.  It is not sufficient on its own: after the text shrinks,
    new text saved at its own index can land on a drifted span's generation-0 bytes,
    so fresh KV must also be placed away from every drifted span's source.
* **Budget.** Counted in blocks actually held (``used`` = blocks x ``block_size``), not
  in doubled capacity.  For the same sessions the block store evicts no more often than
  the flat store.

``write`` takes and ``read`` returns rows ``[n, heads, 2D]`` (K then V), as the
reference's store does; ``read`` gathers a copy, since a block layout has no contiguous
view.  The hot path never calls either: the loader and the saver move the pool's blocks
through the session's block table in the launch that rotates (:meth:`table`,
:meth:`kernel_views`).
"""

from __future__ import annotations

import bisect
import heapq
from dataclasses import dataclass, field

import numpy as np
import torch

from .shift_store import DEFAULT_STORE_TOKENS
from .store_core import StoreCore, Window


def store_layout(dtype) -> str:
    """The pool's block layout for elements of ``dtype``: ``"planes"`` (a K plane then a
    V plane per block) for 2- and 4-byte elements, ``"fused"`` (rows of K then V per
    head) for 1-byte ones -- the faster of the two for each, measured on the Qwen3-14B
    multi-span shift."""
    return "planes" if torch.empty(0, dtype=dtype).element_size() >= 2 else "fused"


def _no_blocks() -> np.ndarray:
    return np.zeros(0, dtype=np.int32)


@dataclass
class _BlockEntry(Window):
    """A session's blocks; under the truncate policy the window ``[base, filled)`` (from
    :class:`~marathon_amd.store_core.Window`) says what is held, under the interval
    policy ``valid`` does."""

    table: np.ndarray = field(default_factory=_no_blocks)  # logical block -> pool id (-1: none)
    held: int = 0  # pool blocks this session owns
    valid: list = field(default_factory=list)  # interval policy: sorted disjoint [lo, hi)
    layers: set = field(default_factory=set)  # layers saved at least once


def _add_interval(ivs: list, lo: int, hi: int) -> None:
    """Insert ``[lo, hi)`` into sorted disjoint intervals, merging neighbours."""
    i = bisect.bisect_left(ivs, (lo, lo))
    if i > 0 and ivs[i - 1][1] >= lo:
        i -= 1
    j = i
    while j < len(ivs) and ivs[j][0] <= hi:
        lo, hi = min(lo, ivs[j][0]), max(hi, ivs[j][1])
        j += 1
    ivs[i:j] = [(lo, hi)]


def _covered(ivs: list, lo: int, hi: int) -> bool:
    i = bisect.bisect_right(ivs, (lo, float("inf"))) - 1
    return i >= 0 and ivs[i][0] <= lo and hi <= ivs[i][1]


class BlockShiftStore(StoreCore):
    """Session-keyed KV in ``block_size``-token blocks of a per-layer device pool."""

    def __init__(
        self,
        budget_tokens: int = DEFAULT_STORE_TOKENS,
        device: str = "cuda",
        allocate: bool = True,
        block_size: int = 16,
        truncate: bool = True,
    ) -> None:
        super().__init__(budget_tokens)
        self.block_size = int(block_size)
        if self.block_size <= 0 or self.budget <= 0:
            raise ValueError("budget_tokens and block_size must be positive")
        self.pool_blocks = -(-self.budget // self.block_size)
        self.device = device
        self.allocate = allocate
        self.truncate = bool(truncate)
        self._free = list(range(self.pool_blocks))  # a heap: lowest id first
        self._pools: dict[str, torch.Tensor] = {}
        self._sigs: dict[str, tuple] = {}  # layer -> (row shape, dtype) of its pool
        self._planar: dict[str, bool] = {}  # layer -> whether its pool holds K/V planes
        self._plane_lists: dict[tuple, tuple] = {}  # layers -> (pools existing, (k, v))
        self._target_lists: dict[tuple, tuple] = {}  # layers -> (pools existing, pools)
        self._sig_ok: dict[tuple, tuple] = {}  # layers -> the row signature all pools have

    # --------------------------------------------------------------- store hooks

    def _new_entry(self) -> _BlockEntry:
        return _BlockEntry()

    def _admits(self, entry: _BlockEntry, start: int, n: int) -> bool:
        return start >= 0 and (not self.truncate or entry.leaves_no_hole(start))

    def _make_room(self, session: str, entry: _BlockEntry, start: int, end: int) -> bool:
        return self._ensure_blocks(session, entry, start, end)

    def _commit(self, entry: _BlockEntry, start: int, end: int) -> None:
        if self.truncate:
            entry.extend(start, end)
            # everything above the new top is gone, as in the flat window: free it
            self._release(entry, -(-end // self.block_size), entry.table.size)
        else:
            _add_interval(entry.valid, start, end)

    def _holds(self, entry: _BlockEntry, start: int, n: int) -> bool:
        if n <= 0 or start < 0:
            return False
        if self.truncate:
            return entry.contains(start, n)
        return _covered(entry.valid, start, start + n)

    def _has_layer(self, entry: _BlockEntry, layer: str) -> bool:
        return layer in entry.layers

    def _has_layers(self, entry: _BlockEntry, layers) -> bool:
        return entry.layers.issuperset(layers)

    def _held_tokens(self, entry: _BlockEntry) -> int:
        if self.truncate:
            return entry.size
        return sum(hi - lo for lo, hi in entry.valid)

    def _forget(self, entry: _BlockEntry) -> None:
        self._release(entry, 0, entry.table.size)

    def _extra_stats(self) -> dict:
        return {"pool_blocks": self.pool_blocks, "free_blocks": len(self._free)}

    # ----------------------------------------------------------------- allocator

    @property
    def used(self) -> int:
        return (self.pool_blocks - len(self._free)) * self.block_size

    @property
    def free_blocks(self) -> int:
        return len(self._free)

    def _release(self, entry: _BlockEntry, lo_block: int, hi_block: int) -> None:
        if max(lo_block, 0) < min(hi_block, entry.table.size):
            part = entry.table[max(lo_block, 0):min(hi_block, entry.table.size)]
            freed = part[part >= 0]
            for b in freed.tolist():
                heapq.heappush(self._free, b)
            entry.held -= int(freed.size)
            part[:] = -1
        elif entry.table.size == 0 or entry.table[-1] >= 0:
            return  # nothing in the range and no unheld tail to trim (an append)
        live = np.flatnonzero(entry.table >= 0)
        entry.table = entry.table[: int(live[-1]) + 1 if live.size else 0]

    def _ensure_blocks(self, session: str, entry: _BlockEntry, lo: int, hi: int) -> bool:
        """Give ``session`` a block for every position in ``[lo, hi)``, evicting
        least-recently-used other sessions when the free list runs short."""
        bs = self.block_size
        k0, k1 = lo // bs, -(-hi // bs)
        if entry.table.size < k1:
            entry.table = np.concatenate(
                (entry.table, np.full(k1 - entry.table.size, -1, dtype=np.int32)))
        if k1 - k0 <= 2:  # a decode step's save: one or two blocks, no numpy needed
            missing = np.array([k for k in range(k0, k1) if entry.table[k] < 0], dtype=np.int64)
        else:
            missing = k0 + np.flatnonzero(entry.table[k0:k1] < 0)
        if not self._evict_until(session, lambda: len(self._free) >= missing.size):
            return False
        if missing.size:
            entry.table[missing] = [heapq.heappop(self._free) for _ in range(missing.size)]
        entry.held += int(missing.size)
        return True

    # -------------------------------------------------------------------- public

    def pool(self, layer: str) -> torch.Tensor | None:
        """The layer's pool (None before any save): ``[pool_blocks, 2, block_size, heads,
        D]`` (planes) or ``[pool_blocks, block_size, heads, 2D]`` (fused rows)."""
        return self._pools.get(layer)

    def kernel_views(self, layers) -> tuple:
        """``(caches, v_caches)``, the layers' pools as the kernels address them: with
        planes, the K planes and the V planes (views ``[pool_blocks, block_size, heads,
        D]``); with fused rows, the pools and None.  Two lists (None for a layer with no
        pool yet), reused while no pool changes: a step's loader and saver ask for the
        same layers every step."""
        key = tuple(layers)
        got = self._plane_lists.get(key)
        if got is None or got[0] != len(self._pools):
            pools = [self._pools.get(n) for n in key]
            planar = {self._planar[n] for n in key if n in self._planar}
            if len(planar) > 1:
                raise ValueError("these layers' pools mix block layouts")
            if planar == {True}:
                views = ([None if p is None else p[:, 0] for p in pools],
                         [None if p is None else p[:, 1] for p in pools])
            else:
                views = (pools, None)
            got = self._plane_lists[key] = (len(self._pools), views)
        return got[1]

    def _pool_for(self, layer: str, row_shape, dtype, device) -> torch.Tensor:
        sig = (tuple(row_shape), dtype)
        p = self._pools.get(layer)
        if p is None:
            *heads, two_d = sig[0]
            if two_d % 2:
                raise ValueError(f"layer {layer}: rows of {two_d} elements are not K and V halves")
            planar = store_layout(dtype) == "planes"
            if planar:
                shape = (self.pool_blocks, 2, self.block_size, *heads, two_d // 2)
            else:
                shape = (self.pool_blocks, self.block_size, *sig[0])
            p = torch.zeros(shape, dtype=dtype, device=device)
            self._pools[layer] = p
            self._sigs[layer] = sig
            self._planar[layer] = planar
        elif self._sigs[layer] != sig:
            raise ValueError(f"layer {layer}: rows {sig[0]} {dtype} do not match "
                             f"the pool's {self._sigs[layer][0]} {p.dtype}")
        return p

    def table(self, session: str) -> np.ndarray | None:
        """The session's block table (int32, -1 where no block is held; read-only)."""
        entry = self._sessions.get(session)
        if entry is None:
            return None
        view = entry.table.view()
        view.flags.writeable = False
        return view

    def _positions_ok(self, entry: _BlockEntry | None, dst_start: int, n: int) -> bool:
        if entry is None or not self.allocate or n <= 0 or dst_start < 0:
            return False
        bs = self.block_size
        lo_block, hi_block = dst_start // bs, -(-(dst_start + n) // bs)
        if hi_block > entry.table.size:
            return False
        if hi_block - lo_block <= 2:  # a decode step's save: no numpy reduction needed
            return all(entry.table[k] >= 0 for k in range(lo_block, hi_block))
        return bool((entry.table[lo_block:hi_block] >= 0).all())

    def holds_blocks(self, session: str, dst_start: int, n: int) -> bool:
        """Whether every position of ``[dst_start, dst_start + n)`` has a block."""
        return self._positions_ok(self._sessions.get(session), dst_start, n)

    def write_targets(
        self, session: str, layers, dst_start: int, n: int, row_shape, dtype, device
    ) -> list | None:
        """:meth:`write_target` for several layers, the span checked once."""
        entry = self._sessions.get(session)
        if not self._positions_ok(entry, dst_start, n):
            return None
        sig = (tuple(row_shape), dtype)
        key = tuple(layers)
        hit = self._target_lists.get(key)
        if hit is not None and hit[0] == len(self._pools) and self._sig_ok.get(key) == sig:
            out = hit[1]  # the steady state: every pool exists with these rows
        else:
            pools, sigs = self._pools, self._sigs
            out = [pools[layer] if sigs.get(layer) == sig else
                   self._pool_for(layer, row_shape, dtype, device) for layer in layers]
            self._target_lists[key] = (len(self._pools), out)
            self._sig_ok[key] = sig
        if not entry.layers.issuperset(key):
            entry.layers.update(key)
        self.saved_token_layers += n * len(out)
        return out

    def write_target(
        self, session: str, layer: str, dst_start: int, n: int, row_shape, dtype, device
    ) -> torch.Tensor | None:
        """The pool a device-side save of ``[dst_start, dst_start + n)`` writes into,
        through :meth:`table`; None unless :meth:`reserve` gave the span its blocks.
        Accounting as in :meth:`write`."""
        got = self.write_targets(session, (layer,), dst_start, n, row_shape, dtype, device)
        return None if got is None else got[0]

    def write(self, session: str, layer: str, dst_start: int, src: torch.Tensor) -> None:
        """Copy ``src`` ``[n, heads, 2D]`` into the session's blocks (shift_store.py:225-236)."""
        n = src.shape[0]
        p = self.write_target(session, layer, dst_start, n, src.shape[1:], src.dtype, self.device)
        if p is None:
            return
        blk, off = self._rows(session, dst_start, n, p.device)
        rows = src.to(p.device, non_blocking=True)
        if self._planar[layer]:
            d = rows.shape[-1] // 2
            p[blk, 0, off] = rows[..., :d]
            p[blk, 1, off] = rows[..., d:]
        else:
            p[blk, off] = rows

    def _rows(self, session: str, start: int, n: int, device):
        pos = torch.arange(start, start + n, dtype=torch.int64)
        tab = torch.from_numpy(self._sessions[session].table.astype(np.int64))
        return tab[pos // self.block_size].to(device), (pos % self.block_size).to(device)

    def read(self, session: str, layer: str, start: int, n: int) -> torch.Tensor | None:
        """``[n, heads, 2D]`` rows of ``[start, start + n)`` (a gathered copy), or None
        where any position is not held (shift_store.py:238-250)."""
        if not self.lookup(session, layer, start, n):
            return None
        return self.gather(session, layer, start, n)

    def gather(self, session: str, layer: str, start: int, n: int) -> torch.Tensor:
        """``[n, heads, 2D]`` rows of ``[start, start + n)`` from the pool, K then V, with
        no checks and no accounting (the caller knows the rows are held)."""
        p = self._pools[layer]
        blk, off = self._rows(session, start, n, p.device)
        if self._planar[layer]:
            return torch.cat((p[blk, 0, off], p[blk, 1, off]), dim=-1)
        return p[blk, off]
