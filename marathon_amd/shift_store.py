"""Session-keyed KV store and load/save planning: the host API of src/marathon/shift_store.py.

Same names, return values, counters and decline reasons as the reference module
(shift_store.py:56-333), on this package's own bookkeeping core
(:mod:`marathon_amd.store_core`), which the block-layout store shares:

* :func:`slots` -- flat slot indices of positions ``[lo, hi)`` through a block table.
* :class:`SessionTable` -- one in-flight writer per session (shift_store.py:63-91).
* :class:`ShiftStore` -- per session and layer, one position-indexed ``[capacity, heads,
  2*head_size]`` device slab under a token budget; a slab grows by doubling, and whole
  sessions are evicted least recently used first (shift_store.py:101-266).
  ``allocate=False`` is the tensor-free scheduler-side mirror.
* :func:`plan_load` / :func:`plan_save` / :class:`LoadDecision` -- the connector's load
  and save decisions (shift_store.py:269-333).  A ``None`` decision always means
  recompute, never guess.

The slabs are what the HIP kernels read as a ``flat`` source
(:class:`marathon_amd.spans.CacheSet`): position ``p`` of a session is row ``p``.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .store_core import StoreCore, Window

SLAB = 2048  # a session's first slab holds at least this many positions; slabs double
DEFAULT_STORE_TOKENS = 32768


def slots(block_ids, lo: int, hi: int, block_size: int) -> torch.Tensor:
    """Flat slot indices (int64, CPU) of positions ``[lo, hi)`` through a block table
    (shift_store.py:56-60): every block expands to its ``block_size`` consecutive slots,
    and positions index that expansion.  The table must cover ``hi``; a negative ``lo``
    is refused (the reference would wrap around to the table's end)."""
    lo, hi, bs = int(lo), int(hi), int(block_size)
    if hi <= lo:
        return torch.zeros(0, dtype=torch.int64)
    if lo < 0:
        raise ValueError(f"negative position {lo}")
    first, last = lo // bs, (hi - 1) // bs
    table = torch.as_tensor(block_ids, dtype=torch.int64).reshape(-1)
    if last >= table.numel():
        raise IndexError(f"positions up to {hi} need {last + 1} blocks, the table has "
                         f"{table.numel()}")
    run = (table[first:last + 1, None] * bs + torch.arange(bs, dtype=torch.int64)).reshape(-1)
    return run[lo - first * bs:hi - first * bs]


class SessionTable:
    """Who writes each session: a second in-flight request on a session is refused (and
    counted), so a load can never race a save of the same session."""

    def __init__(self) -> None:
        self._writer: dict[str, str] = {}  # session -> request writing it
        self._claimed: dict[str, str] = {}  # request -> the session it claimed
        self.conflicts = 0

    def acquire(self, request_id: str, session: str) -> bool:
        if self._writer.setdefault(session, request_id) != request_id:
            self.conflicts += 1
            return False
        self._claimed[request_id] = session
        return True

    def session_of(self, request_id: str) -> str | None:
        return self._claimed.get(request_id)

    def release(self, request_id: str) -> None:
        session = self._claimed.pop(request_id, None)
        if session is not None and self._writer.get(session) == request_id:
            self._writer.pop(session)

    def __len__(self) -> int:
        return len(self._writer)


@dataclass
class _Slab(Window):
    capacity: int = 0  # positions each layer's slab holds
    layers: dict = field(default_factory=dict)  # layer name -> [capacity, heads, 2D]


def _doubled(floor: int, want: int) -> int:
    """The smallest ``floor * 2**k`` (k >= 0) that is at least ``want``."""
    if floor <= 0:
        return want
    steps = max(0, (-(-want // floor) - 1).bit_length())
    return floor << steps


class ShiftStore(StoreCore):
    """Position-indexed KV per session, under a total token budget with LRU eviction."""

    def __init__(
        self,
        budget_tokens: int = DEFAULT_STORE_TOKENS,
        device: str = "cuda",
        allocate: bool = True,
        slab: int | None = None,
        session_cap: int | None = None,
    ) -> None:
        super().__init__(budget_tokens)
        self.slab = min(int(slab or SLAB), self.budget)
        # a caller that knows how many positions a session will ever need sizes its
        # first slab for them, so no later save has to grow it
        self.session_cap = min(int(session_cap), self.budget) if session_cap else 0
        self.device = device
        self.allocate = allocate

    # --------------------------------------------------------------- store hooks

    def _new_entry(self) -> _Slab:
        return _Slab()

    def _admits(self, entry: _Slab, start: int, n: int) -> bool:
        return entry.leaves_no_hole(start)

    def _make_room(self, session: str, entry: _Slab, start: int, end: int) -> bool:
        if end > entry.capacity:
            self._regrow(session, entry, end)
        return True

    def _commit(self, entry: _Slab, start: int, end: int) -> None:
        entry.extend(start, end)

    def _holds(self, entry: _Slab, start: int, n: int) -> bool:
        return entry.contains(start, n)

    def _readable(self, entry: _Slab, start: int, n: int) -> bool:
        return entry.contains(start, n)  # a read, unlike covers, accepts n <= 0

    def _has_layer(self, entry: _Slab, layer: str) -> bool:
        return entry.layers.get(layer) is not None

    def _held_tokens(self, entry: _Slab) -> int:
        return entry.size

    @property
    def used(self) -> int:
        """Positions allocated across sessions (slab capacities, not what is filled)."""
        return sum(e.capacity for e in self._sessions.values())

    def _regrow(self, session: str, entry: _Slab, want: int) -> None:
        """Give every slab of ``session`` room for ``want`` positions: capacity doubles
        from ``max(session_cap, slab, 2 * capacity)`` until it fits, capped at the
        budget; other sessions are evicted, least recently used first, until the total
        fits (shift_store.py:149-175).  Held positions move to the new slabs."""
        size = min(self.budget,
                   _doubled(max(self.session_cap, self.slab, 2 * entry.capacity), want))
        # the total is re-read after every eviction
        self._evict_until(session, lambda: self.used - entry.capacity + size <= self.budget)
        keep = entry.filled
        for name, old in entry.layers.items():
            new = torch.zeros((size, *old.shape[1:]), dtype=old.dtype, device=old.device)
            n = min(keep, old.shape[0])
            new[:n].copy_(old[:n])
            entry.layers[name] = new
        entry.capacity = size

    # ------------------------------------------------------------------ public

    def write(self, session: str, layer: str, dst_start: int, src: torch.Tensor) -> None:
        """Copy ``src`` ``[n, heads, 2*head_size]`` into the session's slab at
        ``dst_start`` (shift_store.py:225-236); ignored when the session is unknown, the
        rows exceed its capacity, or this is the tensor-free mirror."""
        buf = self.write_target(session, layer, dst_start, src.shape[0], src.shape[1:],
                                src.dtype, self.device)
        if buf is not None:
            buf[dst_start:dst_start + src.shape[0]] = src.to(buf.device, non_blocking=True)

    def write_target(self, session: str, layer: str, dst_start: int, n: int, row_shape,
                     dtype, device) -> torch.Tensor | None:
        """The slab a device-side save of ``[dst_start, dst_start + n)`` writes into, with
        :meth:`write`'s preconditions and accounting; the layer's slab is allocated on
        first use.  The caller fills the rows (the save kernel gathers them straight out
        of the paged cache)."""
        entry = self._sessions.get(session)
        if entry is None or not self.allocate or dst_start + n > entry.capacity:
            return None
        buf = entry.layers.get(layer)
        if buf is None:
            buf = entry.layers[layer] = torch.zeros((entry.capacity, *row_shape), dtype=dtype,
                                                    device=device)
        self.saved_token_layers += n
        return buf

    def write_targets(self, session: str, layers, dst_start: int, n: int, row_shape, dtype,
                      device) -> list | None:
        """:meth:`write_target` for several layers; None if any is refused."""
        out = []
        for layer in layers:
            buf = self.write_target(session, layer, dst_start, n, row_shape, dtype, device)
            if buf is None:
                return None
            out.append(buf)
        return out

    def read(self, session: str, layer: str, start: int, n: int) -> torch.Tensor | None:
        """The view ``slab[start:start + n]``, or None outside ``[base, filled)``."""
        if not self.lookup(session, layer, start, n):
            return None
        return self._sessions[session].layers[layer][start:start + n]

    def buffer(self, session: str, layer: str) -> torch.Tensor | None:
        """The whole ``[capacity, heads, 2D]`` slab (what a batched load reads)."""
        entry = self._sessions.get(session)
        return None if entry is None else entry.layers.get(layer)


@dataclass(frozen=True)
class LoadDecision:
    """A resolved load: destination ``[lo, hi)``, source starting at ``lo - delta``."""

    lo: int
    hi: int
    delta: int

    @property
    def src_start(self) -> int:
        return self.lo - self.delta


def _whole_blocks(pos: int, block_size: int) -> int:
    return pos // block_size * block_size


def plan_load(
    store: StoreCore,
    session: str | None,
    request: dict | None,
    num_computed: int,
    num_prompt_tokens: int,
    block_size: int,
) -> tuple[LoadDecision | None, str]:
    """Whether a request's ``load`` can be served: ``(decision, why)``
    (shift_store.py:282-315).

    The load runs from the engine's own prefix hit ``num_computed`` (which must reach
    ``dst_start``: the engine cannot skip a hole) up to ``dst_end``, cut back to whole
    blocks and to before the prompt's last block-aligned position, so that the engine
    computes at least one token; the store must still hold the shifted source.
    """
    if not (session and request):
        return None, "no session or no load requested"
    if num_computed < int(request["dst_start"]):
        return None, f"local hit {num_computed} < dst_start {request['dst_start']}"
    delta = int(request["delta"])
    lo = int(num_computed)
    hi = _whole_blocks(min(int(request["dst_end"]),
                           _whole_blocks(num_prompt_tokens - 1, block_size)), block_size)
    if lo >= hi:
        return None, f"nothing left after block alignment (hi={hi} <= lo={lo})"
    src_lo, src_hi = lo - delta, hi - delta
    if not store.covers(session, src_lo, hi - lo):
        return None, f"store no longer holds [{src_lo},{src_hi})"
    return LoadDecision(lo, hi, delta), "ok"


def plan_save(
    store: StoreCore, session: str | None, mode: object, lo: int, hi: int
) -> tuple[int, int] | None:
    """The positions a step saves, reserved in ``store``: ``[lo, hi)``, or ``[0, hi)`` for
    ``mode="full"`` (the edit turn's one-shot re-gather); None when nothing is saved
    (shift_store.py:318-333)."""
    if not (session and mode) or hi <= lo:
        return None
    start = 0 if mode == "full" else lo
    return (start, hi) if store.reserve(session, start, hi - start) else None
