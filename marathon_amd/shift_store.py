"""Session-keyed KV store and load/save planning: the host API of src/marathon/shift_store.py.

Same names, semantics and return values as the reference module (shift_store.py:56-333):

* :func:`slots` -- flat slot indices of positions ``[lo, hi)`` through a block table.
* :class:`SessionTable` -- one in-flight writer per session (shift_store.py:63-91).
* :class:`ShiftStore` -- per session, per layer, a position-indexed ``[capacity, heads,
  2*head_size]`` device buffer under a token budget, with geometric growth and LRU
  eviction of whole sessions (shift_store.py:101-266).  ``allocate=False`` is the
  tensor-free scheduler-side mirror.
* :func:`plan_load` / :func:`plan_save` / :class:`LoadDecision` -- the connector's
  load and save decisions (shift_store.py:269-333).  A ``None`` decision always means
  recompute, never guess.

The buffers are exactly what the HIP kernels read as a ``flat`` source
(:class:`marathon_amd.spans.CacheSet`): position ``p`` of a session is row ``p``.
"""

from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass, field

import torch

SLAB = 2048  # floor of a session's first allocation; capacity doubles from there
DEFAULT_STORE_TOKENS = 32768


def slots(block_ids, lo: int, hi: int, block_size: int) -> torch.Tensor:
    """Flat slot indices (int64, CPU) of positions ``[lo, hi)`` given a block table."""
    pos = torch.arange(lo, hi, dtype=torch.int64)
    table = torch.as_tensor(block_ids, dtype=torch.int64)
    return table[pos // block_size] * block_size + pos % block_size


class SessionTable:
    """Which request currently writes each session; a second writer is refused."""

    def __init__(self) -> None:
        self._owner: dict[str, str] = {}
        self._session: dict[str, str] = {}
        self.conflicts = 0

    def acquire(self, request_id: str, session: str) -> bool:
        owner = self._owner.get(session)
        if owner is not None and owner != request_id:
            self.conflicts += 1
            return False
        self._owner[session] = request_id
        self._session[request_id] = session
        return True

    def session_of(self, request_id: str) -> str | None:
        return self._session.get(request_id)

    def release(self, request_id: str) -> None:
        session = self._session.pop(request_id, None)
        if session is not None and self._owner.get(session) == request_id:
            del self._owner[session]

    def __len__(self) -> int:
        return len(self._owner)


@dataclass
class _Entry:
    capacity: int = 0  # positions the buffers hold
    base: int = -1  # first position ever written (-1: nothing yet)
    filled: int = 0  # [base, filled) holds valid KV
    layers: dict = field(default_factory=dict)


class ShiftStore:
    """Position-indexed KV per session, under a total token budget with LRU eviction."""

    def __init__(
        self,
        budget_tokens: int = DEFAULT_STORE_TOKENS,
        device: str = "cuda",
        allocate: bool = True,
        slab: int | None = None,
        session_cap: int | None = None,
    ) -> None:
        self.budget = int(budget_tokens)
        self.slab = min(int(slab or SLAB), self.budget)
        self.session_cap = min(int(session_cap), self.budget) if session_cap else 0
        self.device = device
        self.allocate = allocate
        self._sessions: OrderedDict[str, _Entry] = OrderedDict()  # oldest first
        self.hits = 0
        self.misses = 0
        self.evictions = 0
        self.refusals = 0
        self.loaded_token_layers = 0
        self.saved_token_layers = 0

    # ----------------------------------------------------------------- internals

    def _touch(self, session: str) -> _Entry:
        entry = self._sessions.get(session)
        if entry is None:
            entry = self._sessions[session] = _Entry()
        else:
            self._sessions.move_to_end(session)
        return entry

    @property
    def used(self) -> int:
        return sum(e.capacity for e in self._sessions.values())

    def _grow(self, session: str, entry: _Entry, want: int) -> None:
        """Double from the current capacity (floored at slab / session_cap) to fit
        ``want``, capped at the budget, evicting least-recently-used *other* sessions
        until it fits (shift_store.py:149-175)."""
        size = max(self.session_cap, self.slab, 2 * entry.capacity)
        while size < want:
            size *= 2
        size = min(self.budget, size)
        while self.used - entry.capacity + size > self.budget:
            victim = next((s for s in self._sessions if s != session), None)
            if victim is None:
                break
            self.drop(victim)
            self.evictions += 1
        keep = entry.filled
        for name, old in list(entry.layers.items()):
            new = torch.zeros((size, *old.shape[1:]), dtype=old.dtype, device=old.device)
            n = min(keep, old.shape[0])
            new[:n] = old[:n]
            entry.layers[name] = new
        entry.capacity = size

    # -------------------------------------------------------------------- public

    def reserve(self, session: str, dst_start: int, n: int) -> bool:
        """Make room for ``[dst_start, dst_start + n)``; False (and nothing stored) if
        it would leave a hole above ``filled`` or cannot fit the budget.  A start at or
        below ``filled`` truncates what is above the span.  Idempotent."""
        need = dst_start + n
        entry = self._touch(session)
        first = entry.base < 0
        if need > self.budget or n <= 0 or (not first and dst_start > entry.filled):
            self.refusals += 1
            return False
        if need > entry.capacity:
            self._grow(session, entry, need)
        if first:
            entry.base = dst_start
        entry.filled = need
        return True

    def covers(self, session: str, start: int, n: int) -> bool:
        """Whether ``[start, start + n)`` is held for ``session`` (counts a hit/miss)."""
        entry = self._sessions.get(session)
        ok = (
            entry is not None
            and entry.base >= 0
            and start >= entry.base
            and n > 0
            and start + n <= entry.filled
        )
        if ok:
            self.hits += 1
            self._touch(session)
        else:
            self.misses += 1
        return ok

    def write(self, session: str, layer: str, dst_start: int, src: torch.Tensor) -> None:
        """Copy ``src`` ``[n, heads, 2*head_size]`` into the session's buffer."""
        entry = self._sessions.get(session)
        n = src.shape[0]
        if entry is None or dst_start + n > entry.capacity or not self.allocate:
            return
        buf = entry.layers.get(layer)
        if buf is None:
            buf = torch.zeros((entry.capacity, *src.shape[1:]), dtype=src.dtype, device=self.device)
            entry.layers[layer] = buf
        buf[dst_start : dst_start + n] = src.to(buf.device, non_blocking=True)
        self.saved_token_layers += n

    def lookup(self, session: str, layer: str, start: int, n: int) -> bool:
        """:meth:`read`'s check and accounting without making the view: what a batched
        load calls once per (load, layer) (vllm_shift_connector.py:506-513)."""
        entry = self._sessions.get(session)
        if entry is None or entry.base < 0 or start < entry.base or start + n > entry.filled:
            return False
        if entry.layers.get(layer) is None:
            return False
        self.loaded_token_layers += n
        self._touch(session)  # same LRU order as the scheduler mirror's covers()
        return True

    def lookup_layers(self, session: str, layers, start: int, n: int):
        """:meth:`lookup` of every layer in order, with the same accounting; returns the
        first layer that misses, or None when all hit."""
        entry = self._sessions.get(session)
        if entry is None or entry.base < 0 or start < entry.base or start + n > entry.filled:
            return next(iter(layers), None)
        hit = 0
        try:
            for layer in layers:
                if entry.layers.get(layer) is None:
                    return layer
                self.loaded_token_layers += n
                hit += 1
            return None
        finally:
            if hit:
                self._touch(session)  # the LRU order one touch per layer would leave

    def read(self, session: str, layer: str, start: int, n: int) -> torch.Tensor | None:
        """The view ``buf[start:start + n]``, or None outside ``[base, filled)``."""
        if not self.lookup(session, layer, start, n):
            return None
        return self._sessions[session].layers[layer][start : start + n]

    def buffer(self, session: str, layer: str) -> torch.Tensor | None:
        """The whole ``[capacity, heads, 2D]`` buffer (what a batched load reads)."""
        entry = self._sessions.get(session)
        return None if entry is None else entry.layers.get(layer)

    def write_target(
        self, session: str, layer: str, dst_start: int, n: int, row_shape, dtype, device
    ) -> torch.Tensor | None:
        """The buffer a device-side save of ``[dst_start, dst_start + n)`` writes into.

        Same preconditions and accounting as :meth:`write` (shift_store.py:225-236):
        None when the session is unknown, the span exceeds the capacity or the store is
        the tensor-free mirror; the layer's buffer is allocated on first use.  The caller
        fills the rows (the save kernel gathers them straight out of the paged cache).
        """
        entry = self._sessions.get(session)
        if entry is None or dst_start + n > entry.capacity or not self.allocate:
            return None
        buf = entry.layers.get(layer)
        if buf is None:
            buf = torch.zeros((entry.capacity, *row_shape), dtype=dtype, device=device)
            entry.layers[layer] = buf
        self.saved_token_layers += n
        return buf

    def write_targets(
        self, session: str, layers, dst_start: int, n: int, row_shape, dtype, device
    ) -> list | None:
        """:meth:`write_target` for several layers; None if any is refused."""
        out = []
        for layer in layers:
            t = self.write_target(session, layer, dst_start, n, row_shape, dtype, device)
            if t is None:
                return None
            out.append(t)
        return out

    def drop(self, session: str) -> None:
        self._sessions.pop(session, None)

    def stats(self) -> dict:
        return {
            "budget_tokens": self.budget,
            "used_tokens": self.used,
            "sessions": {s: max(e.filled - max(e.base, 0), 0) for s, e in self._sessions.items()},
            "hits": self.hits,
            "misses": self.misses,
            "evictions": self.evictions,
            "refusals": self.refusals,
            "loaded_token_layers": self.loaded_token_layers,
            "saved_token_layers": self.saved_token_layers,
        }


@dataclass(frozen=True)
class LoadDecision:
    """A resolved load: destination ``[lo, hi)``, source starting at ``lo - delta``."""

    lo: int
    hi: int
    delta: int

    @property
    def src_start(self) -> int:
        return self.lo - self.delta


def plan_load(
    store: ShiftStore,
    session: str | None,
    request: dict | None,
    num_computed: int,
    num_prompt_tokens: int,
    block_size: int,
) -> tuple[LoadDecision | None, str]:
    """Whether a request's ``load`` can be served: ``(decision, why)``.

    Whole blocks only, at least one token left for the engine to compute, the engine's
    own prefix hit must reach ``dst_start``, and the store must still hold the source
    (shift_store.py:282-315).
    """
    if not session or not request:
        return None, "no session or no load requested"
    lo = int(num_computed)
    dst_end, delta = int(request["dst_end"]), int(request["delta"])
    if num_computed < int(request["dst_start"]):
        return None, f"local hit {num_computed} < dst_start {request['dst_start']}"
    hi = min(dst_end, (num_prompt_tokens - 1) // block_size * block_size)
    hi -= hi % block_size
    if hi <= lo:
        return None, f"nothing left after block alignment (hi={hi} <= lo={lo})"
    if not store.covers(session, lo - delta, hi - lo):
        return None, f"store no longer holds [{lo - delta},{hi - delta})"
    return LoadDecision(lo, hi, delta), "ok"


def plan_save(
    store: ShiftStore, session: str | None, mode: object, lo: int, hi: int
) -> tuple[int, int] | None:
    """The position range a step saves; ``mode="full"`` widens it to ``[0, hi)``
    (shift_store.py:318-333)."""
    if hi <= lo or not session or not mode:
        return None
    if mode == "full":
        lo = 0
    if not store.reserve(session, lo, hi - lo):
        return None
    return lo, hi
