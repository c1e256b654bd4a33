"""Bookkeeping shared by the session stores: LRU order, counters, the validity window.

The connector's two stores differ only in how they lay KV out in memory:
:class:`~marathon_amd.shift_store.ShiftStore` keeps one position-indexed slab per session
and layer (the reference's layout, src/marathon/shift_store.py:101-266), and
:class:`~marathon_amd.block_store.BlockShiftStore` keeps fixed blocks of a preallocated
per-layer pool.  Everything else -- which sessions exist and in what LRU order, the
hit/miss/eviction/refusal/load/save counters, when a save is admitted, which positions
count as held -- is decided here, once, by :class:`StoreCore`.  A store supplies the
memory side through a few hooks:

* ``_new_entry()``                      -- a session's empty record;
* ``_admits(entry, start, n)``          -- layout-specific admission (beyond budget and n);
* ``_make_room(session, entry, start, end)`` -- give the session memory for
  ``[start, end)``, evicting through :meth:`StoreCore._evict_until`; False refuses;
* ``_commit(entry, start, end)``        -- record a save as held;
* ``_holds(entry, start, n)`` / ``_readable(entry, start, n)`` -- what ``covers`` and
  ``lookup`` accept;
* ``_has_layer(entry, layer)``, ``_held_tokens(entry)``, ``_forget(entry)``.

The scheduler keeps a tensor-free mirror of the worker's store (``allocate=False``) and
must reach the same decisions from the same calls; sharing one implementation of the
decisions is what keeps the two kinds of store and their mirrors in step.
"""

from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass

COUNTERS = ("hits", "misses", "evictions", "refusals", "loaded_token_layers",
            "saved_token_layers")


@dataclass
class Window:
    """The positions a session holds under the truncating rule: ``[base, filled)``.

    ``base`` is -1 until the first save, whose start it then keeps (a request's first
    save begins at its prefix-cache hit, and the store never claims what lies below).
    A later save must start at or below ``filled`` (no hole) and moves ``filled`` to its
    end, which drops whatever was held above it: an edit recomputes everything after
    itself.
    """

    base: int = -1
    filled: int = 0

    @property
    def empty(self) -> bool:
        return self.base < 0

    def leaves_no_hole(self, start: int) -> bool:
        return self.empty or start <= self.filled

    def contains(self, start: int, n: int) -> bool:
        return not self.empty and self.base <= start and start + n <= self.filled

    def extend(self, start: int, end: int) -> None:
        if self.empty:
            self.base = start
        self.filled = end

    @property
    def size(self) -> int:
        return max(self.filled - max(self.base, 0), 0)


class StoreCore:
    """Session records in LRU order (oldest first) plus the store counters."""

    def __init__(self, budget_tokens: int) -> None:
        self.budget = int(budget_tokens)
        self._sessions: OrderedDict = OrderedDict()
        for name in COUNTERS:
            setattr(self, name, 0)

    # ---------------------------------------------------------------- store hooks

    def _new_entry(self):
        raise NotImplementedError

    def _admits(self, entry, start: int, n: int) -> bool:
        return True

    def _make_room(self, session: str, entry, start: int, end: int) -> bool:
        raise NotImplementedError

    def _commit(self, entry, start: int, end: int) -> None:
        raise NotImplementedError

    def _holds(self, entry, start: int, n: int) -> bool:
        raise NotImplementedError

    def _readable(self, entry, start: int, n: int) -> bool:
        return self._holds(entry, start, n)

    def _has_layer(self, entry, layer: str) -> bool:
        raise NotImplementedError

    def _has_layers(self, entry, layers) -> bool:
        """Whether every one of ``layers`` can be read (a fast path for the usual case;
        False sends the caller through :meth:`_has_layer` one layer at a time)."""
        return False

    def _held_tokens(self, entry) -> int:
        raise NotImplementedError

    def _forget(self, entry) -> None:
        """Release what a dropped session held (default: nothing to release)."""

    def _extra_stats(self) -> dict:
        return {}

    # ------------------------------------------------------------------ shared core

    def _touch(self, session: str):
        """The session's record, created on first use, marked most recently used."""
        entry = self._sessions.get(session)
        if entry is None:
            entry = self._sessions.setdefault(session, self._new_entry())
        else:
            self._sessions.move_to_end(session)
        return entry

    def _evict_until(self, session: str, fits) -> bool:
        """Drop whole sessions other than ``session``, least recently used first, until
        ``fits()``; returns whether it fits in the end."""
        for victim in [s for s in self._sessions if s != session]:
            if fits():
                return True
            self.drop(victim)
            self.evictions += 1
        return fits()

    def reserve(self, session: str, dst_start: int, n: int) -> bool:
        """Make room for positions ``[dst_start, dst_start + n)`` of ``session``.

        False -- and nothing stored -- when the span exceeds the whole budget, is empty,
        is not admitted by the layout (a hole above ``filled`` under the truncating
        rule), or cannot be given memory.  A start at or below ``filled`` truncates what
        lies above the span.  Idempotent for a repeated ``(session, dst_start, n)``: the
        worker calls it once per layer or per step, the scheduler once per step
        (shift_store.py:177-199)."""
        end = dst_start + n
        entry = self._touch(session)
        ok = (end <= self.budget and n > 0 and self._admits(entry, dst_start, n)
              and self._make_room(session, entry, dst_start, end))
        if not ok:
            self.refusals += 1
            return False
        self._commit(entry, dst_start, end)
        return True

    def covers(self, session: str, start: int, n: int) -> bool:
        """Whether ``[start, start + n)`` is held for ``session``; counts a hit or a miss
        and marks the session used on a hit (shift_store.py:201-214)."""
        entry = self._sessions.get(session)
        held = entry is not None and n > 0 and self._holds(entry, start, n)
        if not held:
            self.misses += 1
            return False
        self.hits += 1
        self._touch(session)
        return True

    def lookup(self, session: str, layer: str, start: int, n: int) -> bool:
        """A read's check and accounting without the data: whether ``layer`` of
        ``[start, start + n)`` can be read; on success counts ``n`` loaded token-layers
        and marks the session used, in the order the scheduler's ``covers`` does
        (shift_store.py:238-250)."""
        entry = self._sessions.get(session)
        if entry is None or not self._readable(entry, start, n) or not self._has_layer(entry, layer):
            return False
        self.loaded_token_layers += n
        self._touch(session)
        return True

    def lookup_layers(self, session: str, layers, start: int, n: int):
        """:meth:`lookup` of ``layers`` in order with the same accounting, as one call:
        returns the first layer that cannot be read, or None when every one can."""
        entry = self._sessions.get(session)
        if entry is None or not self._readable(entry, start, n):
            return next(iter(layers), None)
        missing = None
        if self._has_layers(entry, layers):
            loaded = len(layers)
        else:
            loaded = 0
            for layer in layers:
                if not self._has_layer(entry, layer):
                    missing = layer
                    break
                loaded += 1
        if loaded:
            self.loaded_token_layers += n * loaded
            self._touch(session)  # the LRU order one touch per layer leaves
        return missing

    def drop(self, session: str) -> None:
        entry = self._sessions.pop(session, None)
        if entry is not None:
            self._forget(entry)

    def stats(self) -> dict:
        out = {"budget_tokens": self.budget, "used_tokens": self.used}
        out.update(self._extra_stats())
        out["sessions"] = {s: self._held_tokens(e) for s, e in self._sessions.items()}
        out.update((name, getattr(self, name)) for name in COUNTERS)
        return out

    @property
    def used(self) -> int:
        raise NotImplementedError
