"""Generation-0 address book: which store index backs each logical position.

Host logic of src/marathon/remap.py, the no-resave alternative to the ``save="full"``
re-gather.  Store index ``i`` always holds keys as computed at position ``i``.  A reused
span that now sits at logical ``p`` therefore needs exactly one rotation, by ``p - i``.
The book records that offset per logical range.  Offsets add up across turns because
rotations compose, so reuse never stitches from stitched bytes.

A piece ``(lo, hi, off)`` says: logical ``[lo, hi)`` lives at store ``[lo - off, hi - off)``.
Logical positions that no piece covers have offset 0: they were computed and saved at
their own index.

Wiring it needs a store whose saves never truncate other positions: the per-position
policy of :class:`marathon_amd.block_store.BlockShiftStore` (``truncate=False``).
"""

from __future__ import annotations

from dataclasses import dataclass, field

Piece = tuple  # (lo, hi, off)


def _normalise(pieces, total: int) -> list:
    """Sorted, clipped to ``[0, total)``, empties dropped, touching equal offsets joined."""
    out: list = []
    for lo, hi, off in sorted(pieces):
        lo, hi = max(int(lo), 0), min(int(hi), int(total))
        if lo >= hi:
            continue
        if out and out[-1][2] == off and out[-1][1] == lo:
            out[-1] = (out[-1][0], hi, off)
        else:
            out.append((lo, hi, off))
    return out


@dataclass
class Remap:
    """Logical-position -> store-index offsets of one session (remap.py:35-100)."""

    pieces: list = field(default_factory=list)

    def translate(self, lo: int, hi: int) -> list:
        """``[lo, hi)`` cut into ``(lo, hi, off)`` runs in logical order, gaps at offset 0
        (remap.py:41-64)."""
        runs: list = []
        at = lo
        for p_lo, p_hi, off in sorted(self.pieces):
            a, b = max(p_lo, at), min(p_hi, hi)
            if b <= a:
                if p_lo >= hi:
                    break
                continue
            if a > at:
                runs.append((at, a, 0))
            runs.append((a, b, off))
            at = b
            if at >= hi:
                break
        if at < hi:
            runs.append((at, hi, 0))
        return runs

    def after_turn(self, segments, total: int) -> "Remap":
        """The book after a turn that reused ``(dst_lo, dst_hi, delta)`` segments: each
        reused run keeps its old offset plus ``delta``; everything else was recomputed
        and drops out (remap.py:66-82)."""
        moved = []
        for dst_lo, dst_hi, delta in sorted(segments):
            if dst_hi > dst_lo:
                for a, b, off in self.translate(dst_lo - delta, dst_hi - delta):
                    moved.append((a + delta, b + delta, off + delta))
        return Remap(_normalise(moved, total))

    def restrict(self, hi: int) -> "Remap":
        """Only what lies below ``hi`` (remap.py:84-92)."""
        return Remap(_normalise(self.pieces, hi))

    def offsets(self) -> set:
        return {off for _, _, off in self.pieces}

    def depth(self) -> int:
        """The largest accumulated offset (remap.py:97-99)."""
        return max((abs(off) for _, _, off in self.pieces), default=0)


def loads_for(remap: Remap, segments) -> list:
    """Plan segments as loads whose ``delta`` reaches generation-0 bytes (remap.py:115-132).

    ``remap`` is the book as it stood before this turn: a plan's ``delta`` is measured
    against the previous turn's positions.
    """
    loads = []
    for seg in segments:
        lo, hi, delta = int(seg["dst_start"]), int(seg["dst_end"]), int(seg["delta"])
        for a, b, off in remap.translate(lo - delta, hi - delta):
            loads.append({"dst_start": a + delta, "dst_end": b + delta, "delta": off + delta})
    return loads
