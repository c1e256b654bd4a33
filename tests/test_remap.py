"""The generation-0 address book (marathon_amd.remap) on the CPU.

Each case restates a case of the reference's tests/test_remap.py (line cited per test);
a brute-force per-position model checks translate / after_turn on random turns.
"""

from __future__ import annotations

import numpy as np

from marathon_amd.remap import Remap, loads_for


def seg(lo, hi, delta):
    return {"dst_start": lo, "dst_end": hi, "delta": delta}


def test_empty_book_is_the_identity():  # :18-21
    r = Remap()
    assert r.translate(0, 100) == [(0, 100, 0)]
    assert loads_for(r, [seg(100, 200, -50)]) == [seg(100, 200, -50)]


def test_one_reuse_turn_records_its_delta():  # :24-28
    r = Remap().after_turn([(100, 400, -50)], total=1000)
    assert r.pieces == [(100, 400, -50)]
    assert r.translate(100, 400) == [(100, 400, -50)]


def test_offsets_add_across_turns():  # :31-41
    r0 = Remap().after_turn([(100, 400, -50)], total=1000)
    assert loads_for(r0, [seg(50, 350, -50)]) == [seg(50, 350, -100)]
    assert r0.after_turn([(50, 350, -50)], total=1000).pieces == [(50, 350, -100)]


def test_depth_grows_and_a_turn_without_reuse_clears_it():  # :44-50
    r = Remap()
    for _ in range(5):
        r = r.after_turn([(100, 400, -20)], total=1000)
    assert r.depth() == 100
    assert Remap().after_turn([], total=1000).pieces == []


def test_a_span_over_two_offsets_becomes_two_loads():  # :53-60
    r = Remap(pieces=[(0, 100, -10), (100, 200, -30)])
    assert loads_for(r, [seg(0, 200, 0)]) == [seg(0, 100, -10), seg(100, 200, -30)]


def test_uncovered_positions_have_offset_zero():  # :63-66
    r = Remap(pieces=[(100, 200, -30)])
    assert r.translate(0, 300) == [(0, 100, 0), (100, 200, -30), (200, 300, 0)]


def test_recomputed_text_leaves_the_book():  # :69-74
    r = Remap(pieces=[(0, 400, -50)]).after_turn([(0, 100, 0)], total=1000)
    assert r.pieces == [(0, 100, -50)]
    assert r.translate(100, 400) == [(100, 400, 0)]


def test_translate_partitions_the_range():  # :77-82
    pieces = Remap(pieces=[(50, 150, -5), (300, 400, -9)]).translate(0, 500)
    assert pieces[0][0] == 0 and pieces[-1][1] == 500
    assert all(a[1] == b[0] for a, b in zip(pieces, pieces[1:]))


def test_generation_zero_over_a_long_session():  # :85-106
    total, lo, hi = 10000, 6000, 9000
    r = Remap()
    origin = {p: p for p in range(lo, hi)}
    for _ in range(12):
        d = -200
        r = r.after_turn([(lo + d, hi + d, d)], total=total)
        origin = {p + d: o for p, o in origin.items()}
        lo, hi = lo + d, hi + d
        for ld in loads_for(r, [seg(lo, hi, 0)]):
            assert ld["dst_start"] - ld["delta"] == origin[ld["dst_start"]]
    assert r.depth() == 2400


def test_neighbours_join_and_the_prompt_clips():  # :109-111
    r = Remap().after_turn([(0, 100, -5), (100, 200, -5)], total=150)
    assert r.pieces == [(0, 150, -5)]


def test_random_turns_against_a_per_position_model():
    """Per-position truth: ``origin[p]`` is the store index that holds position p's
    generation-0 KV.  After any sequence of turns, every load must reach it."""
    rng = np.random.default_rng(11)
    total = 600
    for _ in range(40):
        r = Remap()
        origin = np.arange(total)
        for _turn in range(6):
            segs = []
            at = int(rng.integers(0, 60))
            while at < total - 20 and len(segs) < 3:
                n = int(rng.integers(10, 150))
                d = int(rng.integers(-40, 41))
                dst_lo, dst_hi = at, min(at + n, total)
                src_lo, src_hi = dst_lo - d, dst_hi - d
                if src_lo >= 0 and src_hi <= total:
                    segs.append((dst_lo, dst_hi, d))
                at = dst_hi + int(rng.integers(1, 80))
            # the loads of this turn reach the generation-0 index of their source
            for lo, hi, d in segs:
                for ld in loads_for(r, [seg(lo, hi, d)]):
                    for p in range(ld["dst_start"], ld["dst_end"]):
                        assert p - ld["delta"] == origin[p - d]
            new_origin = np.arange(total)  # recomputed text is stored where it sits
            for lo, hi, d in segs:
                new_origin[lo:hi] = origin[lo - d:hi - d]
            origin = new_origin
            r = r.after_turn(segs, total)
            # the book agrees with the model at every position
            for lo, hi, off in r.translate(0, total):
                assert np.array_equal(origin[lo:hi], np.arange(lo, hi) - off)
