"""The block-layout store (marathon_amd.block_store) on the CPU.

* Under ``truncate=True`` it must reach the flat store's decisions exactly: the
  reference's store tests (tests/test_shift_store.py, cited per case) are restated on
  it, and a random operation sequence is replayed on both stores side by side.
* The allocator: lowest ids first, no block held twice, drop and eviction return
  blocks, growth never moves stored rows.
* Under ``truncate=False`` validity is per position: a save below what is held keeps
  the positions above it.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from marathon_amd.block_store import BlockShiftStore
from marathon_amd.shift_store import ShiftStore, plan_load


def _kv(n, value, heads=2, dim=4):
    return torch.full((n, heads, dim), float(value))


def _store(**kw):
    kw.setdefault("budget_tokens", 4096)
    kw.setdefault("device", "cpu")
    return BlockShiftStore(**kw)


def _check_allocator(st: BlockShiftStore):
    held = [b for e in st._sessions.values() for b in e.table if b >= 0]
    assert len(held) == len(set(held)), "a block is held twice"
    assert sorted(held + list(st._free)) == list(range(st.pool_blocks))
    for e in st._sessions.values():
        assert e.held == sum(b >= 0 for b in e.table)


# ------------------------------------------------- the reference's store cases


def test_append_only_saves_extend_the_filled_span():  # :62-67
    st = _store()
    assert st.reserve("a", 0, 100) and st.reserve("a", 100, 50)
    assert st.covers("a", 0, 150) and not st.covers("a", 0, 151)


def test_a_save_that_would_leave_a_hole_is_refused():  # :70-75
    st = _store()
    st.reserve("a", 0, 100)
    assert not st.reserve("a", 200, 10)
    assert st.covers("a", 0, 100) and st.refusals == 1


def test_an_edit_truncates_everything_above_it():  # :78-84
    st = _store()
    st.reserve("a", 0, 500)
    free_before = st.free_blocks
    assert st.reserve("a", 100, 50)
    assert st.covers("a", 0, 150) and not st.covers("a", 0, 151)
    # the blocks above the new top went back to the pool, nothing was copied
    assert st.free_blocks == free_before + (-(-500 // 16) - -(-150 // 16))
    _check_allocator(st)


def test_a_span_larger_than_the_budget_is_refused():  # :87-90
    st = _store(budget_tokens=1000)
    assert not st.reserve("a", 0, 1001)
    assert st.refusals == 1


def test_reserve_is_idempotent():  # :93-97
    st = _store()
    for _ in range(3):
        assert st.reserve("a", 0, 64)
    assert st.covers("a", 0, 64) and st.used == 64
    _check_allocator(st)


def test_write_read_round_trip_and_session_isolation():  # :103-113
    st = _store()
    st.reserve("a", 0, 40)
    st.reserve("b", 0, 40)
    st.write("a", "l0", 0, _kv(40, 1.0))
    st.write("b", "l0", 0, _kv(40, 2.0))
    assert torch.equal(st.read("a", "l0", 0, 40), _kv(40, 1.0))
    assert torch.equal(st.read("b", "l0", 0, 40), _kv(40, 2.0))
    assert st.read("a", "l1", 0, 40) is None  # a layer never saved


def test_read_past_the_filled_span_returns_none():  # :116-120
    st = _store()
    st.reserve("a", 0, 10)
    st.write("a", "l0", 0, _kv(10, 1.0))
    assert st.read("a", "l0", 5, 6) is None
    assert st.read("a", "l0", 5, 5) is not None


def test_growth_keeps_stored_rows_in_place():  # :123-130
    st = _store()
    st.reserve("a", 0, 20)
    rows = torch.arange(20 * 2 * 4, dtype=torch.float32).reshape(20, 2, 4)
    st.write("a", "l0", 0, rows)
    pool, table = st.pool("l0"), st.table("a").copy()
    ptr = pool.data_ptr()
    st.reserve("a", 20, 3000)
    st.write("a", "l0", 20, _kv(3000, 7.0))
    assert st.pool("l0").data_ptr() == ptr  # never reallocated
    assert np.array_equal(st.table("a")[: table.size], table)  # old blocks kept
    assert torch.equal(st.read("a", "l0", 0, 20), rows)


def test_lru_evicts_the_least_recently_used_session():  # :136-145
    st = _store(budget_tokens=3 * 512)
    for s in "abc":
        assert st.reserve(s, 0, 512)
    assert st.covers("a", 0, 512)  # a is now most recent; b is the oldest
    assert st.reserve("d", 0, 512)
    assert "b" not in st.stats()["sessions"] and st.evictions == 1
    _check_allocator(st)


def test_eviction_never_takes_the_session_being_written():  # :148-154
    st = _store(budget_tokens=1024)
    assert st.reserve("a", 0, 512)
    assert st.reserve("a", 512, 512)
    assert st.evictions == 0 and st.covers("a", 0, 1024)


def test_an_evicted_session_is_a_miss_not_a_wrong_load():  # :157-164
    st = _store(budget_tokens=512)
    st.reserve("a", 0, 512)
    st.write("a", "l0", 0, _kv(512, 1.0))
    st.reserve("b", 0, 512)
    assert not st.covers("a", 0, 16) and st.read("a", "l0", 0, 16) is None


def test_bookkeeping_only_mode_tracks_positions_without_tensors():  # :167-175
    st = _store(allocate=False)
    assert st.reserve("a", 0, 100)
    st.write("a", "l0", 0, _kv(100, 1.0))
    assert st.pool("l0") is None and st.covers("a", 0, 100)


def test_stats_reports_tokens_per_session():  # :178-186
    st = _store()
    st.reserve("a", 0, 100)
    st.reserve("b", 16, 50)
    s = st.stats()
    assert s["sessions"] == {"a": 100, "b": 50}
    assert s["used_tokens"] == (7 + 4) * 16 and s["free_blocks"] == s["pool_blocks"] - 11


def test_the_first_save_may_start_above_zero():  # :189-198
    st = _store()
    assert st.reserve("a", 300, 100)
    assert st.covers("a", 300, 100) and not st.covers("a", 299, 2)
    assert st.table("a")[: 300 // 16].tolist() == [-1] * (300 // 16)  # no blocks below


def test_plan_load_runs_against_the_block_store():  # shift_store.py:282-315
    st = _store(allocate=False)
    st.reserve("s", 0, 1000)
    d, why = plan_load(st, "s", {"dst_start": 64, "dst_end": 900, "delta": -30}, 64, 1200, 16)
    assert why == "ok" and (d.lo, d.hi, d.delta) == (64, 896, -30)


# ------------------------------------------------------------- the allocator


def test_fresh_sessions_get_contiguous_lowest_blocks():
    st = _store()
    st.reserve("a", 0, 100)
    st.reserve("b", 0, 40)
    assert st.table("a").tolist() == list(range(7))
    assert st.table("b").tolist() == [7, 8, 9]
    st.drop("a")
    st.reserve("c", 0, 20)
    assert st.table("c").tolist() == [0, 1]  # lowest ids come back first
    _check_allocator(st)


def test_random_operations_keep_the_allocator_consistent():
    rng = np.random.default_rng(5)
    for truncate in (True, False):
        st = _store(budget_tokens=2048, truncate=truncate, allocate=False)
        for _ in range(3000):
            s = "abcde"[int(rng.integers(5))]
            op = rng.random()
            if op < 0.7:
                st.reserve(s, int(rng.integers(0, 1800)), int(rng.integers(1, 400)))
            elif op < 0.95:
                st.covers(s, int(rng.integers(0, 1800)), int(rng.integers(1, 400)))
            else:
                st.drop(s)
        _check_allocator(st)


# ------------------------------------------ truncate=True: the flat store's rules


def test_truncate_policy_replays_the_flat_store_decisions():
    """Same operations on both stores (a budget no sequence outgrows, since eviction
    timing is the one documented difference): every return value and every window
    agree, and every valid position has a block."""
    rng = np.random.default_rng(7)
    flat = ShiftStore(budget_tokens=1 << 16, device="cpu", allocate=False, slab=256)
    blk = BlockShiftStore(budget_tokens=1 << 16, device="cpu", allocate=False)
    for _ in range(5000):
        s = "abcd"[int(rng.integers(4))]
        op = rng.random()
        start, n = int(rng.integers(-2, 3000)), int(rng.integers(-1, 500))
        if op < 0.55:
            if start < 0:
                start = 0
            assert flat.reserve(s, start, n) == blk.reserve(s, start, n), (s, start, n)
        elif op < 0.97:
            assert flat.covers(s, start, n) == blk.covers(s, start, n), (s, start, n)
        else:
            flat.drop(s)
            blk.drop(s)
        assert flat.stats()["sessions"] == blk.stats()["sessions"]
    for s, e in blk._sessions.items():
        lo, hi = max(e.base, 0), e.filled
        for p in range(lo, hi):
            assert e.table[p // 16] >= 0
    assert flat.refusals == blk.refusals and flat.hits == blk.hits
    _check_allocator(blk)


# ----------------------------------------- truncate=False: per-position validity


def test_interval_policy_allows_holes_and_never_truncates():
    st = _store(truncate=False)
    assert st.reserve("a", 0, 100)
    assert st.reserve("a", 300, 50)  # a hole: allowed
    assert st.covers("a", 300, 50) and not st.covers("a", 90, 20)
    assert st.reserve("a", 20, 10)  # a save below the top truncates nothing
    assert st.covers("a", 0, 100) and st.covers("a", 300, 50)
    assert st.reserve("a", 100, 200)  # filling the hole joins the intervals
    assert st.covers("a", 0, 350) and st.stats()["sessions"]["a"] == 350


def test_lookup_layers_matches_per_layer_lookups():
    """The loader's bulk check leaves the same counters and LRU order as one lookup per
    layer, on both stores."""
    for make in (lambda: ShiftStore(budget_tokens=4096, device="cpu"),
                 lambda: _store()):
        a, b = make(), make()
        for st in (a, b):
            for s in ("x", "y"):
                st.reserve(s, 0, 100)
                st.write(s, "l0", 0, _kv(100, 1.0))
                st.write(s, "l1", 0, _kv(100, 1.0))
        names = ["l0", "l1", "l2"]
        for sess, start, n in (("x", 0, 50), ("y", 10, 90), ("x", 60, 50), ("z", 0, 5)):
            miss_a = a.lookup_layers(sess, names[:2], start, n)
            miss_b = next((nm for nm in names[:2] if not b.lookup(sess, nm, start, n)), None)
            assert miss_a == miss_b
            miss_a = a.lookup_layers(sess, names, start, n)
            miss_b = next((nm for nm in names if not b.lookup(sess, nm, start, n)), None)
            assert miss_a == miss_b
            assert a.stats() == b.stats()
            assert list(a._sessions) == list(b._sessions)


def test_pool_holds_each_block_as_a_k_plane_then_a_v_plane():
    """Rows written as [heads, 2D] land as K and V planes of their blocks; the planes are
    views of the pool, reused while no pool changes; reads give the rows back."""
    st = _store()
    st.reserve("a", 0, 40)
    rows = torch.arange(40 * 3 * 8, dtype=torch.float32).reshape(40, 3, 8)
    st.write("a", "l0", 0, rows)
    pool, tab = st.pool("l0"), st.table("a")
    assert pool.shape == (st.pool_blocks, 2, 16, 3, 4)
    for pos in (0, 15, 16, 39):
        blk, off = int(tab[pos // 16]), pos % 16
        assert torch.equal(pool[blk, 0, off], rows[pos, :, :4])
        assert torch.equal(pool[blk, 1, off], rows[pos, :, 4:])
    k, v = st.kernel_views(["l0"])
    assert k[0].data_ptr() == pool.data_ptr() and v[0].data_ptr() == pool[:, 1].data_ptr()
    assert k[0].shape == v[0].shape == (st.pool_blocks, 16, 3, 4)
    assert st.kernel_views(["l0"])[0] is k  # the same lists while no pool changes
    assert torch.equal(st.read("a", "l0", 3, 30), rows[3:33])
    with pytest.raises(ValueError, match="K and V halves"):
        st.write("a", "l1", 0, torch.zeros(40, 3, 7))


def test_one_byte_elements_keep_fused_rows():
    """fp8 pools hold rows of K then V per head; the kernels see them as fused caches."""
    st = _store()
    st.reserve("a", 0, 40)
    rows = torch.randn(40, 2, 8).to(torch.float8_e4m3fn)
    st.write("a", "l0", 0, rows)
    pool, tab = st.pool("l0"), st.table("a")
    assert pool.shape == (st.pool_blocks, 16, 2, 8)
    assert torch.equal(pool[int(tab[1]), 3].view(torch.uint8), rows[19].view(torch.uint8))
    caches, v_caches = st.kernel_views(["l0"])
    assert caches[0] is pool and v_caches is None
    assert torch.equal(st.read("a", "l0", 0, 40).view(torch.uint8), rows.view(torch.uint8))
    st.reserve("a", 0, 40)
    st.write("a", "l1", 0, torch.zeros(40, 2, 8))  # a float32 layer: planes
    with pytest.raises(ValueError, match="mix block layouts"):
        st.kernel_views(["l0", "l1"])
