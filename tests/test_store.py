"""Host bookkeeping of the shift path on the CPU: slots, the single-writer table, the
session store and the load/save planners.

Each case restates a case of the reference's tests/test_shift_store.py (cited per test)
against marathon_amd.shift_store; the store holds CPU tensors here exactly as the
reference's tests do -- bookkeeping, not KV math.
"""

from __future__ import annotations

import pytest
import torch

from marathon_amd.connector import accept_multi, detect_hnd, paged_planes
from marathon_amd.shift_store import (
    LoadDecision,
    SessionTable,
    ShiftStore,
    plan_load,
    plan_save,
    slots,
)


def _kv(n: int, value: float, heads: int = 2, dim: int = 4) -> torch.Tensor:
    return torch.full((n, heads, dim), value)


def test_slots_map_positions_through_the_block_table():  # :24-27
    assert slots([7, 3], 2, 6, block_size=4).tolist() == [30, 31, 12, 13]


def test_session_table_refuses_a_second_in_flight_writer():  # :33-41
    t = SessionTable()
    assert t.acquire("r1", "s")
    assert not t.acquire("r2", "s")
    assert t.session_of("r2") is None
    assert t.conflicts == 1
    t.release("r1")
    assert t.acquire("r2", "s")
    assert t.session_of("r2") == "s"


def test_session_table_reacquire_by_the_same_request_is_fine():  # :44-48
    t = SessionTable()
    assert t.acquire("r1", "s") and t.acquire("r1", "s")
    assert t.conflicts == 0


def test_session_table_release_of_an_unknown_request_is_a_noop():  # :51-56
    t = SessionTable()
    t.acquire("r1", "s")
    t.release("nobody")
    assert t.session_of("r1") == "s" and len(t) == 1


def test_append_only_saves_extend_the_filled_span():  # :62-67
    st = ShiftStore(slab=1024, budget_tokens=4096, device="cpu")
    assert st.reserve("a", 0, 100) and st.reserve("a", 100, 50)
    assert st.covers("a", 0, 150) and not st.covers("a", 0, 151)


def test_a_save_that_would_leave_a_hole_is_refused():  # :70-75
    st = ShiftStore(slab=1024, budget_tokens=4096, device="cpu")
    st.reserve("a", 0, 100)
    assert not st.reserve("a", 200, 10)
    assert st.covers("a", 0, 100) and st.refusals == 1


def test_an_edit_truncates_everything_above_it():  # :78-84
    st = ShiftStore(slab=1024, budget_tokens=4096, device="cpu")
    st.reserve("a", 0, 500)
    assert st.reserve("a", 200, 60)
    assert st.covers("a", 0, 260) and not st.covers("a", 0, 300)


def test_a_span_larger_than_the_budget_is_refused():  # :87-90
    st = ShiftStore(slab=1024, budget_tokens=1024, device="cpu")
    assert not st.reserve("a", 0, 2000)
    assert not st.covers("a", 0, 1)


def test_reserve_is_idempotent_so_the_worker_may_call_it_per_layer():  # :93-97
    st = ShiftStore(slab=1024, budget_tokens=4096, device="cpu")
    for _ in range(5):
        assert st.reserve("a", 0, 300)
    assert st.stats()["sessions"] == {"a": 300}


def test_write_read_round_trip_and_session_isolation():  # :103-113
    st = ShiftStore(slab=1024, budget_tokens=4096, device="cpu")
    st.reserve("a", 0, 8)
    st.reserve("b", 0, 8)
    st.write("a", "layer0", 0, _kv(8, 1.0))
    st.write("b", "layer0", 0, _kv(8, 2.0))
    assert torch.equal(st.read("a", "layer0", 0, 8), _kv(8, 1.0))
    assert torch.equal(st.read("b", "layer0", 0, 8), _kv(8, 2.0))
    assert st.read("a", "layer1", 0, 8) is None
    assert st.read("nobody", "layer0", 0, 8) is None


def test_read_past_the_filled_span_returns_none():  # :116-120
    st = ShiftStore(slab=1024, budget_tokens=4096, device="cpu")
    st.reserve("a", 0, 8)
    st.write("a", "layer0", 0, _kv(8, 1.0))
    assert st.read("a", "layer0", 4, 8) is None


def test_growth_preserves_already_stored_kv():  # :123-130
    st = ShiftStore(slab=1024, budget_tokens=8192, device="cpu")
    st.reserve("a", 0, 100)
    st.write("a", "layer0", 0, _kv(100, 3.0))
    st.reserve("a", 100, 2000)
    st.write("a", "layer0", 100, _kv(2000, 4.0))
    assert torch.equal(st.read("a", "layer0", 0, 100), _kv(100, 3.0))
    assert torch.equal(st.read("a", "layer0", 100, 2000), _kv(2000, 4.0))


def test_lru_evicts_the_least_recently_used_session():  # :136-145
    st = ShiftStore(slab=1024, budget_tokens=3072, device="cpu")
    st.reserve("a", 0, 1000)
    st.reserve("b", 0, 1000)
    st.reserve("c", 0, 1000)
    st.covers("a", 0, 1000)
    st.reserve("c", 1000, 500)
    assert st.stats()["evictions"] == 1
    assert set(st.stats()["sessions"]) == {"a", "c"}
    assert not st.covers("b", 0, 10)


def test_eviction_never_takes_the_session_being_written():  # :148-154
    st = ShiftStore(slab=1024, budget_tokens=2048, device="cpu")
    st.reserve("a", 0, 1000)
    st.reserve("b", 0, 1000)
    st.reserve("b", 1000, 1000)
    assert set(st.stats()["sessions"]) == {"b"}
    assert st.covers("b", 0, 2000)


def test_an_evicted_session_is_a_miss_not_a_wrong_load():  # :157-164
    st = ShiftStore(slab=1024, budget_tokens=2048, device="cpu")
    st.reserve("a", 0, 1000)
    st.write("a", "layer0", 0, _kv(1000, 9.0))
    st.reserve("b", 0, 2000)
    assert not st.covers("a", 0, 1000)
    assert st.read("a", "layer0", 0, 1000) is None
    assert st.misses == 1


def test_bookkeeping_only_mode_tracks_positions_without_tensors():  # :167-175
    sched = ShiftStore(slab=1024, budget_tokens=4096, device="cpu", allocate=False)
    worker = ShiftStore(slab=1024, budget_tokens=4096, device="cpu")
    for start, n in ((0, 500), (500, 500), (200, 100)):
        assert sched.reserve("a", start, n) == worker.reserve("a", start, n)
    sched.write("a", "layer0", 0, _kv(8, 1.0))
    assert sched.read("a", "layer0", 0, 8) is None
    assert sched.stats()["sessions"] == worker.stats()["sessions"] == {"a": 300}


def test_stats_reports_tokens_per_session():  # :178-186
    st = ShiftStore(slab=1024, budget_tokens=4096, device="cpu")
    st.reserve("a", 0, 300)
    st.reserve("b", 0, 700)
    st.write("b", "layer0", 0, _kv(700, 1.0))
    s = st.stats()
    assert s["sessions"] == {"a": 300, "b": 700}
    assert s["saved_token_layers"] == 700 and s["budget_tokens"] == 4096


def test_the_first_save_may_start_above_zero():  # :189-198
    st = ShiftStore(slab=1024, budget_tokens=4096, device="cpu")
    assert st.reserve("a", 16, 600) and st.reserve("a", 616, 600)
    assert st.covers("a", 616, 600) and st.covers("a", 16, 1200)
    assert not st.covers("a", 0, 1216)
    assert st.read("a", "layer0", 0, 16) is None


def test_hnd_gather_permute_matches_separated_advanced_indexing():  # :201-218
    blocks, heads, block_size, dim = 7, 4, 16, 8
    s = torch.tensor([0, 5, 17, 33, 71, 96, 111], dtype=torch.int64)
    blk, off = s // block_size, s % block_size
    hnd = torch.randn(blocks, heads, block_size, dim)
    assert torch.equal(hnd[blk, :, off], hnd.permute(0, 2, 1, 3)[blk, off])
    nhd = torch.randn(blocks, block_size, heads, dim)
    assert nhd[blk, off].shape == (s.numel(), heads, dim)


def test_session_cap_pre_sizes_the_first_allocation():  # shift_store.py:114-123
    st = ShiftStore(slab=1024, budget_tokens=8192, device="cpu", session_cap=4096)
    st.reserve("a", 0, 10)
    assert st.used == 4096


# ------------------------------------------------------------------- planners


def test_plan_load_declines_without_session_or_request():
    st = ShiftStore(device="cpu", allocate=False)
    assert plan_load(st, None, {"dst_start": 0, "dst_end": 64, "delta": 0}, 0, 100, 16)[0] is None
    assert plan_load(st, "s", None, 0, 100, 16)[0] is None


def test_plan_load_aligns_to_whole_blocks_and_leaves_a_token():  # shift_store.py:308-312
    st = ShiftStore(budget_tokens=8192, device="cpu", allocate=False)
    st.reserve("s", 0, 1000)
    req = {"dst_start": 32, "dst_end": 500, "delta": -10}
    d, why = plan_load(st, "s", req, 48, 490, 16)
    # hi = min(500, (490 - 1) // 16 * 16 = 480) = 480; lo = num_computed = 48
    assert why == "ok" and d == LoadDecision(48, 480, -10) and d.src_start == 58
    d, why = plan_load(st, "s", req, 48, 60, 16)  # nothing left after alignment
    assert d is None and "block alignment" in why
    d, why = plan_load(st, "s", req, 16, 490, 16)  # local hit stops before dst_start
    assert d is None and "local hit" in why


def test_plan_load_declines_when_the_store_lost_the_source():
    st = ShiftStore(budget_tokens=8192, device="cpu", allocate=False)
    st.reserve("s", 0, 100)
    d, why = plan_load(st, "s", {"dst_start": 0, "dst_end": 400, "delta": 50}, 0, 500, 16)
    assert d is None and "no longer holds" in why


def test_plan_save_full_widens_to_zero_once():  # shift_store.py:327-333
    st = ShiftStore(budget_tokens=8192, device="cpu", allocate=False)
    assert plan_save(st, "s", "full", 100, 200) == (0, 200)
    assert plan_save(st, "s", True, 200, 201) == (200, 201)
    assert plan_save(st, "s", True, 5, 5) is None
    assert plan_save(st, None, True, 0, 5) is None
    assert plan_save(st, "s", False, 0, 5) is None


def test_accept_multi_block_aligns_and_drops_what_it_cannot_serve():
    """vllm_shift_connector.py:225-245."""
    held = {(32, 96)}

    def covers(start, n):
        return any(a <= start and start + n <= b for a, b in held)

    loads = [
        {"dst_start": 40, "dst_end": 120, "delta": -8},  # -> [48, 112) src [56, 120): lost
        {"dst_start": 17, "dst_end": 90, "delta": -5},  # -> [32, 80) src [37, 85): held
        {"dst_start": 100, "dst_end": 110, "delta": 0},  # < one block after alignment
    ]
    got = accept_multi(loads, num_computed=20, num_prompt_tokens=200, block_size=16, covers=covers)
    assert got == [{"dst_start": 32, "dst_end": 80, "delta": -5}]


@pytest.mark.parametrize(
    "shape,hnd",
    [((10, 8, 16, 256), True), ((10, 16, 8, 256), False), ((10, 16, 16, 256), False)],
)
def test_layout_detection(shape, hnd):  # vllm_shift_connector.py:396-402
    assert detect_hnd(shape, 16) is hnd


def test_paged_index_tables_and_slots():
    """Device-side slots: each item's window of its block table (the blocks its positions
    touch), concatenated, with per-item (position in the window, offset); a batch with
    any host slots falls back to concatenated int64 slots (from_blocks items expanded)."""
    from marathon_amd.connector import Load, Save, paged_index

    a = Load.from_blocks("s", [7, 3, 9], 5, 40, -2)
    b = Load.from_blocks("t", [1, 2], 16, 32, 4)
    mode, index, rows = paged_index([a, b], 16)
    assert mode == "table" and index.tolist() == [7, 3, 9, 2]
    assert rows == [(5, 0), (0, 3)]
    # the windows resolve to the same slots as the whole tables
    for it, (pos, off) in zip((a, b), rows):
        got = [index[off + (pos + i) // 16].item() * 16 + (pos + i) % 16 for i in range(it.n)]
        assert got == slots(it.block_ids, it.paged_pos, it.paged_pos + it.n, 16).tolist()
    assert (a.src_start, a.n, b.src_start, b.n) == (7, 35, 12, 16)
    c = Load("u", slots([4], 0, 3, 16), 0, 0)
    mode, index, rows = paged_index([a, c], 16)
    assert mode == "slots" and rows == [(0, 0), (0, 35)]
    assert index.tolist() == slots([7, 3, 9], 5, 40, 16).tolist() + [64, 65, 66]
    with pytest.raises(ValueError):
        paged_index([Save.from_blocks("s", [1, 2], 20, 40)], 16)  # 40 > 2 blocks


def test_store_from_config_follows_the_reference_order(monkeypatch):
    """Budget from extra config, else MARATHON_STORE_TOKENS, else 32,768; tensors only
    on the worker; session_tokens pre-sizes a session (vllm_shift_connector.py:168-178)."""
    from marathon_amd import BlockShiftStore, ShiftStore
    from marathon_amd.connector import store_from_config

    monkeypatch.delenv("MARATHON_STORE_TOKENS", raising=False)
    st = store_from_config(None, worker=False)
    assert isinstance(st, ShiftStore) and st.budget == 32768 and not st.allocate
    monkeypatch.setenv("MARATHON_STORE_TOKENS", "5000")
    assert store_from_config({}, worker=True).budget == 5000
    st = store_from_config({"store_tokens": 7000, "store_device": "cpu",
                            "session_tokens": 3000}, worker=True)
    assert (st.budget, st.device, st.allocate, st.session_cap) == (7000, "cpu", True, 3000)
    bst = store_from_config({"store_tokens": 640}, worker=True, block_layout=True)
    assert isinstance(bst, BlockShiftStore) and bst.budget == 640 and bst.pool_blocks == 40


def test_paged_planes_split_and_fused_layouts():
    """Fused 4-D caches pass through; 5-D caches split along their axis of size 2 into K
    and V planes (vLLM's [2, blocks, bs, heads, D] and [blocks, 2, bs, heads, D])."""
    fused = torch.zeros(6, 8, 16, 256)
    assert paged_planes(fused, 16) == ("hnd", fused, None)
    a0 = torch.arange(2 * 6 * 16 * 4 * 128, dtype=torch.float32).reshape(2, 6, 16, 4, 128)
    layout, k, v = paged_planes(a0, 16)
    assert layout == "nhd" and torch.equal(k, a0[0]) and torch.equal(v, a0[1])
    a1 = a0.permute(1, 0, 2, 3, 4)  # [blocks, 2, bs, heads, D], strided planes
    layout, k, v = paged_planes(a1, 16)
    assert layout == "nhd" and torch.equal(k, a0[0]) and torch.equal(v, a0[1])
    assert k.data_ptr() == a0[0].data_ptr() and v.data_ptr() == a0[1].data_ptr()
    hnd = torch.zeros(2, 6, 4, 16, 128)
    assert paged_planes(hnd, 16)[0] == "hnd"
    with pytest.raises(ValueError, match="fused 4-D or a split 5-D"):
        paged_planes(torch.zeros(3, 6, 16, 4, 128), 16)


# ------------------------------------------- the store's own formulations, pinned


def test_slots_equal_brute_force_and_refuse_what_the_table_cannot_hold():
    """``slots`` expands blocks into their slots and slices the positions; brute force
    maps each position through the table one by one."""
    import numpy as np

    rng = np.random.default_rng(0)
    for _ in range(200):
        bs = int(rng.choice([1, 4, 16, 24]))
        table = rng.permutation(64)[: int(rng.integers(1, 20))].tolist()
        lo = int(rng.integers(0, len(table) * bs))
        hi = int(rng.integers(lo, len(table) * bs + 1))
        want = [table[p // bs] * bs + p % bs for p in range(lo, hi)]
        assert slots(table, lo, hi, bs).tolist() == want
    assert slots([3], 5, 5, 16).numel() == 0
    with pytest.raises(IndexError):
        slots([3, 4], 0, 33, 16)
    with pytest.raises(ValueError):
        slots([3, 4], -1, 8, 16)


def test_slab_capacity_doubles_from_the_floor_and_stops_at_the_budget():
    """Capacities a session's slabs take as it grows: the first fits the save in the
    smallest slab * 2^k, later ones double the current capacity first."""
    from marathon_amd.shift_store import _doubled

    for floor in (1, 3, 256, 2048):
        for want in (1, floor, floor + 1, 3 * floor, 4 * floor, 4 * floor + 1, 1000 * floor):
            size = floor
            while size < want:
                size *= 2
            assert _doubled(floor, want) == size
    st = ShiftStore(budget_tokens=20000, device="cpu", allocate=False, slab=1000)
    caps = []
    for end in (10, 1000, 1001, 2500, 4001, 9000, 17000):
        assert st.reserve("a", 0, end)
        caps.append(st._sessions["a"].capacity)
    assert caps == [1000, 1000, 2000, 4000, 8000, 16000, 20000]


def test_growth_evicts_least_recently_used_others_until_it_fits():
    """Three sessions fill the budget; touching one through ``covers`` (the scheduler)
    or ``read`` (the worker) makes it the last to go when a fourth grows."""
    for touch in ("covers", "read"):
        st = ShiftStore(budget_tokens=8, device="cpu", slab=2)
        for s in ("a", "b", "c"):
            assert st.reserve(s, 0, 2)
            st.write(s, "l0", 0, torch.zeros(2, 1, 2))
        if touch == "covers":
            assert st.covers("a", 0, 2)
        else:
            assert st.read("a", "l0", 0, 2) is not None
        assert st.reserve("d", 0, 2) and st.evictions == 0  # 8 of 8 used
        assert st.reserve("d", 2, 2)  # d grows 2 -> 4: evicts b (oldest untouched)
        assert list(st._sessions) == ["c", "a", "d"] and st.evictions == 1
        assert st.reserve("d", 4, 1)  # 4 -> 8: evicts c, then a
        assert list(st._sessions) == ["d"] and st.evictions == 3
        assert st.stats()["used_tokens"] == 8
