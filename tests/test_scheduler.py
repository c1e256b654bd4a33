"""The connector's scheduler half (``connector.ShiftScheduler``) on the CPU.

The reference tests these decisions through a fingerprint engine whose "KV" of the
token at position p is the token id (tests/test_paged_depth.py:53-180): re-rotation is
exact in that model, so a wrong id means wrong coordinates.  Here the same model runs
with every decision taken by ``ShiftScheduler`` over a tensor-free mirror store, and a
worker that applies each step's loads and saves to a CPU store and a CPU paged cache.
The kernels are not involved; the GPU session test runs the same scheduler against them.
"""

from __future__ import annotations

import pytest
import torch

from marathon_amd import BlockShiftStore, ShiftStore, slots
from marathon_amd.connector import ShiftScheduler

BS = 16
FILLER = "deterministic filler that makes a message worth several blocks of tokens "


class FingerprintWorker:
    """A paged cache of token ids with vLLM's block-level prefix caching; every
    connector decision comes from the scheduler."""

    def __init__(self, device_slots: bool, store: str = "flat"):
        if store == "flat":
            self.store = ShiftStore(1 << 20, device="cpu")
            mirror = ShiftStore(1 << 20, allocate=False)
        else:
            self.store = BlockShiftStore(1 << 16, device="cpu", block_size=BS)
            mirror = BlockShiftStore(1 << 16, allocate=False, block_size=BS)
        self.sched = ShiftScheduler(mirror, BS, device_slots=device_slots)
        self.paged: list[int] = []
        self.prefix: dict[tuple, int] = {}
        self.corruptions: list[tuple] = []
        self.saves: list[tuple] = []  # (request, lo, hi)
        self.loads: list[tuple] = []  # (request, dst lo, n, delta)
        self.n_req = 0

    def _new_block(self) -> int:
        self.paged.extend([0] * BS)
        return len(self.paged) // BS - 1

    def _blocks_for(self, ids):
        blocks, hit, broken = [], 0, False
        for k in range(-(-len(ids) // BS)):
            cached = None if broken else self.prefix.get(tuple(ids[: (k + 1) * BS]))
            if cached is not None and (k + 1) * BS <= len(ids):
                blocks.append(cached)
                hit = (k + 1) * BS
            else:
                broken = True
                blocks.append(self._new_block())
        return blocks, hit

    @staticmethod
    def _slots(item, lo):
        if item.slots is not None:
            return item.slots.tolist()
        return slots(list(item.block_ids), lo, lo + item.n, BS).tolist()

    def _run_loads(self, rid, meta):
        for ld in meta.loads:
            lo = ld.src_start + ld.delta
            src = self.store.read(ld.session, "L0", ld.src_start, ld.n)
            assert src is not None, "the scheduler planned a load the worker's store lacks"
            for s, v in zip(self._slots(ld, lo), src[:, 0, 0].tolist(), strict=True):
                self.paged[s] = int(v)
            self.loads.append((rid, lo, ld.n, ld.delta))

    def _run_saves(self, rid, meta):
        for sv in meta.saves:
            # the worker's reserve mirrors the scheduler's (vllm_shift_connector.py:546-553)
            assert self.store.reserve(sv.session, sv.dst_start, sv.n)
            vals = [self.paged[s] for s in self._slots(sv, sv.dst_start)]
            # rows [heads=1, 2D=2]: the token's fingerprint as its K and its V
            self.store.write(sv.session, "L0", sv.dst_start,
                             torch.tensor(vals, dtype=torch.float32).reshape(-1, 1, 1)
                             .expand(-1, 1, 2).contiguous())
            self.saves.append((rid, sv.dst_start, sv.dst_start + sv.n))

    def generate(self, ids, session, max_tokens, load=None, save=False):
        rid = f"r{self.n_req}"
        self.n_req += 1
        blocks, hit = self._blocks_for(ids)
        self.sched.on_new_request(rid, {"session": session, "load": load, "save": save})
        ext, async_load = self.sched.get_num_new_matched_tokens(rid, hit, len(ids))
        assert async_load is False
        self.sched.update_state_after_alloc(rid, ext)
        computed = hit + ext
        meta = self.sched.build_connector_meta(
            new_reqs=[(rid, blocks, computed, len(ids) - computed)])
        self._run_loads(rid, meta)
        for s, v in zip(slots(blocks, computed, len(ids), BS).tolist(), ids[computed:],
                        strict=True):
            self.paged[s] = v
        for pos, s in enumerate(slots(blocks, 0, len(ids), BS).tolist()):
            if self.paged[s] != ids[pos]:
                self.corruptions.append((rid, pos, ids[pos], self.paged[s]))
        self._run_saves(rid, meta)
        for k in range(max_tokens):
            cur = len(ids) + k
            new = None
            if cur // BS >= len(blocks):
                new = [self._new_block()]
                blocks.append(new[0])
            self.paged[slots(blocks, cur, cur + 1, BS).item()] = 1
            meta = self.sched.build_connector_meta(cached_reqs=[(rid, new, cur, 1)])
            assert not meta.loads
            self._run_saves(rid, meta)
        self.sched.build_connector_meta(finished=[rid])
        for k in range(len(ids) // BS):
            self.prefix.setdefault(tuple(ids[: (k + 1) * BS]), blocks[k])
        return rid


def _prompt(messages):
    pieces = [list(f"{m['role']}: {m['content']}\n".encode()) for m in messages]
    return [i for p in pieces for i in p] + [10], pieces


def _front_edit_session(w: FingerprintWorker, turns: int, keep_last: int = 4, max_tokens=3):
    """Demote the oldest live message every turn (test_paged_depth.py:183-197): a
    front-of-view shrink edit, served as the reference's two phases (reuse_plan.py:312-342):
    a prefix request up to the reused span, then the full prompt with the load."""
    messages, prev, rows = [], None, []
    for t in range(turns):
        load = None
        if t >= keep_last:
            i = 2 * (t - keep_last)
            messages[i] = {"role": "user", "content": f"[cold #{t - keep_last} {t:08x}]"}
            new = _prompt(messages)[1]
            old_start = sum(len(p) for p in prev[: i + 1])
            new_start = sum(len(p) for p in new[: i + 1])
            end = new_start + sum(len(p) for p in prev[i + 1:])
            load = {"dst_start": new_start, "dst_end": end, "delta": new_start - old_start}
        messages.append({"role": "user", "content": f"Turn {t}. {FILLER * 3}"})
        ids, prev = _prompt(messages)
        lo = -(-load["dst_start"] // BS) * BS if load else 0
        hi = load["dst_end"] // BS * BS if load else 0
        if load and hi - lo >= BS and 0 < lo and hi < len(ids):
            w.generate(ids[:lo], "s", 1)
            rid = w.generate(ids, "s", max_tokens, load={**load, "dst_start": lo, "dst_end": hi},
                             save="full")
        else:
            rid = w.generate(ids, "s", max_tokens, save="full" if t else True)
        rows.append((rid, len(ids), load))
        messages.append({"role": "assistant", "content": f"ok {t}"})
    return rows


@pytest.mark.parametrize("device_slots,store", [(False, "flat"), (True, "flat"),
                                                (True, "blocks")])
def test_front_edits_keep_every_coordinate(device_slots, store):
    """Thirty consecutive front edits: every position of every prompt holds its own
    token, loads actually happen, with negative deltas, and nothing is declined."""
    w = FingerprintWorker(device_slots, store)
    _front_edit_session(w, 30)
    assert w.corruptions == [], w.corruptions[:3]
    assert w.sched.declines == []
    assert len(w.loads) >= 20
    assert all(d < 0 for _, _, _, d in w.loads)


def test_full_save_is_one_shot():
    """``save="full"`` widens the prefill step's save to [0, hi) once; the decode steps
    then save one position each (vllm_shift_connector.py:296-330)."""
    w = FingerprintWorker(False)
    rows = _front_edit_session(w, 8, max_tokens=40)
    for rid, n_prompt, load in rows:
        mine = [(lo, hi) for r, lo, hi in w.saves if r == rid]
        if not mine:
            continue
        assert mine[0] == (0, n_prompt)  # "full" (or the first turn's plain True from 0)
        assert mine[1:] == [(n_prompt + k, n_prompt + k + 1) for k in range(40)]


def test_second_writer_of_a_session_runs_without_reuse():
    """One in-flight writer per session (vllm_shift_connector.py:211-223): a second
    request of the session neither loads nor saves until the first finishes."""
    w = FingerprintWorker(False)
    ids = list(range(1, 100))
    w.generate(ids, "s", 0, save=True)
    s = w.sched
    s.on_new_request("a", {"session": "s", "save": True})
    s.on_new_request("b", {"session": "s", "save": True,
                           "load": {"dst_start": 0, "dst_end": 96, "delta": 0}})
    assert s.get_num_new_matched_tokens("b", 0, 120) == (0, False)
    s.update_state_after_alloc("b", 0)
    meta = s.build_connector_meta(new_reqs=[("a", list(range(100, 108)), 99, 20),
                                            ("b", list(range(108, 116)), 99, 20)])
    assert meta.loads == [] and [(sv.session, sv.dst_start) for sv in meta.saves] == [("s", 99)]
    s.request_finished("a")
    s.on_new_request("c", {"session": "s", "load": {"dst_start": 0, "dst_end": 96, "delta": 0}})
    assert s.get_num_new_matched_tokens("c", 0, 120) == (96, False)


def test_no_session_is_a_pass_through():
    s = ShiftScheduler(ShiftStore(1 << 16, allocate=False), BS)
    s.on_new_request("r", None)
    assert s.get_num_new_matched_tokens("r", 0, 200) == (0, False)
    meta = s.build_connector_meta(new_reqs=[("r", [0, 1], 0, 20)],
                                  cached_reqs=[("r", [2], 20, 1)], finished=["r"])
    assert meta.loads == [] and meta.saves == []
    assert s.declines == []


def test_load_and_saves_of_a_step_share_one_block_table():
    """Device-side slots: a request's load and save in one step carry the same table
    object, so the worker uploads it once; the next step gets a fresh snapshot."""
    s = ShiftScheduler(ShiftStore(1 << 16, allocate=False), BS)
    assert s.store.reserve("s", 0, 200)
    s.on_new_request("r", {"session": "s", "save": True,
                           "load": {"dst_start": 32, "dst_end": 160, "delta": -5}})
    assert s.get_num_new_matched_tokens("r", 32, 181) == (128, False)
    s.update_state_after_alloc("r", 128)
    blocks = [9, 4, 7, 1, 3, 8, 2, 6, 5, 0, 11, 12]
    meta = s.build_connector_meta(new_reqs=[("r", blocks, 160, 21)])
    (ld,), (sv,) = meta.loads, meta.saves
    assert ld.slots is None and ld.block_ids is sv.block_ids
    assert (ld.src_start, ld.delta, ld.paged_pos, ld.n) == (37, -5, 32, 128)
    assert (sv.dst_start, sv.n) == (160, 21)
    assert list(ld.block_ids) == blocks
    meta2 = s.build_connector_meta(cached_reqs=[("r", [13], 181, 12)])
    (sv2,) = meta2.saves
    assert sv2.block_ids is not sv.block_ids and list(sv2.block_ids) == blocks + [13]
    assert list(sv.block_ids) == blocks  # the earlier step's table is unchanged


def test_host_slots_match_the_reference_lists():
    """``device_slots=False`` builds the reference's host slot lists (:349-366, :320)."""
    s = ShiftScheduler(ShiftStore(1 << 16, allocate=False), BS, device_slots=False)
    assert s.store.reserve("s", 0, 200)
    s.on_new_request("r", {"session": "s", "save": "full",
                           "load": {"dst_start": 16, "dst_end": 96, "delta": 7}})
    assert s.get_num_new_matched_tokens("r", 16, 120) == (80, False)
    s.update_state_after_alloc("r", 80)
    blocks = [5, 3, 8, 1, 0, 2, 4, 6]
    meta = s.build_connector_meta(new_reqs=[("r", blocks, 96, 24)])
    (ld,), (sv,) = meta.loads, meta.saves
    assert torch.equal(ld.slots, slots(blocks, 16, 96, BS)) and ld.src_start == 9
    assert sv.dst_start == 0 and torch.equal(sv.slots, slots(blocks, 0, 120, BS))
    assert s._params["r"]["save"] is True  # the one-shot downgrade


def _random_edit_sessions(w: FingerprintWorker, seed: int, turns: int, sessions: int):
    """Sessions taking turns; each turn may rewrite any earlier message (shorter or
    longer), and the reused span is what the previous prompt held after it."""
    import numpy as np

    rng = np.random.default_rng(seed)
    state = {f"s{k}": ([], None) for k in range(sessions)}
    edits = 0
    for t in range(turns):
        name = f"s{int(rng.integers(sessions))}"
        messages, prev = state[name]
        load = None
        if prev is not None and messages and rng.random() < 0.7:
            i = int(rng.integers(len(messages)))
            messages[i] = {"role": messages[i]["role"],
                           "content": f"edit {t} " + "x" * int(rng.integers(0, 120))}
            new = _prompt(messages)[1]
            old_start = sum(len(p) for p in prev[: i + 1])
            new_start = sum(len(p) for p in new[: i + 1])
            end = new_start + sum(len(p) for p in prev[i + 1:])
            if end > new_start:
                load = {"dst_start": new_start, "dst_end": end, "delta": new_start - old_start}
        messages.append({"role": "user", "content": f"{name} turn {t}. " + FILLER *
                         int(rng.integers(1, 4))})
        ids, pieces = _prompt(messages)
        lo = -(-load["dst_start"] // BS) * BS if load else 0
        hi = load["dst_end"] // BS * BS if load else 0
        n_out = int(rng.integers(0, 6))
        if load and hi - lo >= BS and 0 < lo and hi < len(ids):
            edits += 1
            w.generate(ids[:lo], name, 1)
            w.generate(ids, name, n_out, load={**load, "dst_start": lo, "dst_end": hi},
                       save="full")
        else:
            w.generate(ids, name, n_out, save="full")
        messages.append({"role": "assistant", "content": f"ok {t} " + "y" * int(rng.integers(0, 40))})
        state[name] = (messages, pieces)
    return edits


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("store,budget", [("flat", 1 << 20), ("blocks", 1 << 16),
                                          ("flat", 6000), ("blocks", 6000)])
def test_random_edit_sessions_keep_every_coordinate(seed, store, budget):
    """Edits anywhere in the history, of any length, in three interleaved sessions, with
    stores large enough for all of them or small enough to evict: every position of
    every prompt still holds its own token.  A load the store can no longer serve is
    declined (and recomputed), never guessed at; with room for every session, edit
    turns reuse."""
    w = FingerprintWorker(seed % 2 == 1, store)
    if budget != (1 << 20 if store == "flat" else 1 << 16):
        if store == "flat":
            w.store = ShiftStore(budget, device="cpu")
            w.sched.store = ShiftStore(budget, allocate=False)
        else:
            w.store = BlockShiftStore(budget, device="cpu", block_size=BS)
            w.sched.store = BlockShiftStore(budget, allocate=False, block_size=BS)
    edits = _random_edit_sessions(w, seed, 24, 3)
    assert w.corruptions == [], w.corruptions[:3]
    assert all("store no longer holds" in why or "local hit" in why for why in w.sched.declines), \
        w.sched.declines[:3]
    if budget >= 1 << 16:  # room for every session: every edit turn reuses
        assert len(w.loads) == edits > 0, (len(w.loads), edits, w.sched.declines[:3])
