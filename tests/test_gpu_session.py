"""End-to-end paged sessions on the GPU: the real store, planners, loader and saver.

The reference's CPU harness (tests/test_paged_depth.py:53-180, FingerprintEngine) models
KV as the token id, which proves placement but never values.  Here every token's KV is
real: K at position p is RoPE(table_k[token], p) (bf16), V is table_v[token].  A
session of front-of-view edits -- the oldest message demoted to a stub every turn, so
every turn shifts the rest of the history left -- runs through plan_load, the HIP
loader (re-rotation), a prefill of what is left, and per-step saves through the HIP
saver (paged -> store).  After every request every position of every layer is checked:
V bit-exact, K within the rounding that its history of shifts allows.
"""

from __future__ import annotations

import pytest
import torch

from marathon_amd import BlockShiftStore, ShiftStore, plan_load, plan_save, slots
from marathon_amd.connector import Load, Save, ShiftLoader, ShiftSaver, ShiftScheduler
from marathon_amd.shift_kernels import inv_freq_for

pytestmark = pytest.mark.gpu

H, D, BS, LAYERS = 8, 128, 16, 4
FILLER = "deterministic filler that makes a message worth several blocks of tokens "


class RealKVEngine:
    """A paged KV cache with block-level prefix caching, driven by the real decisions."""

    def __init__(self, dev, blocks=1024, seed=0, store="flat", device_slots=False,
                 budget=None):
        self.dev = dev
        self.device_slots = device_slots
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.table_k = torch.randn(256, H, D, dtype=torch.float64, device=dev, generator=g)
        self.table_v = torch.randn(256, H, D, device=dev, generator=g).to(torch.bfloat16)
        self.inv = inv_freq_for(D, 1e6)
        self.inv64 = self.inv.to(dev, torch.float64)
        self.kv = {f"layer{i}": torch.zeros(blocks, H, BS, 2 * D, dtype=torch.bfloat16, device=dev)
                   for i in range(LAYERS)}
        self.budget = budget or (1 << 16 if store == "flat" else 1 << 14)
        if store == "flat":
            self.store = ShiftStore(budget_tokens=self.budget, device=str(dev), slab=1024)
        else:
            self.store = BlockShiftStore(budget_tokens=self.budget, device=str(dev),
                                         block_size=BS)
        self.loader = ShiftLoader(self.store, BS, self.inv)
        self.loader.register_kv_caches(self.kv)
        self.saver = ShiftSaver(self.store, BS)
        self.next_block = 0
        self.n_blocks = blocks
        self.prefix: dict[tuple, int] = {}
        self.shifts = torch.zeros(blocks * BS, dtype=torch.int32)  # per slot: re-rotations
        self.store_shifts: dict[str, torch.Tensor] = {}
        self.loads = 0
        self.declines: list[str] = []

    # -- model: fresh KV of tokens at positions
    def fresh(self, ids: torch.Tensor, pos: torch.Tensor):
        ang = pos.to(self.dev, torch.float64)[:, None] * self.inv64[None, :]
        emb = torch.cat((ang, ang), -1)[:, None, :]
        base = self.table_k[ids.to(self.dev)]
        rot = torch.cat((-base[..., D // 2:], base[..., : D // 2]), -1)
        return base * emb.cos() + rot * emb.sin(), self.table_v[ids.to(self.dev)]

    def _write_fresh(self, blocks, ids, lo, hi):
        if hi <= lo:
            return
        # host-side bound: the paged cache holds n_blocks blocks (torch indexing on the
        # device must never go out of range)
        assert self.next_block <= self.n_blocks, "the test ran out of paged blocks"
        sl = slots(blocks, lo, hi, BS)
        k, v = self.fresh(torch.tensor(ids[lo:hi]), torch.arange(lo, hi))
        row = torch.cat((k.to(torch.bfloat16), v), -1)
        s = sl.to(self.dev)
        for cache in self.kv.values():
            cache[s // BS, :, s % BS] = row
        self.shifts[sl] = 0

    def _blocks_for(self, ids):
        blocks, hit, broken = [], 0, False
        for k in range(-(-len(ids) // BS)):
            key = tuple(ids[: (k + 1) * BS])
            cached = None if broken else self.prefix.get(key)
            if cached is not None and (k + 1) * BS <= len(ids):
                blocks.append(cached)
                hit = (k + 1) * BS
            else:
                broken = True
                blocks.append(self.next_block)
                self.next_block += 1
        # host-side bound, before any load or save addresses these blocks
        assert self.next_block <= self.n_blocks, "the test ran out of paged blocks"
        return blocks, hit

    def _verify(self, blocks, ids):
        n = len(ids)
        sl = slots(blocks, 0, n, BS)
        k_want, v_want = self.fresh(torch.tensor(ids), torch.arange(n))
        s = sl.to(self.dev)
        nshift = self.shifts[sl].to(self.dev, torch.float64)[:, None, None]
        m = torch.maximum(k_want.abs(), torch.roll(k_want, D // 2, -1).abs())
        bound = 2.0**-8 * (2 + 2 * nshift) * m + 1e-6
        for name, cache in self.kv.items():
            got = cache[s // BS, :, s % BS]
            assert torch.equal(got[..., D:], v_want), f"{name}: V differs"
            err = (got[..., :D].to(torch.float64) - k_want).abs()
            assert bool((err <= bound).all()), f"{name}: K beyond its rounding bound"

    def _save(self, params, blocks, lo, hi, session):
        window = plan_save(self.store, session, params.get("save"), lo, hi)
        if window is None:
            return
        if params.get("save") == "full":
            params["save"] = True
        lo, hi = window
        sl = slots(blocks, lo, hi, BS)
        sv = Save.from_blocks(session, list(blocks), lo, hi) if self.device_slots else Save(
            session, sl, lo)
        assert self.saver.save_all(self.kv, [sv]) == (hi - lo) * LAYERS
        st = self.store_shifts.setdefault(session, torch.zeros(1 << 16, dtype=torch.int32))
        st[lo:hi] = self.shifts[sl]

    def generate(self, ids, session, max_tokens, load=None, save=False):
        blocks, num_computed = self._blocks_for(ids)
        params = {"save": save}
        decision, why = plan_load(self.store, session, load, num_computed, len(ids), BS)
        if load and decision is None:
            self.declines.append(why)
        if decision is not None:
            sl = slots(blocks, decision.lo, decision.hi, BS)
            if self.device_slots:
                ld = Load.from_blocks(session, list(blocks), decision.lo, decision.hi,
                                      decision.delta)
            else:
                ld = Load(session, sl, decision.src_start, decision.delta)
            assert self.loader.start_load_kv([ld]) == len(sl) * LAYERS
            st = self.store_shifts[session]
            self.shifts[sl] = st[decision.src_start:decision.src_start + len(sl)] + int(
                decision.delta != 0)
            num_computed = decision.hi
            self.loads += 1
        self._write_fresh(blocks, ids, num_computed, len(ids))
        torch.cuda.synchronize(self.dev)
        self._verify(blocks, ids)
        self._save(params, blocks, num_computed, len(ids), session)
        cur_ids = list(ids)
        for _ in range(max_tokens):
            cur = len(cur_ids)
            if cur // BS >= len(blocks):
                blocks.append(self.next_block)
                self.next_block += 1
            cur_ids.append(1)
            self._write_fresh(blocks, cur_ids, cur, cur + 1)
            self._save(params, blocks, cur, cur + 1, session)
        for k in range(len(ids) // BS):
            self.prefix.setdefault(tuple(ids[: (k + 1) * BS]), blocks[k])
        torch.cuda.synchronize(self.dev)


class ScheduledKVEngine(RealKVEngine):
    """The same engine with every decision taken by ``ShiftScheduler``, the connector's
    scheduler half, over a tensor-free mirror of the worker's store: the engine only
    reports what vLLM's scheduler would (prefix hit, blocks, tokens per step), and the
    worker runs each step's loads before the forward and its saves after it."""

    def __init__(self, dev, store="flat", device_slots=False, **kw):
        super().__init__(dev, store=store, device_slots=device_slots, **kw)
        if store == "flat":
            mirror = ShiftStore(budget_tokens=self.budget, allocate=False, slab=1024)
        else:
            mirror = BlockShiftStore(budget_tokens=self.budget, allocate=False, block_size=BS)
        self.sched = ShiftScheduler(mirror, BS, device_slots=device_slots)
        self.n_req = 0

    @staticmethod
    def _paged(item, lo):
        if item.slots is not None:
            return item.slots
        return slots(list(item.block_ids), lo, lo + item.n, BS)

    def _run_loads(self, meta):
        if not meta.loads:
            return
        assert self.loader.start_load_kv(meta.loads) == sum(ld.n for ld in meta.loads) * LAYERS
        for ld in meta.loads:
            sl = self._paged(ld, ld.src_start + ld.delta)
            st = self.store_shifts[ld.session]
            self.shifts[sl] = st[ld.src_start:ld.src_start + ld.n] + int(ld.delta != 0)
            self.loads += 1

    def _run_saves(self, meta):
        if not meta.saves:
            return
        assert self.saver.save_all(self.kv, meta.saves) == sum(sv.n for sv in meta.saves) * LAYERS
        for sv in meta.saves:
            sl = self._paged(sv, sv.dst_start)
            st = self.store_shifts.setdefault(sv.session, torch.zeros(1 << 16, dtype=torch.int32))
            st[sv.dst_start:sv.dst_start + sv.n] = self.shifts[sl]

    def generate(self, ids, session, max_tokens, load=None, save=False):
        rid = f"req{self.n_req}"
        self.n_req += 1
        blocks, hit = self._blocks_for(ids)
        self.sched.on_new_request(rid, {"session": session, "load": load, "save": save})
        ext, _ = self.sched.get_num_new_matched_tokens(rid, hit, len(ids))
        self.sched.update_state_after_alloc(rid, ext)
        computed = hit + ext
        meta = self.sched.build_connector_meta(new_reqs=[(rid, blocks, computed,
                                                          len(ids) - computed)])
        assert len(meta.loads) == int(ext > 0)
        self._run_loads(meta)
        self._write_fresh(blocks, ids, computed, len(ids))
        torch.cuda.synchronize(self.dev)
        self._verify(blocks, ids)
        self._run_saves(meta)
        cur_ids = list(ids)
        for _ in range(max_tokens):
            cur = len(cur_ids)
            new = None
            if cur // BS >= len(blocks):
                new = [self.next_block]
                blocks.append(self.next_block)
                self.next_block += 1
            meta = self.sched.build_connector_meta(cached_reqs=[(rid, new, cur, 1)])
            assert not meta.loads
            cur_ids.append(1)
            self._write_fresh(blocks, cur_ids, cur, cur + 1)
            self._run_saves(meta)
        self.sched.request_finished(rid)
        for k in range(len(ids) // BS):
            self.prefix.setdefault(tuple(ids[: (k + 1) * BS]), blocks[k])
        torch.cuda.synchronize(self.dev)
        self.declines = self.sched.declines


class ConnectorKVEngine(RealKVEngine):
    """Every decision and every copy through the connector object as vLLM drives it: one
    ``MarathonShiftConnector`` per role, the scheduler's hooks fed vLLM-shaped requests
    and scheduler outputs, the worker's hooks a forward context whose attention layers
    hold the paged caches (stand-ins: tests/vllm_fakes.py).  Saves go through the
    per-layer ``save_kv_layer`` hook and are flushed by ``wait_for_save``."""

    def __init__(self, dev, store="blocks", device_slots=True, **kw):
        from marathon_amd.vllm_connector import MarathonShiftConnector
        from tests import vllm_fakes as F

        super().__init__(dev, store=store, device_slots=True, **kw)
        self.F = F
        extra = {"store_layout": "block" if store == "blocks" else "flat",
                 "store_tokens": self.budget, "store_device": str(dev)}
        cfg = F.vllm_config(block_size=BS, extra=extra)
        self.sched = MarathonShiftConnector(cfg, "scheduler")
        self.worker = MarathonShiftConnector(cfg, "worker")
        self.store = self.worker.store
        self.fwd = F.forward_context(self.kv)
        self.n_req = 0
        self.loaded_tokens = 0

    def _step(self, meta, ids, lo, hi, blocks):
        """One forward pass: loads, the computed tokens' fresh KV, per-layer saves."""
        w = self.worker
        w.bind_connector_metadata(meta)
        w.start_load_kv(self.fwd)
        for ld in meta.loads:
            sl = ScheduledKVEngine._paged(ld, ld.src_start + ld.delta)
            st = self.store_shifts[ld.session]
            self.shifts[sl] = st[ld.src_start:ld.src_start + ld.n] + int(ld.delta != 0)
            self.loads += 1
            self.loaded_tokens += ld.n
        self._write_fresh(blocks, ids, lo, hi)
        for name, cache in self.kv.items():
            w.save_kv_layer(name, cache, None)
        w.wait_for_save()
        for sv in meta.saves:
            sl = ScheduledKVEngine._paged(sv, sv.dst_start)
            st = self.store_shifts.setdefault(sv.session, torch.zeros(1 << 16, dtype=torch.int32))
            st[sv.dst_start:sv.dst_start + sv.n] = self.shifts[sl]
        w.clear_connector_metadata()

    def generate(self, ids, session, max_tokens, load=None, save=False):
        F = self.F
        rid = f"req{self.n_req}"
        self.n_req += 1
        blocks, hit = self._blocks_for(ids)
        req = F.Request(rid, {"session": session, "load": load, "save": save}, len(ids))
        self.sched.on_new_request(req)
        ext, is_async = self.sched.get_num_new_matched_tokens(req, hit)
        assert is_async is False
        self.sched.update_state_after_alloc(req, None, ext)
        computed = hit + ext
        meta = self.sched.build_connector_meta(
            F.step_output(new=[(rid, blocks, computed, len(ids) - computed)]))
        assert len(meta.loads) == int(ext > 0)
        self._step(meta, ids, computed, len(ids), blocks)
        torch.cuda.synchronize(self.dev)
        self._verify(blocks, ids)
        cur_ids = list(ids)
        for _ in range(max_tokens):
            cur = len(cur_ids)
            new = None
            if cur // BS >= len(blocks):
                new = [self.next_block]
                blocks.append(self.next_block)
                self.next_block += 1
            meta = self.sched.build_connector_meta(F.step_output(cached=[(rid, new, cur, 1)]))
            assert not meta.loads
            cur_ids.append(1)
            self._step(meta, cur_ids, cur, cur + 1, blocks)
        assert self.sched.request_finished(req, blocks) == (False, None)
        for k in range(len(ids) // BS):
            self.prefix.setdefault(tuple(ids[: (k + 1) * BS]), blocks[k])
        torch.cuda.synchronize(self.dev)
        self.declines = self.sched._sched.declines


def _prompt(messages):
    pieces = [list(f"{m['role']}: {m['content']}\n".encode()) for m in messages]
    return [i for p in pieces for i in p] + [10], pieces


def _phases(load, n_prompt):
    """The reference's phases() for one segment (reuse_plan.py:312-342)."""
    lo = -(-load["dst_start"] // BS) * BS
    hi = load["dst_end"] // BS * BS
    if not (hi - lo >= BS and lo > 0 and hi < n_prompt):
        return []
    return [(lo, None), (n_prompt, {"dst_start": lo, "dst_end": hi, "delta": load["delta"]})]


@pytest.mark.parametrize("store,device_slots,engine", [
    ("flat", False, RealKVEngine), ("flat", True, RealKVEngine),
    ("blocks", False, RealKVEngine), ("blocks", True, RealKVEngine),
    ("flat", False, ScheduledKVEngine), ("blocks", True, ScheduledKVEngine),
    ("blocks", True, ConnectorKVEngine), ("flat", True, ConnectorKVEngine)])
def test_front_edits_through_the_real_kernels(gpu, store, device_slots, engine):
    """``ScheduledKVEngine`` takes every decision through the connector's scheduler
    half, ``ConnectorKVEngine`` every decision and copy through the connector object's
    hooks; the others call the planners directly."""
    eng = engine(gpu, store=store, device_slots=device_slots)
    messages, keep_last, turns = [], 3, 9
    prompt_pieces = None  # pieces of the previous request's prompt: what the store holds
    for t in range(turns):
        print(f"case session {engine.__name__} store={store} device_slots={device_slots} "
              f"turn {t}", flush=True)
        load = None
        if t >= keep_last:
            d = t - keep_last
            i = 2 * d  # the oldest live user message (user/assistant alternate)
            old_pieces = prompt_pieces
            messages[i] = {"role": "user", "content": f"[cold #{d} {d:08x}]"}
            new_pieces = _prompt(messages)[1]
            # reused: the messages after the edited one that the previous prompt held
            # (the assistant reply appended since then was never in the store)
            old_start = sum(len(p) for p in old_pieces[: i + 1])
            new_start = sum(len(p) for p in new_pieces[: i + 1])
            end = new_start + sum(len(p) for p in old_pieces[i + 1:])
            load = {"dst_start": new_start, "dst_end": end, "delta": new_start - old_start}
        messages.append({"role": "user", "content": f"Turn {t}. {FILLER * 3}"})
        ids, pieces = _prompt(messages)
        prompt_pieces = pieces
        phases = _phases(load, len(ids)) if load else []
        if phases:
            for length, ld in phases[:-1]:
                eng.generate(ids[:length], "s", 1, load=ld)
            eng.generate(ids, "s", 3, load=phases[-1][1], save="full")
        else:
            eng.generate(ids, "s", 3, save="full" if t else True)
        messages.append({"role": "assistant", "content": f"ok {t}"})
    assert eng.loads >= turns - keep_last - 1, (eng.loads, eng.declines)
    assert int(eng.shifts.max()) >= 2  # some KV was re-rotated more than once
    if engine is ConnectorKVEngine:
        from marathon_amd.vllm_connector import merged_stats

        sched, worker = eng.sched.store.stats(), eng.worker.store.stats()
        # the scheduler's mirror and the worker's store took the same decisions
        assert sched["sessions"] == worker["sessions"]
        assert sched["hits"] == eng.loads  # one coverage check per load served
        assert worker["loaded_token_layers"] == eng.loaded_tokens * LAYERS
        merged = merged_stats([eng.sched.store, eng.worker.store])
        assert merged["sessions"] == worker["sessions"]
        assert merged["saved_token_layers"] == worker["saved_token_layers"]


def test_saver_matches_a_torch_gather(gpu):
    """save_all / save_kv_layer land exactly the paged rows (both layouts)."""
    for hnd in (True, False):
        print(f"case saver hnd={hnd}", flush=True)
        g = torch.Generator(device=gpu)
        g.manual_seed(int(hnd))
        shape = (64, H, BS, 2 * D) if hnd else (64, BS, H, 2 * D)
        kv = {f"l{i}": torch.randn(shape, device=gpu, generator=g).to(torch.bfloat16)
              for i in range(3)}
        store = ShiftStore(budget_tokens=8192, device=str(gpu), slab=512)
        saver = ShiftSaver(store, BS)
        perm = torch.randperm(64).tolist()
        sa = Save("a", slots(perm[:20], 5, 5 + 300, BS), 0)
        sb = Save("b", slots(perm[20:], 16, 16 + 200, BS), 16)
        assert store.reserve("b", 0, 16)  # "b" holds [0, 16) already
        n = saver.save_all(kv, [sa, sb])
        assert n == 500 * 3
        layer_rows = saver.save_kv_layer("l0", kv["l0"], [Save("a", slots(perm[:20], 5, 5 + 300, BS), 0)])
        assert layer_rows == 300
        torch.cuda.synchronize(gpu)
        for name, cache in kv.items():
            src = cache.permute(0, 2, 1, 3) if hnd else cache
            for sv in (sa, sb):
                s = sv.slots.to(gpu)
                want = src[s // BS, s % BS]
                got = store.read(sv.session, name, sv.dst_start, s.numel())
                assert torch.equal(got, want), (hnd, name, sv.session)


@pytest.mark.parametrize("store_bs", [16, 32])
def test_block_store_saver_and_loader_match_torch(gpu, store_bs):
    """Saves into the block store's pool (host slots and block tables), read back
    through the store, then a load out of the pool: bytes equal a torch gather.  The
    store's blocks need not be the paged cache's size."""
    g = torch.Generator(device=gpu)
    g.manual_seed(7)
    kv = {f"l{i}": torch.randn(64, H, BS, 2 * D, device=gpu, generator=g).to(torch.bfloat16)
          for i in range(3)}
    store = BlockShiftStore(budget_tokens=4096, device=str(gpu), block_size=store_bs)
    saver = ShiftSaver(store, BS)
    perm = torch.randperm(64).tolist()
    print(f"case block store saves (store blocks of {store_bs})", flush=True)
    assert store.reserve("b", 0, 16)  # "b" holds [0, 16) already
    sa = Save("a", slots(perm[:20], 5, 5 + 300, BS), 0)
    sb = Save.from_blocks("b", perm[20:], 16, 16 + 200)
    assert saver.save_all(kv, [sa, sb]) == 500 * 3
    torch.cuda.synchronize(gpu)
    for name, cache in kv.items():
        src = cache.permute(0, 2, 1, 3)
        for sess, sl, start in (("a", sa.slots, 0), ("b", slots(perm[20:], 16, 216, BS), 16)):
            s = sl.to(gpu)
            assert torch.equal(store.read(sess, name, start, s.numel()), src[s // BS, s % BS])
    print("case block store load, rotated", flush=True)
    out = {name: torch.zeros_like(c) for name, c in kv.items()}
    loader = ShiftLoader(store, BS, inv_freq_for(D, 1e6))
    loader.register_kv_caches(out)
    dst_blocks = torch.randperm(64).tolist()
    n = loader.start_load_kv([Load.from_blocks("a", dst_blocks, 37, 37 + 250, 37),
                              Load.from_blocks("b", dst_blocks, 300, 300 + 100, 290)])
    assert n == 350 * 3
    torch.cuda.synchronize(gpu)
    for name, cache in out.items():
        for sess, lo, hi, delta in (("a", 37, 287, 37), ("b", 300, 400, 290)):
            s = slots(dst_blocks, lo, hi, BS).to(gpu)
            got = cache[s // BS, :, s % BS]
            want = store.read(sess, name, lo - delta, hi - lo)
            assert torch.equal(got[..., D:], want[..., D:])  # V bit-exact
            # K: rotated by delta, within the reference rotation's rounding of the input
            k0 = want[..., :D].to(torch.float64)
            ang = float(delta) * inv_freq_for(D, 1e6).to(gpu, torch.float64)
            emb = torch.cat((ang, ang))
            rot = torch.cat((-k0[..., D // 2:], k0[..., : D // 2]), -1)
            ref = k0 * emb.cos() + rot * emb.sin()
            pair = torch.maximum(k0.abs(), torch.roll(k0, D // 2, -1).abs())
            assert bool(((got[..., :D].to(torch.float64) - ref).abs()
                         <= 2.0**-8 * (ref.abs() + 2 * pair) + 1e-6).all())


def test_block_store_fp8_saves_and_loads_match_oracle(gpu):
    """fp8 through the block store, whose fp8 pools keep rows of K then V per head:
    saves read back bit for bit, and a rotated load out of the pool equals the oracle's
    fp8 rule with each layer's K scale (V raw)."""
    import numpy as np

    from oracle import kvshift_oracle as orc

    print("case block store fp8 saves and loads", flush=True)
    g = torch.Generator(device=gpu)
    g.manual_seed(17)
    scales = {f"l{i}": s for i, s in enumerate((0.031, 0.058, 0.092))}
    kv = {name: (torch.randn(64, H, BS, 2 * D, device=gpu, generator=g) / s)
          .clamp(-448, 448).to(torch.float8_e4m3fn) for name, s in scales.items()}
    store = BlockShiftStore(budget_tokens=4096, device=str(gpu), block_size=BS)
    perm = torch.randperm(64).tolist()
    sa = Save.from_blocks("a", perm[:30], 3, 3 + 400)
    assert ShiftSaver(store, BS).save_all(kv, [sa]) == 400 * 3
    torch.cuda.synchronize(gpu)
    assert store.pool("l0").shape == (store.pool_blocks, BS, H, 2 * D)  # rows, not planes
    for name, cache in kv.items():
        s = slots(perm[:30], 3, 403, BS).to(gpu)
        want = cache.permute(0, 2, 1, 3)[s // BS, s % BS]
        got = store.read("a", name, 3, 400)
        assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), name
    out = {name: torch.zeros_like(c) for name, c in kv.items()}
    loader = ShiftLoader(store, BS, inv_freq_for(D, 1e6), k_scales=scales)
    loader.register_kv_caches(out)
    inv = inv_freq_for(D, 1e6).numpy()
    # the second load runs after a scale changed in the shared dict: the loader's cached
    # scale tensor must follow it
    for step, delta in enumerate((51, 23)):  # sources at 9 and 37, inside the saved [3, 403)
        if step:
            scales["l1"] = 0.071
        dst_blocks = torch.randperm(64).tolist()
        load = Load.from_blocks("a", dst_blocks, 60, 60 + 330, delta)
        assert loader.start_load_kv([load]) == 330 * 3
        torch.cuda.synchronize(gpu)
        for name, cache in out.items():
            s = slots(dst_blocks, 60, 390, BS).to(gpu)
            got = cache[s // BS, :, s % BS].cpu().view(torch.uint8).numpy()
            src = store.read("a", name, 60 - delta, 330).cpu().view(torch.uint8).numpy()
            want_k = orc.rotate_k_bits(src[..., :D], delta, inv, "fp8", scales[name])
            assert np.array_equal(got[..., :D], want_k), (step, name)
            assert np.array_equal(got[..., D:], src[..., D:]), (step, name)


def test_deferred_per_layer_saves_equal_one_save_all(gpu):
    """vLLM's per-layer hook, deferred: save_kv_layer records, wait_for_save launches
    once; the store ends with the same bytes and the same counters as save_all."""
    print("case deferred per-layer saves", flush=True)
    g = torch.Generator(device=gpu)
    g.manual_seed(5)
    kv = {f"l{i}": torch.randn(48, H, BS, 2 * D, device=gpu, generator=g).to(torch.bfloat16)
          for i in range(4)}
    table = torch.randperm(48).tolist()
    stores = [BlockShiftStore(budget_tokens=4096, device=str(gpu), block_size=BS) for _ in range(2)]
    eager = ShiftSaver(stores[0], BS)
    deferred = ShiftSaver(stores[1], BS, deferred=True)
    saves = [Save.from_blocks("s", table, 0, 500)]
    assert eager.save_all(kv, saves) == 500 * 4
    for name, cache in kv.items():
        assert deferred.save_kv_layer(name, cache, saves) == 0
    assert deferred.wait_for_save() == 500 * 4
    assert deferred.wait_for_save() == 0
    torch.cuda.synchronize(gpu)
    assert stores[0].stats() == stores[1].stats()
    for name in kv:
        assert torch.equal(stores[0].read("s", name, 0, 500), stores[1].read("s", name, 0, 500))


@pytest.mark.parametrize("plane_axis", [0, 1])
@pytest.mark.parametrize("store", ["flat", "blocks"])
def test_split_planes_through_the_connector(gpu, store, plane_axis):
    """vLLM caches that keep K and V in separate planes ([2, blocks, bs, heads, D] or
    [blocks, 2, bs, heads, D]) save and load exactly as the fused 4-D cache holding the
    same rows: the same store bytes, the same loaded rows, and the read-back check."""
    print(f"case split planes store={store} axis={plane_axis}", flush=True)
    g = torch.Generator(device=gpu)
    g.manual_seed(17 + plane_axis)
    nblk, layers = 64, 3
    names = [f"l{i}" for i in range(layers)]
    ks = [torch.randn(nblk, BS, H, D, device=gpu, generator=g).to(torch.bfloat16)
          for _ in names]
    vs = [torch.randn(nblk, BS, H, D, device=gpu, generator=g).to(torch.bfloat16)
          for _ in names]
    fused = {n: torch.cat((k, v), dim=-1) for n, k, v in zip(names, ks, vs)}
    split = {n: torch.stack((k, v), dim=plane_axis) for n, k, v in zip(names, ks, vs)}

    def make_store():
        if store == "flat":
            return ShiftStore(budget_tokens=4096, device=str(gpu), slab=512)
        return BlockShiftStore(budget_tokens=4096, device=str(gpu), block_size=BS)

    st_f, st_s = make_store(), make_store()
    table = torch.randperm(nblk, generator=torch.Generator().manual_seed(3)).tolist()
    saves = [Save.from_blocks("s", table, 0, 500)]
    assert ShiftSaver(st_f, BS).save_all(fused, saves) == 500 * layers
    assert ShiftSaver(st_s, BS).save_all(split, saves) == 500 * layers
    torch.cuda.synchronize(gpu)
    for n in names:
        assert torch.equal(st_f.read("s", n, 0, 500), st_s.read("s", n, 0, 500)), n

    inv = inv_freq_for(D, 1e6)
    out_f = {n: torch.zeros_like(t) for n, t in fused.items()}
    out_s = {n: torch.zeros_like(t) for n, t in split.items()}
    lf, ls = ShiftLoader(st_f, BS, inv), ShiftLoader(st_s, BS, inv, verify=True)
    lf.register_kv_caches(out_f)
    ls.register_kv_caches(out_s)
    assert ls.split and ls.layout == "nhd" and not lf.split
    dst = torch.randperm(nblk, generator=torch.Generator().manual_seed(4)).tolist()
    loads = [Load.from_blocks("s", dst, 37, 37 + 250, 37),
             Load.from_blocks("s", dst, 300, 300 + 150, -13)]
    assert lf.start_load_kv(loads) == ls.start_load_kv(loads) == 400 * layers
    torch.cuda.synchronize(gpu)
    for n in names:
        k_out, v_out = (out_s[n][0], out_s[n][1]) if plane_axis == 0 else (
            out_s[n][:, 0], out_s[n][:, 1])
        assert torch.equal(k_out, out_f[n][..., :D]), n
        assert torch.equal(v_out, out_f[n][..., D:]), n
    assert len(ls.verify_log) == 2 * layers
    assert all(e["v_exact"] and e["max_rel"] < 4e-3 for e in ls.verify_log)


# more seeds for a longer sweep: MKV_SESSION_CASES=40 python -m pytest tests/test_gpu_session.py
_SESSION_SEEDS = [5] + list(range(100, 100 + int(__import__("os").environ.get(
    "MKV_SESSION_CASES", "0"))))


@pytest.mark.parametrize("seed", _SESSION_SEEDS)
@pytest.mark.parametrize("budget", [None, 1200])
@pytest.mark.parametrize("store,device_slots,engine", [
    ("flat", False, ScheduledKVEngine), ("blocks", True, ScheduledKVEngine),
    ("blocks", True, ConnectorKVEngine)])
def test_random_edit_sessions_through_the_real_kernels(gpu, store, device_slots, engine,
                                                        budget, seed):
    """Edits anywhere in the history, in three interleaved sessions, every decision
    through the scheduler half (or the connector object's hooks), every load and save
    through the HIP kernels: after every request every position of every layer holds its
    token's KV (V bit-exact, K within its shifts' rounding).  With a 1,200-token store
    the sessions evict one another: freed blocks go to other sessions with stale bytes
    in them, a load the store no longer holds is declined and recomputed, and every
    position must still hold its own token."""
    from tests.test_scheduler import _random_edit_sessions

    print(f"case random edit sessions store={store} device_slots={device_slots} "
          f"engine={engine.__name__} budget={budget} seed={seed}", flush=True)
    eng = engine(gpu, store=store, device_slots=device_slots, budget=budget)
    edits = _random_edit_sessions(eng, seed, 14, 3)
    assert all("store no longer holds" in why or "local hit" in why
               for why in eng.declines), eng.declines[:3]
    if budget is None:  # room for every session: every edit turn reuses
        assert eng.loads == edits, (eng.loads, edits, eng.declines)
    else:
        assert eng.loads <= edits, (eng.loads, edits)
    if seed == _SESSION_SEEDS[0]:  # the default case edits (a sweep's seed may not)
        assert edits > 0
