"""The connector object (marathon_amd.vllm_connector) on the CPU: its constructor reads the
reference's configuration, its scheduler-role hooks take the reference's decisions through
an edit turn, the worker-role hooks are no-ops without work, and ``stats()`` merges the
counters of every store (src/marathon/vllm_shift_connector.py:112-132, :159-389).
Stand-ins for vLLM's objects: tests/vllm_fakes.py."""

from __future__ import annotations

import pytest
import torch

from marathon_amd import BlockShiftStore, ShiftStore
from marathon_amd import vllm_connector as vc
from marathon_amd.connector import Load, Save
from tests import vllm_fakes as F


def _pair(extra=None, **kw):
    cfg = F.vllm_config(extra=extra, **kw)
    return vc.MarathonShiftConnector(cfg, "scheduler"), vc.MarathonShiftConnector(cfg, "worker")


def test_constructor_reads_the_reference_configuration(monkeypatch):
    monkeypatch.delenv("MARATHON_STORE_TOKENS", raising=False)
    sched, worker = _pair({"store_tokens": 4096})
    assert isinstance(sched.store, BlockShiftStore) and isinstance(worker.store, BlockShiftStore)
    assert not sched.store.allocate and worker.store.allocate
    assert sched.store.budget == worker.store.budget == 4096
    assert sched.store.block_size == 16
    flat, _ = _pair({"store_layout": "flat", "session_tokens": 2048})
    assert isinstance(flat.store, ShiftStore) and flat.store.session_cap == 2048
    monkeypatch.setenv("MARATHON_STORE_TOKENS", "1234")
    assert _pair()[0].store.budget == 1234  # extra config, else the variable, else 32,768
    with pytest.raises(ValueError, match="store_layout"):
        _pair({"store_layout": "ring"})
    # inv_freq as the reference builds it (vllm_shift_connector.py:194-199), partial rotary
    part, _ = _pair(head_dim=128, rope_theta=1e4, partial_rotary_factor=0.5)
    want = 1.0 / (1e4 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))
    assert torch.equal(part._inv_freq, want)
    nohd = vc.MarathonShiftConnector(F.vllm_config(head_dim=None), "worker")
    assert nohd._inv_freq.numel() == 64  # head_dim from hidden_size / heads


def test_an_edit_turn_through_the_scheduler_hooks():
    sched, _ = _pair({"store_tokens": 4096})
    r1 = F.Request("r1", {"session": "s", "save": True}, 100)
    sched.on_new_request(r1)
    assert sched.get_num_new_matched_tokens(r1, 0) == (0, False)
    sched.update_state_after_alloc(r1, None, 0)
    meta = sched.build_connector_meta(F.step_output(new=[("r1", range(7), 0, 100)]))
    assert isinstance(meta, vc.ShiftConnectorMetadata) and not meta.loads
    (sv,) = meta.saves
    assert isinstance(sv, Save) and (sv.session, sv.dst_start, sv.n) == ("s", 0, 100)
    assert list(sv.block_ids) == list(range(7))
    # a decode step: one token, a new block appears
    meta = sched.build_connector_meta(F.step_output(cached=[("r1", [7], 100, 1)]))
    assert [(s.dst_start, s.n) for s in meta.saves] == [(100, 1)]
    assert list(meta.saves[0].block_ids) == list(range(8))
    assert sched.request_finished(r1, list(range(8))) == (False, None)

    # the edit turn: positions [32, 96) reuse the store's [24, 88) moved by +8
    r2 = F.Request("r2", {"session": "s", "load": {"dst_start": 32, "dst_end": 96, "delta": 8},
                          "save": "full"}, 120)
    sched.on_new_request(r2)
    # a second request on the session while r2 is in flight runs with no reuse
    r3 = F.Request("r3", {"session": "s", "load": {"dst_start": 32, "dst_end": 96, "delta": 8},
                          "save": True}, 120)
    sched.on_new_request(r3)
    assert sched.get_num_new_matched_tokens(r3, 32) == (0, False)
    assert sched.get_num_new_matched_tokens(r2, 32) == (64, False)
    sched.update_state_after_alloc(r2, None, 64)
    blocks = [10 + i for i in range(8)]
    meta = sched.build_connector_meta(F.step_output(new=[("r2", blocks, 96, 24)],
                                                    finished={"r3"}))
    (ld,) = meta.loads
    assert isinstance(ld, Load)
    assert (ld.session, ld.dst_start, ld.n, ld.delta, ld.src_start) == ("s", 32, 64, 8, 24)
    assert list(ld.block_ids) == blocks
    (sv,) = meta.saves
    assert (sv.dst_start, sv.n) == (0, 120)  # "full": the whole prompt, once
    meta = sched.build_connector_meta(F.step_output(cached=[("r2", None, 120, 1)]))
    assert not meta.loads and [(s.dst_start, s.n) for s in meta.saves] == [(120, 1)]
    # a load the store cannot serve declines (recompute), with the reference's reason
    r4 = F.Request("r4", {"session": "t", "load": {"dst_start": 0, "dst_end": 64, "delta": 0}},
                   100)
    sched.on_new_request(r4)
    assert sched.get_num_new_matched_tokens(r4, 0) == (0, False)
    assert sched._sched.declines[-1] == "store no longer holds [0,64)"


def test_worker_hooks_without_work_do_nothing():
    _, worker = _pair()
    worker.start_load_kv(F.forward_context({}))  # no metadata bound
    worker.bind_connector_metadata(vc.ShiftConnectorMetadata())
    assert worker._get_connector_metadata() is not None
    worker.start_load_kv(F.forward_context({}))  # no loads
    worker.save_kv_layer("l0", torch.zeros(4, 8, 16, 256), None)  # no saves
    assert worker.wait_for_save() is None
    assert worker.get_finished(set()) == (None, None)
    worker.clear_connector_metadata()
    assert worker._get_connector_metadata() is None


def test_stats_merge_every_store():
    before = vc.stats()
    sched, worker = _pair({"store_tokens": 8192})
    for st in (sched.store, worker.store):
        assert st.reserve("a", 0, 300)
        assert st.covers("a", 0, 300)
    assert sched.store.reserve("b", 0, 100)
    merged = vc.merged_stats([sched.store, worker.store])
    assert merged["hits"] == 2 and merged["sessions"] == {"a": 300, "b": 100}
    assert merged["budget_tokens"] == 8192 and merged["used_tokens"] == (19 + 7) * 16  # blocks
    after = vc.stats()  # the module-wide view includes these two stores
    assert after["hits"] - before["hits"] >= 2
    del sched, worker


def test_fp8_k_scales_are_read_when_vllm_registered_the_caches(monkeypatch):
    """vLLM's worker calls ``register_kv_caches`` itself with tensors only; the layers' K
    scales still come from the first loading forward pass (``_k_scale_float``), so the two
    registration routes requantise fp8 K with the same scales."""
    for registered in (True, False):
        _, worker = _pair()
        caches = {f"l{i}": torch.zeros(4, 8, 16, 256, dtype=torch.float8_e4m3fn) for i in range(3)}
        scales = {"l0": 0.05, "l1": 0.0125, "l2": 0.1}
        if registered:
            worker.register_kv_caches(caches)
        seen = {}

        def fake_load(loads, _seen=seen, _w=worker):
            _seen.update(_w._loader.k_scales)
            return 0

        monkeypatch.setattr(worker._loader, "register_kv_caches", lambda kv: None)
        monkeypatch.setattr(worker._loader, "start_load_kv", fake_load)
        worker.bind_connector_metadata(vc.ShiftConnectorMetadata(
            loads=[Load.from_blocks("s", [0], 0, 16, 0)]))
        worker.start_load_kv(F.forward_context(caches, k_scales=scales))
        assert seen == scales, registered
        assert worker._loader.k_scales is worker._k_scales
