"""The shift connector as vLLM loads it: one object with vLLM's KV-connector hooks.

The reference's ``MarathonShiftConnector`` (src/marathon/vllm_shift_connector.py:159-556)
is one class instantiated twice by vLLM, once per role.  :class:`MarathonShiftConnector`
keeps its constructor, its hook signatures and the attributes it reads from vLLM's
objects, and hands the work to this package's halves:

* scheduler role -- :class:`~marathon_amd.connector.ShiftScheduler` over a tensor-free
  mirror of the worker's store (``on_new_request``, ``get_num_new_matched_tokens``,
  ``update_state_after_alloc``, ``build_connector_meta``, ``request_finished``);
* worker role -- :class:`~marathon_amd.connector.ShiftLoader` (``register_kv_caches``,
  ``start_load_kv``: every load of a step in one HIP launch) and
  :class:`~marathon_amd.connector.ShiftSaver` with deferred saves (``save_kv_layer``
  records the layer, ``wait_for_save`` saves every layer of the step in one launch).

Configuration is the reference's (``kv_connector_extra_config``: ``store_tokens``,
``store_device``, ``session_tokens``; ``MARATHON_STORE_TOKENS``), plus
``store_layout``: ``"block"`` (default, :class:`~marathon_amd.block_store.BlockShiftStore`)
or ``"flat"`` (the reference's layout, :class:`~marathon_amd.shift_store.ShiftStore`).
Both roles build the same kind of store from the same configuration, so the scheduler's
mirror reaches the worker's decisions.

:func:`stats` merges the counters of every store built in this process, scheduler
mirrors and worker stores alike (vllm_shift_connector.py:112-132).

vLLM is not installed here.  When it is importable, the class derives from vLLM's
``KVConnectorBase_V1`` and its metadata from ``KVConnectorMetadata``, so vLLM can load it
through ``KVTransferConfig(kv_connector="MarathonShiftConnector",
kv_connector_module_path="marathon_amd.vllm_connector")``.  Its behaviour inside vLLM is
not checked in this repository: the tests drive the hooks with stand-ins for vLLM's
``VllmConfig``, ``Request``, ``SchedulerOutput`` and ``ForwardContext`` that carry the
attributes the hooks read.
"""

from __future__ import annotations

import logging
import os
import time
import weakref
from dataclasses import dataclass, field
from typing import Any

import torch

from .connector import ShiftLoader, ShiftSaver, ShiftScheduler, StepMeta, store_from_config
from .shift_kernels import inv_freq_for
from .store_core import COUNTERS

try:  # the host framework, when present
    from vllm.distributed.kv_transfer.kv_connector.v1.base import (  # type: ignore
        KVConnectorBase_V1 as _ConnectorBase,
    )
    from vllm.distributed.kv_transfer.kv_connector.v1.base import (  # type: ignore
        KVConnectorMetadata as _MetadataBase,
    )

    HAVE_VLLM = True
except ImportError:
    _ConnectorBase = object
    _MetadataBase = object
    HAVE_VLLM = False

logger = logging.getLogger("vllm.marathon_shift")

#: ``MARATHON_SHIFT_TIMING=1``: synchronise around each step's loads and log the copy time
#: per step, in the reference's per-load units (vllm_shift_connector.py:519-534).
TIMING = os.environ.get("MARATHON_SHIFT_TIMING", "") not in ("", "0")

_STORES: "weakref.WeakSet" = weakref.WeakSet()


def stats() -> dict:
    """Counters merged over every store built by a connector in this process: counters
    summed, per-session positions and used tokens as the largest any store reports
    (scheduler mirrors and worker stores track the same sessions)."""
    return merged_stats(list(_STORES))


def merged_stats(stores) -> dict:
    out: dict[str, Any] = {name: 0 for name in COUNTERS}
    out.update(sessions={}, used_tokens=0, budget_tokens=0)
    for store in stores:
        s = store.stats()
        out["budget_tokens"] = max(out["budget_tokens"], s["budget_tokens"])
        out["used_tokens"] = max(out["used_tokens"], s["used_tokens"])
        for name, held in s["sessions"].items():
            out["sessions"][name] = max(out["sessions"].get(name, 0), held)
        for name in COUNTERS:
            out[name] += s[name]
    return out


@dataclass
class ShiftConnectorMetadata(StepMeta, _MetadataBase):
    """One step's loads and saves, handed from the scheduler role to the worker role
    (vllm_shift_connector.py:143-156)."""

    loads: list = field(default_factory=list)
    saves: list = field(default_factory=list)


def _is_worker(role) -> bool:
    name = getattr(role, "name", role)
    return str(name).lower() == "worker"


def _first_group(block_ids):
    """vLLM passes block ids per KV-cache group; the shift path uses the first group."""
    if block_ids is None:
        return None
    if len(block_ids) and isinstance(block_ids[0], (list, tuple)):
        return list(block_ids[0])
    return list(block_ids)


class MarathonShiftConnector(_ConnectorBase):
    """vLLM's KV connector for position-shifted KV reuse, on the HIP shift kernels."""

    def __init__(self, vllm_config, role, kv_cache_config=None):
        if HAVE_VLLM:
            super().__init__(vllm_config, role, kv_cache_config)
        self._role = role
        self._worker = _is_worker(role)
        self._bs = int(vllm_config.cache_config.block_size)
        ktc = getattr(vllm_config, "kv_transfer_config", None)
        extra = dict(getattr(ktc, "kv_connector_extra_config", None) or {})
        layout = str(extra.get("store_layout", "block"))
        if layout not in ("block", "flat"):
            raise ValueError(f"store_layout {layout!r}: 'block' or 'flat'")
        self._store = store_from_config(extra, self._worker, block_layout=layout == "block",
                                        block_size=self._bs)
        _STORES.add(self._store)
        hf = vllm_config.model_config.hf_text_config
        head_dim = getattr(hf, "head_dim", None) or hf.hidden_size // hf.num_attention_heads
        self._inv_freq = inv_freq_for(int(head_dim), float(getattr(hf, "rope_theta", 10000.0)),
                                      float(getattr(hf, "partial_rotary_factor", 1.0)))
        self._meta: ShiftConnectorMetadata | None = None
        self._timing = bool(extra.get("timing", TIMING))
        # scheduler side
        self._sched = ShiftScheduler(self._store, self._bs)
        # worker side
        self._k_scales: dict[str, float] = {}
        self._loader = ShiftLoader(self._store, self._bs, self._inv_freq,
                                   k_scales=self._k_scales)
        self._saver = ShiftSaver(self._store, self._bs, deferred=True)
        self._registered = False
        self._scales_read = False

    @property
    def store(self):
        return self._store

    # -------------------------------------------------------------- metadata plumbing
    # vLLM's base class provides these; they are restated so the hooks run without it.

    def bind_connector_metadata(self, meta) -> None:
        self._meta = meta
        if HAVE_VLLM:
            super().bind_connector_metadata(meta)

    def clear_connector_metadata(self) -> None:
        self._meta = None
        if HAVE_VLLM:
            super().clear_connector_metadata()

    def _get_connector_metadata(self):
        return self._meta

    # ---------------------------------------------------------------- scheduler side

    def on_new_request(self, request) -> None:
        """Record the request's ``kv_transfer_params``; take the session's writer slot
        (vllm_shift_connector.py:211-223)."""
        self._sched.on_new_request(request.request_id, request.kv_transfer_params or {})

    def get_num_new_matched_tokens(self, request, num_computed_tokens: int):
        """Tokens the store provides beyond vLLM's own prefix hit, and whether they load
        asynchronously (never) (vllm_shift_connector.py:247-288)."""
        return self._sched.get_num_new_matched_tokens(request.request_id,
                                                      int(num_computed_tokens),
                                                      int(request.num_prompt_tokens))

    def update_state_after_alloc(self, request, blocks, num_external_tokens: int) -> None:
        self._sched.update_state_after_alloc(request.request_id, int(num_external_tokens))

    def build_connector_meta(self, scheduler_output) -> ShiftConnectorMetadata:
        """This step's loads (a request's first step) and saves (every step)
        (vllm_shift_connector.py:332-372)."""
        sched = scheduler_output.num_scheduled_tokens
        new = [(req.req_id, _first_group(req.block_ids), int(req.num_computed_tokens),
                int(sched[req.req_id])) for req in scheduler_output.scheduled_new_reqs]
        cached_out = scheduler_output.scheduled_cached_reqs
        cached = [(rid, _first_group(cached_out.new_block_ids[i]),
                   int(cached_out.num_computed_tokens[i]), int(sched[rid]))
                  for i, rid in enumerate(cached_out.req_ids)]
        step = self._sched.build_connector_meta(new_reqs=new, cached_reqs=cached,
                                                finished=list(scheduler_output.finished_req_ids))
        return ShiftConnectorMetadata(loads=step.loads, saves=step.saves)

    def request_finished(self, request, block_ids):
        """Forget the request, free its session's writer slot, log the store; the blocks
        are never held for a transfer (vllm_shift_connector.py:385-389)."""
        self._sched.request_finished(request.request_id)
        return False, None

    # ------------------------------------------------------------------- worker side

    def register_kv_caches(self, kv_caches: dict) -> None:
        """The per-layer paged caches, fused 4-D ``[blocks, heads, bs, 2D]`` /
        ``[blocks, bs, heads, 2D]`` or split into K and V planes
        (vllm_shift_connector.py:393-412)."""
        self._loader.register_kv_caches(kv_caches)
        self._registered = True
        logger.info("marathon shift connector: %d layers, layout %s, store %d tok",
                    len(kv_caches), self._loader.layout, self._store.budget)

    def _register_from(self, forward_context) -> None:
        """The caches of the attention layers of a forward pass, as the reference takes
        them when none were registered (:484-493)."""
        ve = getattr(forward_context, "virtual_engine", 0)
        caches = {}
        for name, layer in forward_context.no_compile_layers.items():
            kv = getattr(layer, "kv_cache", None)
            if kv is None:
                continue
            caches[name] = kv[ve] if isinstance(kv, list) else kv
        if caches:
            self.register_kv_caches(caches)

    def _scales_from(self, forward_context) -> None:
        """The fp8 K scales of the attention layers (``_k_scale_float``, else
        ``_k_scale``), read once from the first forward pass that loads, whichever way
        the caches were registered: vLLM's own ``register_kv_caches`` call passes only
        the tensors.  A layer with no scale keeps 1.0."""
        for name, layer in forward_context.no_compile_layers.items():
            scale = getattr(layer, "_k_scale_float", None)
            if scale is None and getattr(layer, "_k_scale", None) is not None:
                scale = float(layer._k_scale)
            if scale is not None:
                self._k_scales[name] = float(scale)
        self._scales_read = True

    def start_load_kv(self, forward_context, **kwargs) -> None:
        """Every load of the step in one launch, before the forward pass
        (vllm_shift_connector.py:481-534)."""
        meta = self._get_connector_metadata()
        if meta is None or not meta.loads:
            return
        if not self._registered:
            self._register_from(forward_context)
        if not self._scales_read:
            self._scales_from(forward_context)
        t0 = 0.0
        if self._timing:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
        token_layers = self._loader.start_load_kv(meta.loads)
        if self._timing and token_layers:
            torch.cuda.synchronize()
            ms = (time.perf_counter() - t0) * 1e3
            plan = self._loader.last_plan
            src_bytes = plan.algorithmic_bytes // 2  # the source rows, as the reference counts
            for ld in meta.loads:
                logger.info("shift: session %s loaded %d tokens x %d layers from store[%d:%d], "
                            "delta=%d", ld.session, ld.n, len(self._loader.layer_names), ld.src_start,
                            ld.src_start + ld.n, ld.delta)
            logger.info("shift: step of %d loads, copy_ms=%.2f (%.2f MB, %.1f GB/s)",
                        len(meta.loads), ms, src_bytes / 2**20,
                        src_bytes / 2**30 / max(ms / 1e3, 1e-9))
            logger.info("shift: store %s", self._store.stats())

    def wait_for_layer_load(self, layer_name: str) -> None:
        return

    def save_kv_layer(self, layer_name: str, kv_layer: torch.Tensor, attn_metadata,
                      **kwargs) -> None:
        """Record the layer; the step's saves run in ``wait_for_save``
        (vllm_shift_connector.py:539-553)."""
        meta = self._get_connector_metadata()
        if meta is None or not meta.saves:
            return
        self._saver.save_kv_layer(layer_name, kv_layer, meta.saves)

    def wait_for_save(self) -> None:
        """Save every layer recorded this step in one launch."""
        self._saver.wait_for_save()

    def get_finished(self, finished_req_ids):
        return None, None
