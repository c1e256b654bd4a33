"""Batched shifts: every span x every layer x every session in ONE HIP launch.

The reference issues one Triton launch per layer per load
(src/marathon/vllm_shift_connector.py:505-515) and the HF prototype one rotation per
layer per segment (src/marathon/kvshift.py:242-268).  Here a :class:`ShiftPlan` holds a
device-resident span table (``mkv_span_t``), per-(group, layer) base-address tables for
source and destination, and the slot/block-table arrays, and :meth:`ShiftPlan.launch`
enqueues the whole shift as one ``mkv_shift_spans`` call.

Caches are described by :class:`CacheSet`: ``caches[group][layer]`` tensors of one
layout -- ``flat`` ``[rows, heads, 2D]`` (a position-indexed store, the reference's
``ShiftStore`` buffer, shift_store.py:225-236), or paged ``hnd`` ``[blocks, heads, bs,
2D]`` / ``nhd`` ``[blocks, bs, heads, 2D]`` (vLLM's fused layouts,
vllm_shift_connector.py:396-402).  A group is whatever owns a buffer: a session's store,
or the one shared paged cache.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .shift_kernels import current_stream, dtype_code

MODES = {"flat": _lib.MKV_ADDR_FLAT, "slots": _lib.MKV_ADDR_SLOTS, "table": _lib.MKV_ADDR_TABLE}


@dataclass
class CacheSet:
    """``caches[group][layer]`` of one layout; every tensor has the same trailing shape,
    strides and dtype (groups may differ in their number of blocks / rows).

    Rows are fused, ``[..., 2D]`` with K then V, unless ``v_caches`` is given: then
    ``caches`` hold K and ``v_caches`` V, as separate tensors of the same shape and
    strides with rows ``[..., D]`` (split K and V planes, e.g. ``kv[0]`` and ``kv[1]``
    of a ``[2, blocks, bs, heads, D]`` cache)."""

    caches: list
    layout: str  # "flat" | "hnd" | "nhd"
    block_size: int = 1
    v_caches: list | None = None

    def __post_init__(self):
        if self.layout not in ("flat", "hnd", "nhd"):
            raise ValueError(f"layout {self.layout!r}")
        # a flat list of per-layer tensors is one group; wrap it before any truth test,
        # since a tensor has no truth value
        if len(self.caches) and isinstance(self.caches[0], torch.Tensor):
            self.caches = [list(self.caches)]
        if self.v_caches is not None and len(self.v_caches) and isinstance(
                self.v_caches[0], torch.Tensor):
            self.v_caches = [list(self.v_caches)]
        if len(self.caches) == 0 or len(self.caches[0]) == 0:
            raise ValueError("empty CacheSet")
        if self.v_caches is not None:
            if len(self.v_caches) != len(self.caches) or any(
                    len(kr) != len(vr) for kr, vr in zip(self.caches, self.v_caches)):
                raise ValueError("v_caches must match caches group by group, layer by layer")
            for kr, vr in zip(self.caches, self.v_caches):
                for k, v in zip(kr, vr):
                    if (k.shape != v.shape or k.stride() != v.stride() or k.dtype != v.dtype
                            or k.device != v.device):
                        raise ValueError("a V tensor differs from its K tensor in shape, "
                                         "strides, dtype or device")
        first = self.caches[0][0]
        want_dim = 3 if self.layout == "flat" else 4
        for row in self.caches:
            if len(row) != len(self.caches[0]):
                raise ValueError("every group needs the same number of layers")
            for t in row:
                if t.dim() != want_dim:
                    raise ValueError(f"{self.layout} cache must be {want_dim}-D, got {tuple(t.shape)}")
                if t.dtype != first.dtype or t.device != first.device:
                    raise ValueError("caches differ in dtype or device")
                if t.shape[1:] != first.shape[1:] or t.stride() != first.stride():
                    raise ValueError("caches differ in trailing shape or strides")
                if t.stride(-1) != 1:
                    raise ValueError("rows must be contiguous in the last dimension")
        if self.layout == "flat":
            self.block_size = 1
        elif self.layout == "hnd" and first.shape[2] != self.block_size:
            raise ValueError(f"HND cache block dim {first.shape[2]} != block_size {self.block_size}")
        elif self.layout == "nhd" and first.shape[1] != self.block_size:
            raise ValueError(f"NHD cache block dim {first.shape[1]} != block_size {self.block_size}")

    @property
    def groups(self) -> int:
        return len(self.caches)

    @property
    def layers(self) -> int:
        return len(self.caches[0])

    @property
    def first(self) -> torch.Tensor:
        return self.caches[0][0]

    @property
    def heads(self) -> int:
        return self.first.shape[1] if self.layout in ("flat", "hnd") else self.first.shape[2]

    @property
    def split(self) -> bool:
        return self.v_caches is not None

    @property
    def head_size(self) -> int:
        return self.first.shape[-1] if self.split else self.first.shape[-1] // 2

    @property
    def strides(self) -> tuple[int, int, int]:
        s = self.first.stride()
        if self.layout == "flat":
            return s[0], s[1], 0
        return (s[0], s[1], s[2]) if self.layout == "hnd" else (s[0], s[2], s[1])

    def slots_of(self, t: torch.Tensor) -> int:
        return t.shape[0] * (1 if self.layout == "flat" else self.block_size)

    def base_tables(self):
        """``(k, v, caps, min_cap, uniform)``: per-(group, layer) K and V base addresses
        (uint64), per-group slot capacities, their minimum and whether they are all
        equal; computed once per CacheSet."""
        got = getattr(self, "_bases", None)
        if got is None:
            eb = self.first.element_size()
            k = np.array([[t.data_ptr() for t in row] for row in self.caches], dtype=np.uint64)
            if self.split:
                v = np.array([[t.data_ptr() for t in row] for row in self.v_caches],
                             dtype=np.uint64)
            else:
                v = k + np.uint64(self.head_size * eb)
            caps = np.array([self.slots_of(row[0]) for row in self.caches], dtype=np.int64)
            got = self._bases = (k, v, caps, int(caps.min()), bool(np.all(caps == caps[0])))
        return got


class _Staging:
    """Host arrays bound for the device, packed into one pinned buffer and copied with
    one asynchronous H2D: the host never waits for the stream to drain."""

    ALIGN = 256

    def __init__(self) -> None:
        self.parts: list = []
        self.size = 0

    def add(self, a: np.ndarray) -> int:
        a = np.ascontiguousarray(a)
        off = self.size
        self.parts.append((off, a))
        self.size = off + (a.nbytes + self.ALIGN - 1) // self.ALIGN * self.ALIGN
        return off

    def upload(self, device) -> torch.Tensor:
        host = torch.empty(max(self.size, self.ALIGN), dtype=torch.uint8, pin_memory=True)
        view = host.numpy()
        for off, a in self.parts:
            view[off:off + a.nbytes] = a.reshape(-1).view(np.uint8)
        # the caching host allocator keeps ``host`` until this copy has completed
        return host.to(device, non_blocking=True)


class ShiftPlan:
    """A batched shift, resident on the device and launchable any number of times.

    ``spans``: a ``SPAN_DTYPE`` structured array (or anything ``np.asarray`` turns into
    one).  ``src_index`` / ``dst_index``: int64 slots (mode ``slots``), int32 block ids
    (mode ``table``) or ``None`` (mode ``flat``), on the host or the device.
    ``inv_freq``: fp32 [rotary / 2].  ``k_scale``: fp32 [layers] for fp8 caches.

    Everything host-side (span table, per-(group, layer) base addresses, host index
    arrays, tables) goes to the device in one pinned, stream-ordered copy, so building
    a plan never blocks on the GPU.
    """

    def __init__(
        self,
        spans,
        src: CacheSet,
        dst: CacheSet,
        *,
        inv_freq: torch.Tensor | None,
        src_mode: str = "flat",
        src_index: torch.Tensor | None = None,
        dst_mode: str = "slots",
        dst_index: torch.Tensor | None = None,
        k_scale: torch.Tensor | None = None,
    ):
        spans = np.ascontiguousarray(np.asarray(spans, dtype=_lib.SPAN_DTYPE))
        if src.layers != dst.layers:
            raise ValueError(f"src has {src.layers} layers, dst {dst.layers}")
        if src.first.dtype != dst.first.dtype:
            raise TypeError("src and dst dtypes differ")
        if (src.heads, src.head_size) != (dst.heads, dst.head_size):
            raise ValueError("src and dst geometry differ")
        self.device = dst.first.device
        if src.first.device != self.device:
            raise ValueError("src and dst on different devices")
        self.src, self.dst = src, dst
        self.n_spans = int(spans.shape[0])
        # per-span token counts as Python ints (numpy reductions cost more on the few
        # spans of a step than the sums themselves)
        counts = [max(int(c), 0) for c in spans["n_tokens"].tolist()]
        self.tokens = sum(counts)
        self.dtype = dtype_code(dst.first.dtype)
        self._keep: list = []
        stage = _Staging()

        def place(t: torch.Tensor | None, dtype: torch.dtype, np_dtype):
            """A device tensor is used in place; a host one is staged.  Returns
            ``(device tensor or None, staging offset or None, count)``."""
            if t is None:
                return None, None, 0
            t = t.detach().reshape(-1)
            if t.is_cuda:
                t = t.to(device=self.device, dtype=dtype).contiguous()
                self._keep.append(t)
                return t, None, t.numel()
            a = t.numpy() if t.dtype == dtype else t.to(dtype).numpy()
            return None, stage.add(a.astype(np_dtype, copy=False)), a.size

        self.rotary = 0 if inv_freq is None else 2 * int(inv_freq.numel())
        inv = place(inv_freq, torch.float32, np.float32)
        scale = (None, None, 0)
        if self.dtype == _lib.MKV_FP8_E4M3 and self.rotary:
            if k_scale is None:
                raise ValueError("fp8 caches need k_scale [layers]")
            scale = place(k_scale, torch.float32, np.float32)
            if scale[2] < dst.layers:
                raise ValueError("k_scale needs one entry per layer")

        src_plan = self._side(src, src_mode, src_index, stage, place)
        dst_plan = self._side(dst, dst_mode, dst_index, stage, place)
        span_off = stage.add(spans.view(np.uint8).reshape(-1)) if self.n_spans else None
        # the tables are copied on the device's current stream; a launch on another
        # stream first waits for this event (see _launch)
        if self.device.index == torch.cuda.current_device():
            blob = stage.upload(self.device)
            self._ready = torch.cuda.Event()
            self._ready.record()
        else:
            with torch.cuda.device(self.device):
                blob = stage.upload(self.device)
                self._ready = torch.cuda.Event()
                self._ready.record()
        self._keep.append(blob)
        self._synced = {current_stream(self.device)}
        base = blob.data_ptr()

        def ptr(item) -> int | None:
            t, off, _ = item
            if t is not None:
                return t.data_ptr()
            return None if off is None else base + off

        src_side = self._finish_side(src_plan, ptr)
        dst_side = self._finish_side(dst_plan, ptr)

        self.descs = []
        step = _lib.MKV_MAX_SPANS
        chunks = [(lo, min(step, self.n_spans - lo)) for lo in range(0, self.n_spans, step)]
        L = _lib.lib()
        need = max(
            (L.mkv_shift_workspace_size(sum(counts[lo:lo + cnt]), cnt, self.rotary)
             for lo, cnt in chunks),
            default=0,
        )
        # one workspace serves every chunk: the chunks run in stream order
        self.workspace = torch.empty(max(int(need), 16), dtype=torch.uint8, device=self.device)
        for lo, cnt in chunks:
            d = _lib.ShiftDesc()
            d.spans = base + span_off + lo * _lib.SPAN_DTYPE.itemsize
            d.workspace = self.workspace.data_ptr()
            d.workspace_bytes = self.workspace.numel()
            d.total_tokens = sum(counts[lo:lo + cnt])
            d.inv_freq = ptr(inv)
            d.k_scale = ptr(scale)
            d.error_flags = None
            d.n_spans = cnt
            d.layers = dst.layers
            d.heads = dst.heads
            d.head_size = dst.head_size
            d.rotary = self.rotary
            d.dtype = self.dtype
            d.src = src_side
            d.dst = dst_side
            self.descs.append(d)

    @staticmethod
    def _side(cs: CacheSet, mode: str, index, stage: _Staging, place) -> dict:
        if mode not in MODES:
            raise ValueError(f"mode {mode!r}")
        k, v, caps, min_cap, uniform = cs.base_tables()
        out = {
            "cs": cs,
            "mode": mode,
            "k": (None, stage.add(k.reshape(-1)), k.size),
            "v": (None, stage.add(v.reshape(-1)), v.size),
            "num_slots": min_cap,
            "group_slots": None if uniform else (None, stage.add(caps), caps.size),
            "index": (None, None, 0),
        }
        if mode != "flat":
            if index is None:
                raise ValueError(f"mode {mode!r} needs an index array")
            if mode == "slots":
                out["index"] = place(index, torch.int64, np.int64)
            else:
                out["index"] = place(index, torch.int32, np.int32)
        return out

    @staticmethod
    def _finish_side(plan: dict, ptr) -> _lib.Side:
        cs = plan["cs"]
        side = _lib.Side()
        side.k_base = ptr(plan["k"])
        side.v_base = ptr(plan["v"])
        side.num_slots = plan["num_slots"]
        side.group_slots = None if plan["group_slots"] is None else ptr(plan["group_slots"])
        n_index = plan["index"][2]
        side.index = ptr(plan["index"]) if n_index else None
        side.index_len = n_index
        bs, hstr, ostr = cs.strides
        side.block_stride, side.head_stride, side.offset_stride = bs, hstr, ostr
        side.block_size = cs.block_size
        side.mode = MODES[plan["mode"]]
        side.groups = cs.groups
        return side

    @property
    def algorithmic_bytes(self) -> int:
        """K and V read once and written once: 2 * tokens * layers * heads * 2D * elem."""
        eb = self.dst.first.element_size()
        return 2 * self.tokens * self.dst.layers * self.dst.heads * 2 * self.dst.head_size * eb

    def launch(self, stream: int | None = None, error_flags: torch.Tensor | None = None) -> None:
        """Enqueue the shift on ``stream`` (default: current): a plan launch and a shift
        launch per 4096 spans.

        Nothing is allocated, copied or cleared here, so a launch can be captured into a
        HIP graph and replayed.  The plan must be built before the capture begins and the
        capture must start after its tables have arrived (``torch.cuda.graph`` begins
        with a device synchronisation)."""
        if stream is None:
            stream = current_stream(self.device)
        if self.device.index == torch.cuda.current_device():
            self._launch(int(stream), error_flags)
        else:
            with torch.cuda.device(self.device):  # launches go to the current device
                self._launch(int(stream), error_flags)

    def _launch(self, stream: int, error_flags: torch.Tensor | None) -> None:
        L = _lib.lib()
        if stream not in self._synced:
            # the tables were copied on the stream current at build time
            ext = torch.cuda.ExternalStream(stream, device=self.device)
            if not torch.cuda.is_current_stream_capturing():
                ext.wait_event(self._ready)
            for t in (*self._keep, self.workspace):
                t.record_stream(ext)
            self._synced.add(stream)
        flags = error_flags.data_ptr() if error_flags is not None else None
        for d in self.descs:
            d.error_flags = flags
            _lib.check(L.mkv_shift_spans(ctypes.byref(d), ctypes.c_void_p(stream)))


def span_array(rows) -> np.ndarray:
    """Build a ``SPAN_DTYPE`` array from dicts or tuples in field order."""
    out = np.zeros(len(rows), dtype=_lib.SPAN_DTYPE)
    for i, r in enumerate(rows):
        if isinstance(r, dict):
            for k, val in r.items():
                out[i][k] = val
        else:
            out[i] = tuple(r)
    return out
