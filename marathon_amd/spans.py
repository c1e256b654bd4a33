"""Batched shifts: every span x every layer x every session in ONE HIP launch.

The reference issues one Triton launch per layer per load
(src/marathon/vllm_shift_connector.py:505-515) and the HF prototype one rotation per
layer per segment (src/marathon/kvshift.py:242-268).  Here a :class:`ShiftPlan` holds a
device-resident span table (``mkv_span_t``), per-(group, layer) base-address tables for
source and destination, and the slot/block-table arrays, and :meth:`ShiftPlan.launch`
enqueues the whole shift as one ``mkv_shift_spans`` call: a plan launch plus the shift
(optionally with the tokens sorted by destination page), or, for short shifts, the shift
alone (the direct path).  :class:`SmallShifts` runs the steady state of a serving loop --
a decode step's saves, short loads -- with no plan to build.

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

#: Shifts of at most this many (token, layer) rows take the library's direct path when
#: eligible: one launch instead of the plan pass plus the shift.  Measured on MI355X
#: (bf16, 8 heads, 40 layers, one span, flat store -> HND cache through shuffled slots;
#: bench.py's plan_variants): 16, 64, 256 and 512 tokens run in 6.6, 8.8, 21.8 and
#: 34.3 us direct against 10.2, 11.9, 22.5 and 36.8 us; from 1,024 tokens the two-launch
#: path is faster (61.6 against 63.5 us): a direct workgroup resolves its token (span,
#: then slot) before it can load its data, where a record from the plan pass carries the
#: token's rows.  Above 2,560 rows the direct kernel moves four layers per workgroup.
DIRECT_MAX_TOKEN_LAYERS = 20480
#: SmallShifts puts a step's spans and index windows in the launch's own arguments up to
#: this many (token, layer) rows: that saves the host its staging copy, but every
#: workgroup then reads the arguments, which costs more than the copy from about 64
#: tokens x 40 layers on (12.6 against 9.6 us of GPU time; 34 against 22 at 256).
SMALL_ARGS_MAX_TOKEN_LAYERS = 2560


#: Token orders of the two-launch path.  ``"dst_page"``: tokens sorted by the page of their
#: destination row -- computed here and handed over as ``mkv_shift_desc_t.token_order``
#: (no extra launch) when the destination index is on the host, else sorted on the device
#: (``mkv_shift_desc_t.order``, one more launch); ``"dst_page_device"``: always the latter.
ORDERS = {"none": _lib.MKV_ORDER_NONE, "dst_page": _lib.MKV_ORDER_DST_PAGE,
          "dst_page_device": _lib.MKV_ORDER_DST_PAGE, "dst_addr": _lib.MKV_ORDER_NONE}
#: Buckets of the destination-page order (the device's kOrderBuckets).
ORDER_BUCKETS = 256


class _on:
    """``torch.cuda.device(device)`` only when ``device`` is not already current."""

    def __init__(self, device, current: bool):
        self.ctx = None if current else torch.cuda.device(device)

    def __enter__(self):
        if self.ctx is not None:
            self.ctx.__enter__()

    def __exit__(self, *exc):
        if self.ctx is not None:
            return self.ctx.__exit__(*exc)
        return False


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
        first = self.caches[0][0]
        want_dim = 3 if self.layout == "flat" else 4
        # The kernels address every tensor of the set with one set of strides.  A dim
        # of one element never advances an address, and torch gives such dims any
        # stride (a one-row slice is "contiguous" with its parent's strides), so
        # tensors must agree only where a dim has more than one element, and each
        # stride of the set comes from a tensor where its dim does.
        strides = list(first.stride())
        known = [n > 1 for n in first.shape]

        def agree(t) -> bool:
            for d, (n, s) in enumerate(zip(t.shape, t.stride())):
                if n > 1:
                    if known[d] and s != strides[d]:
                        return False
                    strides[d], known[d] = s, True
            return True

        if self.v_caches is not None:
            if len(self.v_caches) != len(self.caches) or any(
                    len(kr) != len(vr) for kr, vr in zip(self.caches, self.v_caches)):
                raise ValueError("v_caches must match caches group by group, layer by layer")
            for kr, vr in zip(self.caches, self.v_caches):
                for k, v in zip(kr, vr):
                    if (k.shape != v.shape or k.dtype != v.dtype or k.device != v.device
                            or not agree(k) or not agree(v)):
                        raise ValueError("a V tensor differs from its K tensor in shape, "
                                         "strides, dtype or device")
        for row in self.caches:
            if len(row) != len(self.caches[0]):
                raise ValueError("every group needs the same number of layers")
            # the device bounds-checks a group's slots against one capacity (its first
            # layer's), so every layer of a group must hold as many blocks / rows
            if any(t.dim() > 0 and t.shape[0] != row[0].shape[0] for t in row):
                raise ValueError("the layers of a group differ in their number of blocks / "
                                 f"rows: {sorted({int(t.shape[0]) for t in row})}")
            for t in row:
                if t.dim() != want_dim:
                    raise ValueError(f"{self.layout} cache must be {want_dim}-D, got {tuple(t.shape)}")
                if t.dtype != first.dtype or t.device != first.device:
                    raise ValueError("caches differ in dtype or device")
                if t.shape[1:] != first.shape[1:] or not agree(t):
                    raise ValueError("caches differ in trailing shape or strides")
                if t.stride(-1) != 1:
                    raise ValueError("rows must be contiguous in the last dimension")
        self._strides = tuple(strides)
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

    def fused(self, group: int, layer: int, index=None) -> torch.Tensor:
        """Rows of the (group, layer) cache with K and V side by side, ``[..., 2D]``:
        ``cache[index]`` (the whole cache when ``index`` is None), and with split planes
        a copy that puts the V plane's rows after the K plane's."""
        k = self.caches[group][layer]
        if index is not None:
            k = k[index]
        if not self.split:
            return k
        v = self.v_caches[group][layer]
        return torch.cat((k, v if index is None else v[index]), dim=-1)

    @property
    def strides(self) -> tuple[int, int, int]:
        """Element strides ``(block or row, head, offset in block)`` of every tensor."""
        s = self._strides
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

    def device_tables(self, device) -> tuple:
        """``(k_ptr, v_ptr, caps_ptr or None, ready)``: the base-address tables (and the
        per-group capacities, when they differ) on ``device``, uploaded once per CacheSet
        with one stream-ordered copy on the current stream; ``ready`` is an event after
        that copy, for launches on other streams.  The upload is kept alive by the set."""
        got = getattr(self, "_dev", None)
        if got is None:
            k, v, caps, _, uniform = self.base_tables()
            stage = _Staging()
            offs = (stage.add(k.reshape(-1)), stage.add(v.reshape(-1)),
                    None if uniform else stage.add(caps))
            blob = stage.upload(device)
            ready = torch.cuda.Event()
            ready.record()
            base = blob.data_ptr()
            got = self._dev = (base + offs[0], base + offs[1],
                               None if offs[2] is None else base + offs[2], ready, blob)
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

    Everything host-side (span table, host index arrays, inv_freq, scales, the direct
    path's prefix and tables) goes to the device in one pinned, stream-ordered copy, so
    building a plan never blocks on the GPU; the caches' base-address tables are
    uploaded once per :class:`CacheSet`.

    ``direct``: None (default) takes the library's single-launch path up to
    :data:`DIRECT_MAX_TOKEN_LAYERS` rows whenever :meth:`direct_eligible` allows it,
    with the token prefix and the per-span rotation tables computed here
    (:func:`span_tables`); False always runs the two-launch path (plan pass and
    workspace), True asks for the direct path where eligible.

    ``order``: the order the two-launch path moves tokens in -- ``"none"`` (span order),
    ``"dst_page"`` (sorted by the page of each token's destination row: here, when the
    destination index is on the host, and handed to the plan pass as ``token_order``;
    otherwise on the device, one more small launch) or ``"dst_page_device"`` (always on
    the device).  None (default): the host-sorted page order when the destination index
    is on the host, span order otherwise.  On the Qwen3-14B multi-span shift the host
    order moves bf16 1.1% and fp8 2.8% faster and costs about 0.2 ms of host time per
    22,141 tokens when the plan is built; a caller that builds a plan for a single launch
    with the host on its critical path (the connector's per-step loads) passes
    ``"none"``.
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
        direct: bool | None = None,
        order: str | None = None,
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
            """A device tensor is used in place; a host tensor or numpy array is staged.  Returns
            ``(device tensor or None, staging offset or None, count)``."""
            if t is None:
                return None, None, 0
            if isinstance(t, np.ndarray):  # host index windows built with numpy
                a = t.reshape(-1)
                return None, stage.add(a.astype(np_dtype, copy=False)), a.size
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

        for mode in (src_mode, dst_mode):
            if mode not in MODES:
                raise ValueError(f"mode {mode!r}")
        dst_index_arg = dst_index
        src_index = self._index(src_mode, src_index, place)
        dst_index = self._index(dst_mode, dst_index, place)
        span_off = stage.add(spans.view(np.uint8).reshape(-1)) if self.n_spans else None
        # the direct path (one launch, no workspace) for small shifts, where the plan
        # pass's launch dominates; the token prefix and per-span tables come from here
        if direct is None:
            direct = self.tokens * dst.layers <= DIRECT_MAX_TOKEN_LAYERS
        self.direct = bool(direct) and self.direct_eligible(src, dst, self.n_spans)
        starts_off = tables_off = None
        if self.direct:
            starts_off = stage.add(np.concatenate(([0], np.cumsum(counts))).astype(np.int64))
            tables_off = stage.add(span_tables(spans["delta"], inv_freq, self.rotary))
        step = _lib.MKV_MAX_SPANS
        chunks = [(lo, min(step, self.n_spans - lo)) for lo in range(0, self.n_spans, step)]
        index_on_host = dst_mode == "flat" or not (isinstance(dst_index_arg, torch.Tensor)
                                                   and dst_index_arg.is_cuda)
        if order is None:
            order = "dst_page" if index_on_host else "none"
        if order not in ORDERS:
            raise ValueError(f"order {order!r}: one of {sorted(ORDERS)}")
        self.order = "none" if self.direct else order
        # the destination-page order computed here when the destination index is on the
        # host: each chunk's tokens stably sorted by page (a radix sort on uint8 keys),
        # handed to the plan pass as token_order, so no sorting launch runs
        order_offs = None
        if self.order in ("dst_page", "dst_addr") and index_on_host:
            host_index = None
            if dst_mode != "flat":
                host_index = (dst_index_arg.numpy() if isinstance(dst_index_arg, torch.Tensor)
                              else np.asarray(dst_index_arg))
            if self.order == "dst_addr":  # the destination rows' addresses, ascending
                pages = dst_page_order(spans, dst, dst_mode, host_index, 65536, 0)
            else:
                pages = dst_page_order(spans, dst, dst_mode, host_index)
            order_offs, t0 = [], 0
            for lo, cnt in chunks:
                t1 = t0 + sum(counts[lo:lo + cnt])
                perm = np.argsort(pages[t0:t1], kind="stable").astype(np.int32)
                order_offs.append(stage.add(perm))
                t0 = t1
            self.order = "dst_page_host" if self.order == "dst_page" else "dst_addr_host"

        on_device = self.device.index == torch.cuda.current_device()
        with _on(self.device, on_device):
            # the caches' base-address tables: uploaded once per CacheSet
            self._tables_ready = []
            sides = []
            for cs in (src, dst):
                k_ptr, v_ptr, caps_ptr, ready, _ = cs.device_tables(self.device)
                self._tables_ready.append(ready)
                sides.append((k_ptr, v_ptr, caps_ptr))
            # this plan's own arrays: one stream-ordered copy on the current stream
            blob = stage.upload(self.device)
            self._build_stream = current_stream(self.device)
        self._keep.append(blob)
        self._synced = {self._build_stream}
        base = blob.data_ptr()

        def ptr(item) -> int | None:
            t, off, _ = item
            if t is not None:
                return t.data_ptr()
            return None if off is None else base + off

        src_side = self._make_side(src, src_mode, src_index, sides[0], ptr)
        dst_side = self._make_side(dst, dst_mode, dst_index, sides[1], ptr)

        self.descs = []
        self.workspace = None
        if not self.direct:
            L = _lib.lib()
            ordered = self.order in ("dst_page", "dst_page_device")  # device sort
            need = max(
                (L.mkv_shift_workspace_size(sum(counts[lo:lo + cnt]), cnt, self.rotary)
                 + (32 * sum(counts[lo:lo + cnt]) + (1 << 20) if ordered else 0)
                 for lo, cnt in chunks),
                default=0,
            )
            # one workspace serves every chunk: the chunks run in stream order
            self.workspace = torch.empty(max(int(need), 16), dtype=torch.uint8,
                                         device=self.device)
        for k, (lo, cnt) in enumerate(chunks):
            d = _lib.ShiftDesc()
            d.spans = base + span_off + lo * _lib.SPAN_DTYPE.itemsize
            if self.direct:  # a single chunk
                d.span_starts = base + starts_off
                d.span_tables = base + tables_off
            else:
                d.workspace = self.workspace.data_ptr()
                d.workspace_bytes = self.workspace.numel()
                if order_offs is not None:
                    d.token_order = base + order_offs[k]
                else:
                    d.order = ORDERS[self.order]
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
    def direct_eligible(src: CacheSet, dst: CacheSet, n_spans: int) -> bool:
        """Whether the library takes the direct path for this shift: at most
        ``MKV_DIRECT_MAX_SPANS`` spans, power-of-two block sizes on both sides, and a
        head count that is a multiple of the rows one wave covers (every row of a wave
        pass then belongs to one token)."""
        eb = dst.first.element_size()
        rows_per_wave = 64 // max(1, dst.head_size * eb // 16)
        pow2 = all(cs.block_size > 0 and cs.block_size & (cs.block_size - 1) == 0
                   for cs in (src, dst))
        return (0 < n_spans <= _lib.MKV_DIRECT_MAX_SPANS and pow2
                and dst.heads % rows_per_wave == 0)

    @staticmethod
    def _index(mode: str, index, place):
        if mode == "flat":
            return None, None, 0
        if index is None:
            raise ValueError(f"mode {mode!r} needs an index array")
        if mode == "slots":
            return place(index, torch.int64, np.int64)
        return place(index, torch.int32, np.int32)

    @staticmethod
    def _make_side(cs: CacheSet, mode: str, index, tables: tuple, ptr) -> _lib.Side:
        side = _lib.Side()
        side.k_base, side.v_base, side.group_slots = tables
        side.num_slots = cs.base_tables()[3]
        n_index = index[2]
        side.index = ptr(index) if n_index else None
        side.index_len = n_index
        bs, hstr, ostr = cs.strides
        side.block_stride, side.head_stride, side.offset_stride = bs, hstr, ostr
        side.block_size = cs.block_size
        side.mode = MODES[mode]
        side.groups = cs.groups
        return side

    @property
    def algorithmic_bytes(self) -> int:
        """K and V read once and written once: 2 * tokens * layers * heads * 2D * elem."""
        eb = self.dst.first.element_size()
        return 2 * self.tokens * self.dst.layers * self.dst.heads * 2 * self.dst.head_size * eb

    @property
    def metadata_bytes(self) -> dict:
        """What a launch moves besides K and V, each counted once: the span table and
        index arrays the kernels read, the per-span rotation tables, and (two-launch
        path) the 32-byte token records the plan pass writes and the shift reads."""
        idx = sum(d.src.index_len * (8 if d.src.mode == MODES["slots"] else 4)
                  + d.dst.index_len * (8 if d.dst.mode == MODES["slots"] else 4)
                  for d in self.descs[:1])
        return {"spans": self.n_spans * _lib.SPAN_DTYPE.itemsize, "index": int(idx),
                "tables": self.n_spans * 2 * self.rotary * 4,
                "records": 0 if self.direct else 32 * self.tokens}

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
            # the plan's arrays were copied on the stream current at build time, the
            # caches' base-address tables when each set was first used
            ext = torch.cuda.ExternalStream(stream, device=self.device)
            if not torch.cuda.is_current_stream_capturing():
                ext.wait_stream(torch.cuda.ExternalStream(self._build_stream,
                                                          device=self.device))
                for ready in self._tables_ready:
                    ext.wait_event(ready)
            for t in self._keep + ([] if self.workspace is None else [self.workspace]):
                t.record_stream(ext)
            self._synced.add(stream)
        flags = error_flags.data_ptr() if error_flags is not None else None
        for d in self.descs:
            d.error_flags = flags
            _lib.check(L.mkv_shift_spans(ctypes.byref(d), ctypes.c_void_p(stream)))


class SmallShifts:
    """Direct-path shifts of a few tokens, with no per-step allocation or descriptor
    building: the steady state of a serving loop (a decode step's saves, short loads).

    One device buffer per (source caches, destination caches, addressing modes) holds a
    step's span table, token prefix, rotation tables and index windows; :meth:`run`
    rewrites it with one pinned copy on the current stream and launches the step with a
    descriptor kept from the previous one.  Stream order keeps a step's copy after the
    previous step's kernel, which still reads the buffer.  Only steps that take the
    library's direct path come here (:meth:`fits`); the rest build a :class:`ShiftPlan`.
    """

    SPANS_AT = 0
    STARTS_AT = _lib.MKV_DIRECT_MAX_SPANS * _lib.SPAN_DTYPE.itemsize  # 3,024 B
    TABLES_AT = STARTS_AT + 64 * 8

    def __init__(self, src: CacheSet, dst: CacheSet, *, inv_freq: torch.Tensor | None,
                 src_mode: str, dst_mode: str, k_scale: torch.Tensor | None = None):
        self.src, self.dst = src, dst
        self.device = dst.first.device
        self.rotary = 0 if inv_freq is None else 2 * int(inv_freq.numel())
        self.inv_host = None if inv_freq is None else inv_freq.detach().to(
            "cpu", torch.float32).contiguous()
        self.dtype = dtype_code(dst.first.dtype)
        self.modes = (src_mode, dst_mode)
        self.eligible_geometry = ShiftPlan.direct_eligible(src, dst, 1)
        self._idx = {"flat": (None, 0), "slots": (np.int64, 8), "table": (np.int32, 4)}
        # the small entry point reads its host arrays during the call: one set of host
        # buffers, addresses taken once, serves every step
        self._h_spans = np.zeros(_lib.MKV_SMALL_MAX_SPANS, dtype=_lib.SPAN_DTYPE)
        self._h_index = [np.zeros(_lib.MKV_SMALL_MAX_INDEX, dtype=self._idx[m][0] or np.int64)
                         for m in (src_mode, dst_mode)]
        self._h_addr = (self._h_spans.ctypes.data, self._h_index[0].ctypes.data,
                        self._h_index[1].ctypes.data)
        self.capacity = 0
        self.buf = None
        self._keep = []
        with _on(self.device, self.device.index == torch.cuda.current_device()):
            static = _Staging()
            inv_off = None if inv_freq is None else static.add(self.inv_host.numpy())
            scale_off = None
            if self.dtype == _lib.MKV_FP8_E4M3 and self.rotary:
                if k_scale is None:
                    raise ValueError("fp8 caches need k_scale [layers]")
                scale = k_scale.detach().to("cpu", torch.float32).reshape(-1).numpy()
                if scale.size < dst.layers:
                    raise ValueError("k_scale needs one entry per layer")
                scale_off = static.add(scale)
            blob = static.upload(self.device)
            self._keep.append(blob)
            sides = [cs.device_tables(self.device)[:3] for cs in (src, dst)]
        base = blob.data_ptr()
        d = self.desc = _lib.ShiftDesc()
        d.inv_freq = None if inv_off is None else base + inv_off
        d.k_scale = None if scale_off is None else base + scale_off
        d.layers, d.heads, d.head_size = dst.layers, dst.heads, dst.head_size
        d.rotary, d.dtype = self.rotary, self.dtype
        d.src = ShiftPlan._make_side(src, src_mode, (None, None, 0), sides[0], None)
        d.dst = ShiftPlan._make_side(dst, dst_mode, (None, None, 0), sides[1], None)
        # the same shift for mkv_shift_spans_small: host span rows and index windows
        self.small_desc = _lib.ShiftDesc()
        ctypes.memmove(ctypes.byref(self.small_desc), ctypes.byref(d), ctypes.sizeof(d))
        self._last: tuple = ()
        self.tokens = 0

    def fits(self, n_spans: int, tokens: int) -> bool:
        return (self.eligible_geometry and 0 < n_spans <= _lib.MKV_DIRECT_MAX_SPANS
                and tokens * self.dst.layers <= DIRECT_MAX_TOKEN_LAYERS)

    def _ensure(self, nbytes: int) -> None:
        if nbytes > self.capacity:
            self.capacity = max(nbytes, 2 * self.capacity, self.TABLES_AT + 4096)
            self.buf = torch.empty(self.capacity, dtype=torch.uint8, device=self.device)
            base = self.buf.data_ptr()
            self.desc.spans = base + self.SPANS_AT
            self.desc.span_starts = base + self.STARTS_AT
            self.desc.span_tables = base + self.TABLES_AT

    def run(self, rows: list, src_index: np.ndarray | None, dst_index: np.ndarray | None,
            error_flags: torch.Tensor | None = None) -> None:
        """Shift ``rows`` (``mkv_span_t`` field tuples) on the current stream, their
        source and destination indices given as host arrays (None for ``flat``).

        Up to ``MKV_SMALL_MAX_SPANS`` spans and ``MKV_SMALL_MAX_INDEX`` index entries a
        side, the rows and windows travel in the launch itself
        (``mkv_shift_spans_small``); beyond that they are copied into this runner's
        device buffer first."""
        n = len(rows)
        n_src = 0 if src_index is None else src_index.size
        n_dst = 0 if dst_index is None else dst_index.size
        tokens = sum(max(int(r[4]), 0) for r in rows)
        if (n <= _lib.MKV_SMALL_MAX_SPANS and n_src <= _lib.MKV_SMALL_MAX_INDEX
                and n_dst <= _lib.MKV_SMALL_MAX_INDEX
                and tokens * self.dst.layers <= SMALL_ARGS_MAX_TOKEN_LAYERS):
            hs = self._h_spans
            for i, r in enumerate(rows):
                hs[i] = r
            if n_src:
                self._h_index[0][:n_src] = src_index
            if n_dst:
                self._h_index[1][:n_dst] = dst_index
            d = self.small_desc
            d.spans = self._h_addr[0]
            d.n_spans = n
            d.total_tokens = self.tokens = tokens
            d.src.index = self._h_addr[1] if n_src else None
            d.src.index_len = n_src
            d.dst.index = self._h_addr[2] if n_dst else None
            d.dst.index_len = n_dst
            self._last = (True,)  # a relaunch reads the host buffers again
            self.launch(error_flags=error_flags)
            return
        self._last = ()
        spans = np.array(rows, dtype=_lib.SPAN_DTYPE)
        counts = np.maximum(spans["n_tokens"], 0).astype(np.int64)
        starts = np.zeros(n + 1, np.int64)
        np.cumsum(counts, out=starts[1:])
        src_t, src_b = self._idx[self.modes[0]]
        dst_t, dst_b = self._idx[self.modes[1]]
        # layout: span rows, prefix, the rotated spans' tables (when any), the indices
        tables = None
        if self.rotary and bool(spans["delta"].any()):
            tables = span_tables(spans["delta"], self.inv_host, self.rotary)
        src_at = self.TABLES_AT + (0 if tables is None else (tables.nbytes + 15) // 16 * 16)
        dst_at = src_at + (n_src * src_b + 15) // 16 * 16
        end = dst_at + n_dst * dst_b
        self._ensure(end)
        host = torch.empty(end, dtype=torch.uint8, pin_memory=True)
        hv = host.numpy()
        hv[self.SPANS_AT:self.SPANS_AT + spans.nbytes] = spans.view(np.uint8)
        hv[self.STARTS_AT:self.STARTS_AT + starts.nbytes] = starts.view(np.uint8)
        if tables is not None:
            hv[self.TABLES_AT:self.TABLES_AT + tables.nbytes] = tables.reshape(-1).view(np.uint8)
        if n_src:
            hv[src_at:src_at + n_src * src_b] = np.ascontiguousarray(
                src_index, dtype=src_t).view(np.uint8)
        if n_dst:
            hv[dst_at:dst_at + n_dst * dst_b] = np.ascontiguousarray(
                dst_index, dtype=dst_t).view(np.uint8)
        # one copy of the step's region (the gaps between parts are never read)
        self.buf[:end].copy_(host, non_blocking=True)
        d = self.desc
        base = self.buf.data_ptr()
        d.src.index = base + src_at if n_src else None
        d.src.index_len = n_src
        d.dst.index = base + dst_at if n_dst else None
        d.dst.index_len = n_dst
        d.n_spans = n
        d.total_tokens = self.tokens = int(starts[-1])
        self.launch(error_flags=error_flags)

    def launch(self, stream: int | None = None, error_flags: torch.Tensor | None = None) -> None:
        """(Re)launch the last step on ``stream`` (default: current); a step that went
        through the device buffer must run on the stream it was copied on."""
        small = bool(self._last)
        d = self.small_desc if small else self.desc
        d.error_flags = None if error_flags is None else error_flags.data_ptr()
        if stream is None:
            stream = current_stream(self.device)
        L = _lib.lib()
        fn = L.mkv_shift_spans_small if small else L.mkv_shift_spans
        _lib.check(fn(ctypes.byref(d), ctypes.c_void_p(int(stream))))

    @property
    def direct(self) -> bool:
        return True

    @property
    def algorithmic_bytes(self) -> int:
        eb = self.dst.first.element_size()
        return 2 * self.tokens * self.dst.layers * self.dst.heads * 2 * self.dst.head_size * eb


def span_tables(deltas, inv_freq: torch.Tensor | None, rotary: int) -> np.ndarray:
    """Per-span rotation tables, fp32 ``[n_spans, 2, rotary]``: the cos of each element's
    angle, then its signed sine (-sin on the first half, +sin on the second), where the
    angle of frequency f is ``fl32(fl32(delta) * inv_freq[f])`` and cos/sin are evaluated
    in double precision and rounded once to fp32 by the library's host routine
    (``mkv_rope_tables``), the one the plan pass runs on the device: the direct path's
    tables and the device's are the same bits (shift_kernels.py:68-84 for the layout)."""
    deltas = np.asarray(deltas, dtype=np.int64)
    if rotary == 0 or deltas.size == 0:
        return np.zeros((deltas.size, 2, rotary), np.float32)
    inv = inv_freq.detach().to(device="cpu", dtype=torch.float32).numpy().reshape(-1)
    return _lib.rope_tables(deltas, inv, rotary)


def dst_page_order(spans: np.ndarray, dst: CacheSet, mode: str, index,
                   buckets: int = ORDER_BUCKETS, min_shift: int = 21) -> np.ndarray:
    """Per token, in span order, the page bucket of its destination row, as the device's
    destination-page order computes it: the row's byte offset in its buffer shifted right
    by the smallest shift of at least ``min_shift`` (21: 2 MB pages) that maps the
    destination's extent into ``buckets`` buckets, offsets past the last bucket sharing
    it.  ``index``: the host slots (``slots``) or block ids (``table``), None for
    ``flat``.  Rows whose index is out of range (the device flags and skips them) land in
    bucket 0.  uint8 [tokens] for up to 256 buckets, else uint16 (up to 65,536)."""
    counts = np.maximum(np.asarray(spans["n_tokens"], np.int64), 0)
    total = int(counts.sum())
    if total == 0:
        return np.zeros(0, np.uint8)
    eb = dst.first.element_size()
    bstride, _, ostride = (x * eb for x in dst.strides)
    bs = dst.block_size
    cap = dst.base_tables()[3]
    extent = (cap // bs + 1) * bstride
    shift = min_shift
    while shift < 62 and (extent >> shift) >= buckets:
        shift += 1
    starts = np.cumsum(counts) - counts
    # position within the token sequence, moved per span onto its own positions or index
    # entries: one repeat of a per-span offset, plus one arange
    field = "dst_pos" if mode != "slots" else "dst_index"
    first = np.repeat(np.asarray(spans[field], np.int64) - starts, counts)
    first += np.arange(total, dtype=np.int64)
    if mode == "flat":
        ok = (first >= 0) & (first < cap)
        byte = first * bstride
    else:
        idx = np.asarray(index).reshape(-1)
        if mode == "slots":
            j = first
        else:
            if int(first.min()) < 0:
                first = np.maximum(first, 0)  # negative positions: flagged on the device
            j = np.repeat(np.asarray(spans["dst_index"], np.int64), counts)
            j += first // bs
        if idx.size and int(j.min()) >= 0 and int(j.max()) < idx.size:
            v, ok = idx[j].astype(np.int64, copy=False), None
        else:
            ok = (j >= 0) & (j < idx.size)
            v = (idx[np.clip(j, 0, max(idx.size - 1, 0))].astype(np.int64, copy=False)
                 if idx.size else np.zeros(total, np.int64))
        limit = cap if mode == "slots" else cap // bs
        if not (int(v.min()) >= 0 and int(v.max()) < limit):
            good = (v >= 0) & (v < limit)
            ok = good if ok is None else ok & good
        pos = v if mode == "slots" else first  # what gives the in-block offset
        blk = v // bs if mode == "slots" else v
        if bs & (bs - 1) == 0:
            off = pos & (bs - 1)
        else:
            off = pos % bs
        byte = blk * bstride + off * ostride
    if ok is not None and not bool(ok.all()):
        byte = np.where(ok, byte, 0)
    page = byte >> shift
    if int(page.max()) >= buckets:
        page = np.minimum(page, buckets - 1)
    return page.astype(np.uint8 if buckets <= 256 else np.uint16)


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
