"""``mkv_shift_spans_noalloc`` against ``mkv_shift_spans``, through the C ABI (collected
last: it leaves the library's scratch array holding its records).

The no-allocation entry point keeps its workspace in the library's per-GPU scratch
array instead of a caller-provided one.  Each case runs the same shift twice into two
identical destination caches -- once through ``mkv_shift_spans`` with its workspace,
once through ``mkv_shift_spans_noalloc`` with the descriptor's workspace fields NULL --
and holds both to the oracle bit for bit.  Two calls in a row, the second smaller, so
the second reads a scratch array that still holds the first call's records.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from marathon_amd import _lib
from marathon_amd import workloads as W
from marathon_amd.shift_kernels import current_stream
from marathon_amd.spans import CacheSet, ShiftPlan
from oracle import kvshift_oracle as orc
from tests.helpers import bits, dname, oracle_side, oracle_spans

pytestmark = pytest.mark.gpu


def _noalloc_desc(d: _lib.ShiftDesc) -> _lib.ShiftDesc:
    out = _lib.ShiftDesc()
    ctypes.memmove(ctypes.byref(out), ctypes.byref(d), ctypes.sizeof(_lib.ShiftDesc))
    out.workspace = None
    out.workspace_bytes = 0
    return out


def _run_case(gpu, wl, order="none"):
    L = _lib.lib()
    dst_b = CacheSet([[c.clone() for c in wl.dst.caches[0]]], "hnd", 16)
    want = oracle_side(wl.dst, wl.dst_mode, wl.dst_index)
    src_o = oracle_side(wl.src, wl.src_mode, wl.src_index)
    orc.shift_spans(oracle_spans(wl.spans), src_o, want, wl.inv_freq.numpy(),
                    dname(wl.dst.first.dtype),
                    None if wl.k_scale is None else wl.k_scale.numpy())
    # the two-launch path (the direct path uses no workspace, so no scratch either)
    plan_a = wl.plan(direct=False, order=order)
    plan_b = ShiftPlan(wl.spans, wl.src, dst_b, inv_freq=wl.inv_freq, src_mode=wl.src_mode,
                       src_index=wl.src_index, dst_mode=wl.dst_mode, dst_index=wl.dst_index,
                       k_scale=wl.k_scale, direct=False, order=order)
    assert not plan_a.direct and not plan_b.direct
    torch.cuda.synchronize(gpu)  # both plans' tables have arrived
    stream = ctypes.c_void_p(current_stream(gpu))
    flags = torch.zeros(2, dtype=torch.int32, device=gpu)
    for d in plan_a.descs:
        d.error_flags = flags.data_ptr()
        _lib.check(L.mkv_shift_spans(ctypes.byref(d), stream))
    for d in plan_b.descs:
        nd = _noalloc_desc(d)
        nd.error_flags = flags.data_ptr() + 4
        _lib.check(L.mkv_shift_spans_noalloc(ctypes.byref(nd), stream))
    torch.cuda.synchronize(gpu)
    assert flags.tolist() == [0, 0]
    for layer in range(wl.layers):
        a = bits(wl.dst.caches[0][layer])
        b = bits(dst_b.caches[0][layer])
        assert np.array_equal(b, a), f"layer {layer}: no-alloc differs from the workspace call"
        assert np.array_equal(a, want.caches[0][layer]), f"layer {layer}: differs from the oracle"


@pytest.mark.parametrize("order", ["none", "dst_page", "dst_page_device"])
@pytest.mark.parametrize("dtype", ["bf16", "fp8"])
def test_noalloc_matches_the_workspace_entry_point_twice(gpu, dtype, order):
    for layers, history in ((3, 6144), (2, 1024)):  # the second call is smaller
        print(f"case no-alloc {dtype} order={order} layers={layers} history={history}",
              flush=True)
        if dtype == "bf16":
            wl = W.qwen3_14b_multispan(gpu, layers=layers, history=history, dst_fill="random")
        else:
            wl = W.qwen3_14b_multispan_fp8(gpu, layers=layers, history=history)
        need = _lib.lib().mkv_shift_workspace_size(wl.tokens, len(wl.spans), 128)
        if order != "none":
            need += 32 * wl.tokens + (1 << 20)  # MKV_ORDER_EXTRA_BYTES(total_tokens)
        assert 0 < need <= _lib.MKV_NOALLOC_SCRATCH_BYTES
        _run_case(gpu, wl, order)
        del wl
        torch.cuda.empty_cache()


def test_noalloc_batched_sessions(gpu):
    """32 sessions (groups) x 2 layers in one no-alloc call, then a 2-session call."""
    for sessions, hist_hi in ((32, 1024), (2, 512)):
        print(f"case no-alloc batched sessions={sessions}", flush=True)
        wl = W.batched_sessions(gpu, layers=2, sessions=sessions, hist_lo=256, hist_hi=hist_hi)
        _run_case(gpu, wl)
        del wl
        torch.cuda.empty_cache()


def test_noalloc_replayed_from_a_captured_graph(gpu):
    """The no-allocation entry point's own use case: a call captured in a HIP graph
    (``torch.cuda.graph``) after one eager call on the device has resolved the scratch
    address, then replayed five times, with the program's own eager work (restoring the
    destination, clearing the flags with a fill kernel: no memset node is captured) and a
    synchronisation between replays.  Every replay must write the oracle's bytes."""
    L = _lib.lib()
    wl = W.qwen3_14b_multispan(gpu, layers=2, history=2048, dst_fill="random")
    want = oracle_side(wl.dst, wl.dst_mode, wl.dst_index)
    orc.shift_spans(oracle_spans(wl.spans), oracle_side(wl.src, wl.src_mode, wl.src_index),
                    want, wl.inv_freq.numpy(), dname(wl.dst.first.dtype))
    pristine = [c.clone() for c in wl.dst.caches[0]]
    plan = wl.plan(direct=False)
    assert not plan.direct
    torch.cuda.synchronize(gpu)
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    descs = []
    for d in plan.descs:
        nd = _noalloc_desc(d)
        nd.error_flags = flags.data_ptr()
        descs.append(nd)

    def check(tag):
        assert int(flags.item()) == 0, tag
        for layer in range(wl.layers):
            got = bits(wl.dst.caches[0][layer])
            assert np.array_equal(got, want.caches[0][layer]), f"{tag}: layer {layer} differs"

    side = torch.cuda.Stream(gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):  # the eager call that resolves the scratch address
        for nd in descs:
            _lib.check(L.mkv_shift_spans_noalloc(ctypes.byref(nd),
                                                 ctypes.c_void_p(side.cuda_stream)))
    torch.cuda.synchronize(gpu)
    check("eager")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for nd in descs:
            _lib.check(L.mkv_shift_spans_noalloc(ctypes.byref(nd),
                                                 ctypes.c_void_p(side.cuda_stream)))
    torch.cuda.synchronize(gpu)
    for replay in range(5):
        print(f"case no-alloc graph replay {replay}", flush=True)
        for c, p in zip(wl.dst.caches[0], pristine):
            c.copy_(p)
        flags.zero_()
        torch.cuda.synchronize(gpu)
        graph.replay()
        torch.cuda.synchronize(gpu)
        check(f"replay {replay}")
    del graph
