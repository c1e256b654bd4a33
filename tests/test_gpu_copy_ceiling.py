"""The benchmark's ceiling copies (tests/hip/copy_ceiling.hip) copy exactly what they claim
to: the stream copy byte for byte with either store policy and by a persistent grid,
and the paged copy every row
of positions [0, n) through both block tables -- bf16 from K/V planes, fp8 from fused
rows, into an HND cache -- leaving every other row untouched, with a wave's rows in one
token (8 heads) or each lane resolving its own row (1, 2 or 8 heads, either store), and
with K and V in separate waves or K's store held behind a dependent table read."""

from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest
import torch

from marathon_amd import workloads as W

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libcopy_ceiling.so")


def _lib():
    lib = ctypes.CDLL(LIB)
    i32, i64, vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p
    lib.ceil_stream_copy.argtypes = [vp, vp, i64, i32, vp]
    lib.ceil_stream_copy_persistent.argtypes = [vp, vp, i64, i32, vp]
    lib.ceil_paged_copy.argtypes = [vp, vp, vp, vp, i32, vp, i64, i64, vp, i64, i64, i64, i32,
                                    i32, i64, i64, i64, i64, i64, i64, vp]
    lib.ceil_paged_copy_lanes.argtypes = [vp, vp, vp, vp, i32, vp, i64, i64, vp, i64, i64, i64,
                                          i32, i32, i64, i64, i64, i64, i64, i64, i32, vp]
    lib.ceil_paged_copy_ex.argtypes = [vp, vp, vp, vp, i32, vp, i64, i64, vp, i64, i64, i64,
                                       i32, i32, i64, i64, i64, i64, i64, i64, i32, vp, vp]
    return lib


@pytest.mark.parametrize("scope", [0, 1])
@pytest.mark.parametrize("nbytes", [16, 4096 * 8 + 48, 3 * 2**20 + 16])
def test_stream_copy(gpu, scope, nbytes):
    print(f"case stream copy scope={scope} bytes={nbytes}", flush=True)
    lib = _lib()
    src = torch.randint(0, 255, (nbytes + 64,), dtype=torch.uint8, device=gpu)
    dst = torch.zeros_like(src)
    assert lib.ceil_stream_copy(src.data_ptr(), dst.data_ptr(), nbytes, scope, None) == 0
    torch.cuda.synchronize(gpu)
    assert torch.equal(dst[:nbytes], src[:nbytes])
    assert int(dst[nbytes:].count_nonzero()) == 0  # nothing past the end
    assert lib.ceil_stream_copy(src.data_ptr(), dst.data_ptr(), 24, scope, None) == 1


@pytest.mark.parametrize("wgs", [1, 7, 300])
@pytest.mark.parametrize("nbytes", [16, 4096 * 8 + 48, 3 * 2**20 + 16])
def test_stream_copy_persistent(gpu, wgs, nbytes):
    print(f"case persistent stream copy workgroups={wgs} bytes={nbytes}", flush=True)
    lib = _lib()
    src = torch.randint(0, 255, (nbytes + 64,), dtype=torch.uint8, device=gpu)
    dst = torch.zeros_like(src)
    assert lib.ceil_stream_copy_persistent(src.data_ptr(), dst.data_ptr(), nbytes, wgs, None) == 0
    torch.cuda.synchronize(gpu)
    assert torch.equal(dst[:nbytes], src[:nbytes])
    assert int(dst[nbytes:].count_nonzero()) == 0
    assert lib.ceil_stream_copy_persistent(src.data_ptr(), dst.data_ptr(), nbytes, 0, None) == 1


# (heads, lanes): lanes None = ceil_paged_copy, 0 / 1 = ceil_paged_copy_lanes with nt /
# sc1 nt stores, "split" / "read" / "split_read" = ceil_paged_copy_ex with K and V in
# separate waves, K behind a table read, or both
CASES = [(8, None), (8, 0), (8, 1), (2, 1), (1, 0), (1, 1), (8, "split"), (8, "read"),
         (8, "split_read")]


@pytest.mark.parametrize("heads,lanes", CASES)
@pytest.mark.parametrize("dtype", ["bf16", "fp8"])
def test_paged_copy(gpu, dtype, heads, lanes):
    print(f"case paged copy {dtype} heads={heads} lanes={lanes}", flush=True)
    lib = _lib()
    make = W.qwen3_14b_multispan if dtype == "bf16" else W.qwen3_14b_multispan_fp8
    wl = make(gpu, layers=3, history=1024, heads=heads)
    eb = wl.dst.first.element_size()
    heads, d = wl.dst.heads, wl.dst.head_size
    src_blocks, dst_blocks = wl.src.first.shape[0], wl.dst.first.shape[0]
    rng = np.random.default_rng(1)
    n = 16 * src_blocks - 5  # ragged last block
    st = rng.permutation(src_blocks).astype(np.int32)
    dt = rng.permutation(dst_blocks)[:src_blocks].astype(np.int32)
    before = [c.clone() for c in wl.dst.caches[0]]
    s_k, s_v, _, _, _ = wl.src.device_tables(gpu)
    d_k, d_v, _, _, _ = wl.dst.device_tables(gpu)
    torch.cuda.synchronize(gpu)
    st_dev, dt_dev = torch.from_numpy(st).to(gpu), torch.from_numpy(dt).to(gpu)
    args = (s_k, s_v, d_k, d_v, wl.layers, st_dev.data_ptr(), st.size, src_blocks,
            dt_dev.data_ptr(), dt.size, dst_blocks, n, heads, d * eb,
            *[x * eb for x in wl.src.strides], *[x * eb for x in wl.dst.strides])
    zeros = torch.zeros(16, dtype=torch.int32, device=gpu)

    def call(a):
        if lanes is None:
            return lib.ceil_paged_copy(*a, None)
        if isinstance(lanes, str):
            return lib.ceil_paged_copy_ex(*a, int("split" in lanes),
                                          zeros.data_ptr() if "read" in lanes else None, None)
        return lib.ceil_paged_copy_lanes(*a, lanes, None)

    assert call(args) == 0
    torch.cuda.synchronize(gpu)
    pos = np.arange(n)
    for layer in range(wl.layers):
        want = before[layer].clone()
        src = wl.src.fused(0, layer, (torch.from_numpy(st[pos // 16].astype(np.int64)),
                                      torch.from_numpy(pos % 16)))
        want[torch.from_numpy(dt[pos // 16].astype(np.int64)), :, torch.from_numpy(pos % 16)] = src
        got = wl.dst.caches[0][layer]
        assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), f"layer {layer}"
    # tables shorter than the positions need are refused
    short = (*args[:6], 2, *args[7:])
    assert call(short) == 1
