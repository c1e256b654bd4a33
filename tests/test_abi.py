"""The C ABI: the library loads, exports every declared symbol, its structs match the
header, and its host-side argument checks answer without touching a GPU."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest
import torch

from marathon_amd import _lib
from marathon_amd.shift_kernels import rope_shift, scatter_shifted

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def _declared_functions() -> set[str]:
    names = set()
    for fn in os.listdir(INCLUDE):
        if fn.endswith(".h"):
            text = open(os.path.join(INCLUDE, fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(mkv_\w+)\s*\(", text))
    return names


def test_library_exports_every_declared_function():
    declared = _declared_functions()
    assert declared == set(_lib.EXPORTED), declared
    lib = _lib.lib()
    for name in declared:
        assert hasattr(lib, name), name


def test_abi_version():
    assert _lib.lib().mkv_abi_version() == _lib.MKV_ABI_VERSION


PROBE = r"""
#include <stddef.h>
#include <stdio.h>
#include "marathon_kvshift.h"
#define O(T, f) printf(#T "." #f " %zu\n", offsetof(T, f))
int main(void) {
  printf("span %zu side %zu desc %zu\n", sizeof(mkv_span_t), sizeof(mkv_side_t),
         sizeof(mkv_shift_desc_t));
  O(mkv_span_t, src_pos); O(mkv_span_t, dst_pos); O(mkv_span_t, src_index);
  O(mkv_span_t, dst_index); O(mkv_span_t, n_tokens); O(mkv_span_t, delta);
  O(mkv_span_t, src_group); O(mkv_span_t, dst_group);
  O(mkv_side_t, k_base); O(mkv_side_t, v_base); O(mkv_side_t, index);
  O(mkv_side_t, group_slots); O(mkv_side_t, index_len); O(mkv_side_t, num_slots);
  O(mkv_side_t, block_stride); O(mkv_side_t, head_stride); O(mkv_side_t, offset_stride);
  O(mkv_side_t, block_size); O(mkv_side_t, mode); O(mkv_side_t, groups);
  O(mkv_shift_desc_t, spans); O(mkv_shift_desc_t, inv_freq); O(mkv_shift_desc_t, k_scale);
  O(mkv_shift_desc_t, error_flags); O(mkv_shift_desc_t, workspace);
  O(mkv_shift_desc_t, workspace_bytes); O(mkv_shift_desc_t, total_tokens);
  O(mkv_shift_desc_t, n_spans); O(mkv_shift_desc_t, layers);
  O(mkv_shift_desc_t, heads); O(mkv_shift_desc_t, head_size); O(mkv_shift_desc_t, rotary);
  O(mkv_shift_desc_t, dtype); O(mkv_shift_desc_t, src); O(mkv_shift_desc_t, dst);
  O(mkv_shift_desc_t, span_starts); O(mkv_shift_desc_t, span_tables);
  O(mkv_shift_desc_t, order);
  return 0;
}
"""


def test_struct_layout_matches_the_header(tmp_path):
    src = tmp_path / "probe.c"
    src.write_text(PROBE)
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c99", f"-I{INCLUDE}", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    sizes = out[0].split()
    assert int(sizes[1]) == ctypes.sizeof(_lib.Span)
    assert int(sizes[3]) == ctypes.sizeof(_lib.Side)
    assert int(sizes[5]) == ctypes.sizeof(_lib.ShiftDesc)
    types = {"mkv_span_t": _lib.Span, "mkv_side_t": _lib.Side, "mkv_shift_desc_t": _lib.ShiftDesc}
    for line in out[1:]:
        if not line:
            continue
        key, off = line.split()
        tname, field = key.split(".")
        assert getattr(types[tname], field).offset == int(off), key
    assert _lib.SPAN_DTYPE.itemsize == ctypes.sizeof(_lib.Span)
    for name in _lib.SPAN_DTYPE.names:
        assert _lib.SPAN_DTYPE.fields[name][1] == getattr(_lib.Span, name).offset


def _scatter(**kw):
    args = dict(src=1 << 20, sts=2048, shs=256, kv=1 << 24, kbs=32768, khs=4096, kos=256,
                nblk=64, slots=1 << 21, n=8, heads=8, d=128, bs=16, dtype=_lib.MKV_BF16,
                cos=1 << 22, sgn=1 << 23, rot=128, scale=None, err=None)
    args.update(kw)
    return _lib.lib().mkv_scatter_shifted(*args.values(), None)


def test_host_side_argument_errors_need_no_gpu():
    lib = _lib.lib()
    assert _scatter(dtype=9) == _lib.MKV_ERR_DTYPE
    assert b"dtype" in lib.mkv_last_error()
    assert _scatter(d=0) == _lib.MKV_ERR_UNSUPPORTED
    assert _scatter(d=1024, rot=128) == _lib.MKV_ERR_UNSUPPORTED
    assert _scatter(rot=256) == _lib.MKV_ERR_ARG  # rotary > head_size (shift_kernels.py:71)
    assert _scatter(rot=72) == _lib.MKV_ERR_UNSUPPORTED  # not a multiple of 16 for bf16
    assert _scatter(d=100) == _lib.MKV_ERR_UNSUPPORTED  # 200-byte head is not 16-byte sized
    assert _scatter(heads=0) == _lib.MKV_ERR_ARG
    assert _scatter(n=-1) == _lib.MKV_ERR_ARG
    assert _scatter(src=None) == _lib.MKV_ERR_ARG
    assert _scatter(sgn=None) == _lib.MKV_ERR_ARG  # cos without sgn
    assert _scatter(dtype=_lib.MKV_FP8_E4M3, scale=None) == _lib.MKV_ERR_ARG
    assert _scatter(src=(1 << 20) + 8) == _lib.MKV_ERR_ALIGN
    assert _scatter(sts=2047) == _lib.MKV_ERR_ALIGN
    assert _scatter(shs=252) == _lib.MKV_ERR_ALIGN  # a 504-byte head stride
    assert b"head stride" in lib.mkv_last_error()
    # the reference returns early on an empty load (shift_kernels.py:185-186)
    assert _scatter(n=0) == _lib.MKV_OK
    assert lib.mkv_last_error() == b""


def test_batched_entry_point_argument_errors_need_no_gpu():
    lib = _lib.lib()
    assert lib.mkv_shift_spans(None, None) == _lib.MKV_ERR_ARG
    d = _lib.ShiftDesc()
    d.heads, d.head_size, d.rotary, d.dtype, d.layers = 8, 128, 128, _lib.MKV_BF16, 2
    d.n_spans = 0
    assert lib.mkv_shift_spans(ctypes.byref(d), None) == _lib.MKV_OK
    d.n_spans = _lib.MKV_MAX_SPANS + 1
    assert lib.mkv_shift_spans(ctypes.byref(d), None) == _lib.MKV_ERR_UNSUPPORTED
    d.n_spans = 1
    d.total_tokens = 100
    assert lib.mkv_shift_spans(ctypes.byref(d), None) == _lib.MKV_ERR_ARG  # NULL spans
    d.spans = 1 << 20
    d.inv_freq = 1 << 21
    for side in (d.src, d.dst):
        side.k_base, side.v_base = 1 << 24, 1 << 25
        side.mode, side.block_size, side.groups = _lib.MKV_ADDR_FLAT, 1, 1
    assert lib.mkv_shift_spans(ctypes.byref(d), None) == _lib.MKV_ERR_ARG
    assert b"workspace" in lib.mkv_last_error()
    need = lib.mkv_shift_workspace_size(100, 1, 128)
    assert need == 2 * 128 * 4 + 100 * 32  # one span's cos/sgn tables + 32 B per token
    assert lib.mkv_shift_workspace_size(-1, 1, 128) == -1
    d.workspace, d.workspace_bytes = 1 << 26, need - 1
    assert lib.mkv_shift_spans(ctypes.byref(d), None) == _lib.MKV_ERR_ARG
    d.workspace_bytes = need
    d.src.mode = 7
    assert lib.mkv_shift_spans(ctypes.byref(d), None) == _lib.MKV_ERR_ARG
    assert b"mode" in lib.mkv_last_error()
    # fp8 needs the layers' K scales only when it rotates (the check precedes any launch)
    d.src.mode = _lib.MKV_ADDR_FLAT
    d.dtype, d.k_scale = _lib.MKV_FP8_E4M3, None
    assert lib.mkv_shift_spans(ctypes.byref(d), None) == _lib.MKV_ERR_ARG
    assert b"k_scale" in lib.mkv_last_error()


def test_noalloc_entry_point_refuses_shifts_beyond_its_scratch_without_a_gpu():
    """The no-allocation entry point checks its size limit before any HIP call."""
    lib = _lib.lib()
    assert lib.mkv_shift_spans_noalloc(None, None) == _lib.MKV_ERR_ARG
    d = _lib.ShiftDesc()
    d.heads, d.head_size, d.rotary, d.dtype, d.layers = 8, 128, 128, _lib.MKV_BF16, 2
    d.n_spans, d.spans, d.inv_freq = 1, 1 << 20, 1 << 21
    for side in (d.src, d.dst):
        side.k_base, side.v_base = 1 << 24, 1 << 25
        side.mode, side.block_size, side.groups = _lib.MKV_ADDR_FLAT, 1, 1
    d.total_tokens = _lib.MKV_NOALLOC_SCRATCH_BYTES // 32  # records alone fill the buffer
    assert lib.mkv_shift_workspace_size(d.total_tokens, 1, 128) > _lib.MKV_NOALLOC_SCRATCH_BYTES
    assert lib.mkv_shift_spans_noalloc(ctypes.byref(d), None) == _lib.MKV_ERR_UNSUPPORTED
    assert b"no-allocation scratch" in lib.mkv_last_error()
    d.n_spans = 0  # an empty shift is a no-op, as for mkv_shift_spans
    assert lib.mkv_shift_spans_noalloc(ctypes.byref(d), None) == _lib.MKV_OK


def test_small_entry_point_checks_its_limits_without_a_gpu():
    """mkv_shift_spans_small refuses what does not fit a launch's arguments, and spans
    that disagree with total_tokens, before any HIP call."""
    import numpy as np

    lib = _lib.lib()
    d = _lib.ShiftDesc()
    d.heads, d.head_size, d.rotary, d.dtype, d.layers = 8, 128, 128, _lib.MKV_BF16, 2
    d.inv_freq = 1 << 21
    for side in (d.src, d.dst):
        side.k_base, side.v_base = 1 << 24, 1 << 25
        side.mode, side.block_size, side.groups = _lib.MKV_ADDR_FLAT, 1, 1
    spans = np.zeros(9, dtype=_lib.SPAN_DTYPE)
    spans["n_tokens"] = 2
    d.spans = spans.ctypes.data
    d.n_spans, d.total_tokens = 9, 18
    assert lib.mkv_shift_spans_small(ctypes.byref(d), None) == _lib.MKV_ERR_UNSUPPORTED
    d.n_spans = 2
    for total in (3, 5):  # the spans hold 4: fewer and more are both refused
        d.total_tokens = total
        assert lib.mkv_shift_spans_small(ctypes.byref(d), None) == _lib.MKV_ERR_ARG
        assert b"total_tokens" in lib.mkv_last_error()
    spans["n_tokens"][0] = -1
    d.total_tokens = 4
    assert lib.mkv_shift_spans_small(ctypes.byref(d), None) == _lib.MKV_ERR_ARG
    spans["n_tokens"][0] = 2
    idx = np.zeros(65, np.int64)
    d.dst.mode, d.dst.block_size, d.dst.index, d.dst.index_len = (
        _lib.MKV_ADDR_SLOTS, 16, idx.ctypes.data, 65)
    assert lib.mkv_shift_spans_small(ctypes.byref(d), None) == _lib.MKV_ERR_UNSUPPORTED
    d.dst.index_len = 4
    d.heads = 2  # 2 of the 4 rows a bf16 wave covers: not the direct geometry
    assert lib.mkv_shift_spans_small(ctypes.byref(d), None) == _lib.MKV_ERR_UNSUPPORTED
    d.heads, d.dst.block_size = 8, 24
    assert lib.mkv_shift_spans_small(ctypes.byref(d), None) == _lib.MKV_ERR_UNSUPPORTED


def test_python_api_refuses_tensors_off_the_gpu():
    src = torch.zeros(4, 8, 256, dtype=torch.bfloat16)
    kv = torch.zeros(4, 8, 16, 256, dtype=torch.bfloat16)
    inv = 1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))
    with pytest.raises(RuntimeError, match="no CPU path"):
        scatter_shifted(src, kv, torch.arange(4), 16, True, rope_shift(3, 128, inv, "cpu"))


def test_fp8_k_scale_outside_the_exact_division_range_is_refused_on_the_host():
    """A Python-float K scale must lie where the fp8 quotient is correctly rounded
    ([2^-90, 2^100]); the check runs before any device tensor is made."""
    from marathon_amd.shift_kernels import _scale_tensor

    for bad in (0.0, -0.05, float("nan"), float("inf"), 2.0 ** -91, 2.0 ** 101):
        with pytest.raises(ValueError, match="outside"):
            _scale_tensor(bad, torch.device("cuda", 0))


def test_rope_shift_asserts_rotary_fits():
    inv = torch.ones(80)
    with pytest.raises(AssertionError, match="rotary 160 > head_size 128"):
        rope_shift(1, 128, inv, "cpu")


def test_cacheset_split_planes_are_validated_and_sized():
    """Split K and V planes: rows of D (not 2D), V base addresses from the V tensors,
    and a V tensor that differs from its K tensor is refused."""
    import numpy as np

    from marathon_amd.spans import CacheSet

    k = [torch.zeros(10, 16, 4, 128, dtype=torch.bfloat16) for _ in range(3)]
    v = [torch.zeros(10, 16, 4, 128, dtype=torch.bfloat16) for _ in range(3)]
    cs = CacheSet([k], "nhd", 16, v_caches=[v])
    assert (cs.split, cs.heads, cs.head_size, cs.layers) == (True, 4, 128, 3)
    kb, vb, caps, min_cap, uniform = cs.base_tables()
    assert list(kb[0]) == [t.data_ptr() for t in k]
    assert list(vb[0]) == [t.data_ptr() for t in v]
    assert min_cap == 160 and uniform and caps.dtype == np.int64
    fused = CacheSet([[torch.zeros(10, 16, 4, 256, dtype=torch.bfloat16)]], "nhd", 16)
    assert (fused.split, fused.head_size) == (False, 128)
    with pytest.raises(ValueError, match="differs from its K tensor"):
        CacheSet([k], "nhd", 16, v_caches=[[*v[:2], torch.zeros(10, 16, 4, 64,
                                                                dtype=torch.bfloat16)]])
    with pytest.raises(ValueError, match="group by group"):
        CacheSet([k], "nhd", 16, v_caches=[v[:2]])


def test_cacheset_takes_a_flat_list_of_layers():
    """A flat list of per-layer tensors is one group, in every layout."""
    from marathon_amd.spans import CacheSet

    flat = CacheSet([torch.zeros(64, 8, 256) for _ in range(2)], "flat")
    assert (flat.groups, flat.layers, flat.heads, flat.head_size) == (1, 2, 8, 128)
    hnd = CacheSet([torch.zeros(4, 8, 16, 256)], "hnd", 16)
    assert (hnd.groups, hnd.layers, hnd.block_size) == (1, 1, 16)
    k = [torch.zeros(4, 16, 8, 128)]
    split = CacheSet(k, "nhd", 16, v_caches=[torch.zeros(4, 16, 8, 128)])
    assert (split.groups, split.split, split.head_size) == (1, True, 128)
    with pytest.raises(ValueError, match="empty"):
        CacheSet([], "flat")
    with pytest.raises(ValueError, match="empty"):
        CacheSet([[]], "flat")


def test_cacheset_strides_ignore_dims_of_one_element():
    """A one-row store cut from a wider tensor keeps its parent's strides (torch calls
    it contiguous): the set accepts it beside a store of many rows, and addresses every
    tensor with the strides of the dims that have more than one element."""
    from marathon_amd.spans import CacheSet

    d = 64
    short = torch.zeros(1, 1, 2 * d)
    long = torch.zeros(200, 1, 2 * d)
    ks = [short[..., :d].contiguous(), long[..., :d].contiguous()]
    vs = [short[..., d:].contiguous(), long[..., d:].contiguous()]
    assert ks[0].stride() == (128, 128, 1) and ks[1].stride() == (64, 64, 1)
    # the row stride is the 200-row store's; the head dim has one element everywhere, so
    # its stride is the first tensor's (it only ever multiplies head 0)
    cs = CacheSet([[ks[0]], [ks[1]]], "flat", v_caches=[[vs[0]], [vs[1]]])
    assert cs.strides == (64, 128, 0)
    cs = CacheSet([[ks[1]], [ks[0]]], "flat", v_caches=[[vs[1]], [vs[0]]])
    assert cs.strides == (64, 64, 0)
    # a real dim that differs is still refused
    wide = torch.zeros(10, 8, 512)[..., :256]  # rows of 256 at a head stride of 512
    with pytest.raises(ValueError, match="trailing shape or strides"):
        CacheSet([[torch.zeros(10, 8, 256)], [wide]], "flat")
    with pytest.raises(ValueError, match="differs from its K tensor"):
        CacheSet([[torch.zeros(10, 8, 256)]], "flat", v_caches=[[wide]])
    # and paged: a one-block cache beside a many-block one, block stride from the latter
    one = torch.zeros(1, 8, 16, 512)[..., :256]
    many = torch.zeros(6, 8, 16, 256)
    with pytest.raises(ValueError, match="trailing shape or strides"):
        CacheSet([[many], [one]], "hnd", 16)  # its head and offset strides are real
    blk = torch.zeros(2, 8, 16, 256)[::2]  # one block, at a block stride of two blocks
    assert blk.shape[0] == 1 and blk.stride(0) == 2 * 8 * 16 * 256
    for groups in ([[blk], [many]], [[many], [blk]]):
        assert CacheSet(groups, "hnd", 16).strides == (8 * 16 * 256, 16 * 256, 256)


def test_store_planes_and_fused_rows_hold_the_same_rows():
    """The workloads' session-store blocks in either layout: a K plane then a V plane per
    block (strided views of one tensor, split K/V caches to the kernels) or rows of K then
    V; ``CacheSet.fused`` gives the same [..., 2D] rows back from either."""
    from marathon_amd import workloads as W

    gen = torch.Generator().manual_seed(3)
    planes = W.store_blocks(5, 4, torch.bfloat16, gen, "cpu", layout="planes")
    assert planes.shape == (5, 2, 16, 4, 128)
    cs = W.store_cache_set([[planes]], "planes")
    assert cs.split and cs.layout == "nhd" and cs.head_size == 128 and cs.heads == 4
    k, v = cs.caches[0][0], cs.v_caches[0][0]
    assert k.data_ptr() == planes.data_ptr()
    assert v.data_ptr() - k.data_ptr() == 16 * 4 * 128 * 2  # the V plane follows the K plane
    rows = torch.cat((planes[:, 0], planes[:, 1]), dim=-1)  # [5, 16, 4, 256]
    fused = W.store_cache_set([[rows.contiguous()]], "fused")
    assert not fused.split and fused.head_size == 128
    blk, off = torch.tensor([4, 0, 2]), torch.tensor([15, 3, 8])
    assert torch.equal(cs.fused(0, 0, (blk, off)), fused.fused(0, 0, (blk, off)))
    assert torch.equal(cs.fused(0, 0), rows)
    with pytest.raises(ValueError, match="store layout"):
        W.store_blocks(5, 4, torch.bfloat16, gen, "cpu", layout="hnd")


def test_cacheset_refuses_a_group_whose_layers_differ_in_length():
    """The device checks a group's slots against one capacity, its first layer's: a
    shorter (or longer) layer in the same group would let a slot past its end through, so
    the set refuses it.  Groups may still differ from one another."""
    from marathon_amd.spans import CacheSet

    with pytest.raises(ValueError, match="layers of a group differ"):
        CacheSet([torch.zeros(8, 8, 16, 256), torch.zeros(6, 8, 16, 256)], "hnd", 16)
    with pytest.raises(ValueError, match="layers of a group differ"):
        CacheSet([[torch.zeros(100, 8, 256), torch.zeros(120, 8, 256)]], "flat")
    cs = CacheSet([[torch.zeros(8, 8, 16, 256)] * 2, [torch.zeros(6, 8, 16, 256)] * 2], "hnd", 16)
    _, _, caps, low, uniform = cs.base_tables()
    assert caps.tolist() == [128, 96] and low == 96 and not uniform


def test_dropin_and_rotary_width_on_the_host():
    """The reference-side binding refuses a CPU cache (no CPU path), and both bindings
    take the rotary width from ``emb_cos`` (host metadata) -- a reference-shaped
    ``RopeShift`` with no ``rotary`` field works, a contradicting field is refused."""
    from types import SimpleNamespace

    from marathon_amd.shift_kernels import shift_rotary
    from marathon_amd.shift_kernels_hip import scatter_shifted as dropin

    inv = 1.0 / (1e6 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))
    shift = rope_shift(7, 128, inv, "cpu")
    assert shift_rotary(shift) == 64 and shift_rotary(None) == 0
    ref_shaped = SimpleNamespace(delta=7, cos=shift.cos, sgn=shift.sgn, partner=shift.partner,
                                 emb_cos=shift.emb_cos, emb_sin=shift.emb_sin)
    assert shift_rotary(ref_shaped) == 64
    ref_shaped.rotary = 128
    with pytest.raises(ValueError, match="rotary"):
        shift_rotary(ref_shaped)
    src = torch.zeros(4, 8, 256, dtype=torch.bfloat16)
    kv = torch.zeros(4, 8, 16, 256, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        dropin(src, kv, torch.arange(4), 16, True, shift)


def test_rope_shift_reference_tables_are_the_reference_construction():
    """``tables="reference"`` builds the reference's tables with torch fp32 (on the CPU
    here): the same bits as the reference's construction restated in oracle/torch_path.py
    (shift_kernels.py:68-84); the default tables are the correctly rounded ones."""
    from oracle import kvshift_oracle as orc
    from oracle import torch_path

    for rotary in (128, 64):
        inv = 1.0 / (1e6 ** (torch.arange(0, rotary, 2, dtype=torch.float32) / rotary))
        for delta in (-3000, 186, 2**25 + 1):
            got = rope_shift(delta, 128, inv, "cpu", tables="reference")
            want = torch_path.rope_shift_tables(delta, 128, inv, "cpu")
            for name in ("cos", "sgn", "partner", "emb_cos", "emb_sin"):
                assert torch.equal(getattr(got, name), want[name]), name
            assert got.rotary == rotary
            exact = rope_shift(delta, 128, inv, "cpu")
            c, s = orc.cos_sin(delta, inv.numpy())
            assert np.array_equal(exact.emb_cos.numpy()[: rotary // 2], c)
            assert np.array_equal(exact.emb_sin.numpy()[: rotary // 2], s)
    with pytest.raises(ValueError, match="tables"):
        rope_shift(1, 128, inv, "cpu", tables="torch")


def test_token_order_and_device_order_are_refused_together():
    """The caller's token order and the device's page sort are two ways to order one
    shift; a descriptor asking for both is refused before anything is enqueued."""
    lib = _lib.lib()
    d = _lib.ShiftDesc()
    d.heads, d.head_size, d.rotary, d.dtype, d.layers = 8, 128, 128, _lib.MKV_BF16, 2
    d.inv_freq = 1 << 21
    d.spans = 1 << 22
    d.n_spans, d.total_tokens = 1, 16
    for side in (d.src, d.dst):
        side.k_base, side.v_base = 1 << 24, 1 << 25
        side.mode, side.block_size, side.groups = _lib.MKV_ADDR_FLAT, 1, 1
    d.order = _lib.MKV_ORDER_DST_PAGE
    d.token_order = 1 << 23
    assert lib.mkv_shift_spans(ctypes.byref(d), None) == _lib.MKV_ERR_ARG
    assert b"token_order" in lib.mkv_last_error()


def test_host_page_order_matches_a_brute_force_restatement():
    """``spans.dst_page_order`` (the pages ShiftPlan sorts by on the host) equals a
    per-token restatement of the device's bucket rule, for slots, block tables and a flat
    destination; the resulting order is a stable permutation."""
    from marathon_amd.spans import CacheSet, dst_page_order, span_array

    rng = np.random.default_rng(5)
    blocks, bs = 3000, 16  # 3,000 x 64 KB: wider than 256 pages of 2 MB
    hnd = CacheSet([torch.zeros(blocks, 8, bs, 256, dtype=torch.bfloat16)], "hnd", bs)
    bstride, ostride = 8 * bs * 256 * 2, 256 * 2
    extent = (blocks + 1) * bstride
    shift = 21
    while (extent >> shift) >= 256:
        shift += 1
    table = rng.permutation(blocks).astype(np.int32)
    slots = rng.permutation(blocks * bs)[:900].astype(np.int64)
    spans = span_array([(0, 5, 0, 0, 400, 7, 0, 0), (0, 900, 0, 400, 500, -3, 0, 0)])
    want_slots, want_table = [], []
    for sp in spans:
        for i in range(int(sp["n_tokens"])):
            s = int(slots[int(sp["dst_index"]) + i])
            want_slots.append(min(((s // bs) * bstride + (s % bs) * ostride) >> shift, 255))
            pos = int(sp["dst_pos"]) + i
            b = int(table[pos // bs])  # the table case below uses dst_index 0
            want_table.append(min((b * bstride + (pos % bs) * ostride) >> shift, 255))
    got = dst_page_order(spans, hnd, "slots", slots)
    assert got.dtype == np.uint8 and got.tolist() == want_slots
    spans_t = spans.copy()
    spans_t["dst_index"] = 0
    assert dst_page_order(spans_t, hnd, "table", table).tolist() == want_table
    perm = np.argsort(got, kind="stable")
    assert sorted(perm.tolist()) == list(range(got.size))
    assert all(got[perm][:-1] <= got[perm][1:])
    flat = CacheSet([torch.zeros(5000, 8, 256, dtype=torch.bfloat16)], "flat")
    fl = dst_page_order(span_array([(0, 10, 0, 0, 4000, 1, 0, 0)]), flat, "flat", None)
    fext = (5000 + 1) * 8 * 256 * 2
    fshift = 21
    while (fext >> fshift) >= 256:
        fshift += 1
    assert fl.tolist() == [min(((10 + i) * 8 * 256 * 2) >> fshift, 255) for i in range(4000)]
    # an out-of-range slot lands in bucket 0 (the device flags and skips it)
    bad = slots.copy()
    bad[3] = blocks * bs + 7
    assert dst_page_order(spans, hnd, "slots", bad)[3] == 0
