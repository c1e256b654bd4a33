"""Small steps (a decode step's saves, short loads) through ``SmallShifts``, on the GPU.

Up to 8 spans and 64 index entries a side, a step travels in the launch's own kernel
arguments (``mkv_shift_spans_small``: rows and index windows from host memory, rotation
tables computed in the kernel); larger direct steps go through the runner's device
buffer (``mkv_shift_spans`` direct path).  Seeded random steps over element types,
source and destination modes, groups and deltas of every magnitude, run one after
another through one runner, each checked byte for byte against the oracle.
"""

from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

from marathon_amd import _lib
from marathon_amd.spans import SMALL_ARGS_MAX_TOKEN_LAYERS, CacheSet, SmallShifts
from oracle import kvshift_oracle as orc
from tests.helpers import bits, dname, inv_freq, oracle_side, oracle_spans, randn

pytestmark = pytest.mark.gpu

BS = 16


def _runner_case(gpu, dtype, src_mode, dst_mode, heads, groups, seed):
    gen = torch.Generator().manual_seed(seed)
    layers, d = 3, 128
    sc = 0.05
    if src_mode == "flat":  # session stores, slot = position
        src_caches = [[randn((300, heads, 2 * d), dtype, gen, sc) for _ in range(layers)]
                      for _ in range(groups)]
        src = CacheSet([[t.to(gpu) for t in row] for row in src_caches], "flat")
    else:  # block-layout store, NHD blocks
        src_caches = [[randn((40, BS, heads, 2 * d), dtype, gen, sc) for _ in range(layers)]]
        src = CacheSet([[t.to(gpu) for t in row] for row in src_caches], "nhd", BS)
    dst_caches = [[randn((40, heads, BS, 2 * d), dtype, gen, sc) for _ in range(layers)]]
    dst = CacheSet([[t.to(gpu) for t in row] for row in dst_caches], "hnd", BS)
    k_scale = (torch.from_numpy(np.float32([0.031, 0.066, 0.05])) if dtype == torch.float8_e4m3fn
               else None)
    runner = SmallShifts(src, dst, inv_freq=inv_freq(), src_mode=src_mode, dst_mode=dst_mode,
                         k_scale=k_scale)
    return runner, src, dst, k_scale


def _step(rng, src_mode, dst_mode, groups, n_spans, max_tokens):
    """Random disjoint destination runs, sources anywhere; index windows as a caller's."""
    rows, src_idx, dst_idx = [], [], []
    dst_blocks = rng.permutation(40)
    free_pos = rng.permutation(np.arange(0, 40 * BS - max_tokens, max_tokens))  # disjoint
    for k in range(n_spans):
        n = int(rng.integers(1, max_tokens + 1))
        delta = int(rng.choice([0, 1, -7, 186, -3000, 2**31 - 1, int(rng.integers(-9999, 9999))]))
        g = int(rng.integers(groups)) if src_mode == "flat" else 0
        if src_mode == "flat":
            spos, sidx = int(rng.integers(0, 300 - n)), 0
        else:  # a window of the store's table: blocks of positions [spos, spos + n)
            p0 = int(rng.integers(0, 40 * BS - n))
            k0, k1 = p0 // BS, -(-(p0 + n) // BS)
            sidx = len(src_idx)
            src_idx.extend(rng.permutation(40)[: k1 - k0].tolist())
            spos = p0 - k0 * BS
        d0 = int(free_pos[k])
        if dst_mode == "slots":
            didx = len(dst_idx)
            pos = np.arange(d0, d0 + n)
            dst_idx.extend((dst_blocks[pos // BS] * BS + pos % BS).tolist())
            dpos = 0
        else:
            k0, k1 = d0 // BS, -(-(d0 + n) // BS)
            didx = len(dst_idx)
            dst_idx.extend(dst_blocks[k0:k1].tolist())
            dpos = d0 - k0 * BS
        rows.append((spos, dpos, sidx, didx, n, delta, g, 0))
    si = None if src_mode == "flat" else np.asarray(src_idx, np.int32)
    di = np.asarray(dst_idx, np.int64 if dst_mode == "slots" else np.int32)
    return rows, si, di


# more seeds for a longer sweep: MKV_SMALL_CASES=50 python -m pytest tests/test_gpu_small.py
_REPS = 1 + int(__import__("os").environ.get("MKV_SMALL_CASES", "0"))


@pytest.mark.parametrize("rep", range(_REPS))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32,
                                   torch.float8_e4m3fn])
@pytest.mark.parametrize("src_mode,dst_mode", [("flat", "slots"), ("table", "table"),
                                               ("flat", "table"), ("table", "slots")])
def test_small_steps_match_oracle(gpu, dtype, src_mode, dst_mode, rep):
    eb = torch.empty(0, dtype=dtype).element_size()
    heads = 64 // (128 * eb // 16)  # the smallest head count a wave pass covers
    groups = 3 if src_mode == "flat" else 1
    # a seed that is the same in every process (str hashes are not)
    seed = zlib.crc32(f"{dtype} {src_mode} {dst_mode}".encode()) % 10_000 + 10_000 * rep
    print(f"case small steps {dtype} {src_mode}->{dst_mode} seed={seed}", flush=True)
    runner, src, dst, k_scale = _runner_case(gpu, dtype, src_mode, dst_mode, heads, groups, seed)
    rng = np.random.default_rng(seed)
    inv = inv_freq().numpy()
    src_bits = [[bits(t) for t in row] for row in src.caches]
    # 1 token (a decode save), a few spans, then steps past the in-launch limits
    for n_spans, max_tokens in ((1, 1), (3, 12), (8, 6), (12, 5), (4, 30)):
        rows, si, di = _step(rng, src_mode, dst_mode, groups, n_spans, max_tokens)
        tokens = sum(r[4] for r in rows)
        small = (n_spans <= _lib.MKV_SMALL_MAX_SPANS and di.size <= _lib.MKV_SMALL_MAX_INDEX
                 and (si is None or si.size <= _lib.MKV_SMALL_MAX_INDEX)
                 and tokens * dst.layers <= SMALL_ARGS_MAX_TOKEN_LAYERS)
        print(f"case small step {dtype} {src_mode}->{dst_mode} spans={n_spans} "
              f"in-launch={small}", flush=True)
        assert runner.fits(n_spans, tokens)
        want = oracle_side(dst, dst_mode, torch.from_numpy(di))
        src_o = orc.Side(src_bits, src.layout, src.block_size, src_mode, si)
        from marathon_amd.spans import span_array

        orc.shift_spans(oracle_spans(span_array(rows)), src_o, want, inv, dname(dtype),
                        None if k_scale is None else k_scale.numpy())
        flags = torch.zeros(1, dtype=torch.int32, device=gpu)
        runner.run(rows, si, di, error_flags=flags)
        torch.cuda.synchronize(gpu)
        assert int(flags.item()) == 0
        assert bool(runner._last) == small
        for layer, t in enumerate(dst.caches[0]):
            got = bits(t)
            assert np.array_equal(got, want.caches[0][layer]), (
                f"layer {layer}: {int((got != want.caches[0][layer]).sum())} elements differ")


def test_small_step_bad_rows_are_flagged_and_skipped(gpu):
    """Out-of-range rows in an in-launch step raise their flags and write nothing."""
    runner, src, dst, _ = _runner_case(gpu, torch.bfloat16, "flat", "table", 8, 2, 5)
    before = [bits(t) for t in dst.caches[0]]
    rows = [(290, 0, 0, 0, 20, 5, 0, 0),   # source rows 290..309 of a 300-row store
            (0, 0, 0, 1, 16, 5, 5, 0),     # group 5 of 2
            (0, 0, 0, 2, 4, 5, 0, 0)]      # destination block id 999
    di = np.asarray([3, 4, 999], np.int32)
    flags = torch.zeros(1, dtype=torch.int32, device=gpu)
    runner.run(rows, None, di, error_flags=flags)
    torch.cuda.synchronize(gpu)
    want = _lib.MKV_FLAG_SRC_RANGE | _lib.MKV_FLAG_DST_RANGE | _lib.MKV_FLAG_SPAN
    assert int(flags.item()) == want
    for t, b in zip(dst.caches[0], before):
        got = bits(t)
        # only span 0's first 10 rows (sources 290..299) may have landed, in block 3
        changed = np.argwhere((got != b).any(axis=-1))
        assert all(blk == 3 and off < 10 for blk, _, off in changed)
