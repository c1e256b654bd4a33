"""The reference-side drop-in (``marathon_amd/shift_kernels_hip.py``) called exactly as the
reference's connector calls ``scatter_shifted`` (src/marathon/vllm_shift_connector.py:515):
``scatter_shifted(row, kv, slot, bs, hnd, shift)`` with the reference's own ``RopeShift``
-- six fields, no rotary width -- built by its ``rope_shift`` on the cache's device
(vllm_shift_connector.py:203-207 -> shift_kernels.py:68-84).

Bar: 0 ulp.  Against the reference's Triton kernel arithmetic with those same tables
(``k * cos + k[partner] * sgn``, shift_kernels.py:117-127, restated on the CPU in
oracle/torch_path.py) at every rotary width, and at full rotary also against its torch
path (:141-159), which cannot broadcast a partial-rotary table.  The package's own
``scatter_shifted`` takes the same reference-shaped tables and must write the same bits,
and ``rope_shift(..., tables="reference")`` must reproduce the torch path bit for bit.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import pytest
import torch

from oracle import torch_path
from tests.helpers import bits, inv_freq, randn

pytestmark = pytest.mark.gpu

HEAD = 128


@dataclass(frozen=True)
class ReferenceRopeShift:
    """The reference's RopeShift (shift_kernels.py:50-65): exactly its six fields."""

    delta: int
    cos: torch.Tensor
    sgn: torch.Tensor
    partner: torch.Tensor
    emb_cos: torch.Tensor
    emb_sin: torch.Tensor


def reference_rope_shift(delta, head_size, inv, device) -> ReferenceRopeShift:
    t = torch_path.rope_shift_tables(delta, head_size, inv, device)
    return ReferenceRopeShift(int(delta), t["cos"], t["sgn"], t["partner"], t["emb_cos"],
                              t["emb_sin"])


def _case(seed, n, hnd, dtype, heads=8, bs=16, nblocks=64, start=5):
    g = torch.Generator().manual_seed(seed)
    src = randn((n, heads, 2 * HEAD), dtype, g)
    shape = (nblocks, heads, bs, 2 * HEAD) if hnd else (nblocks, bs, heads, 2 * HEAD)
    kv = randn(shape, dtype, g)
    table = torch.randperm(nblocks, generator=g)[: -(-(n + start) // bs) + 1]
    pos = torch.arange(start, start + n)
    return src, kv, table[pos // bs] * bs + pos % bs


CASES = [(64, -3000), (37, -566), (64, 4), (53, 186), (40, 10000), (16, 2**20 + 3)]


@pytest.mark.parametrize("rotary", [128, 64, 32])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("hnd", [True, False])
def test_dropin_with_reference_tables_is_bit_exact(gpu, rotary, dtype, hnd):
    from marathon_amd import scatter_shifted as package_scatter
    from marathon_amd.shift_kernels_hip import scatter_shifted

    inv = inv_freq(rotary)
    for n, delta in CASES:
        print(f"case drop-in rotary={rotary} {dtype} hnd={hnd} n={n} delta={delta}", flush=True)
        src, kv, slots = _case(rotary + n + abs(delta) % 997, n, hnd, dtype)
        shift = reference_rope_shift(delta, HEAD, inv, gpu)  # built on the GPU, as the connector does
        assert not hasattr(shift, "rotary")
        row, slot = src.to(gpu), slots.to(gpu)
        kv_dropin = kv.to(gpu)
        scatter_shifted(row, kv_dropin, slot, 16, hnd, shift)  # vllm_shift_connector.py:515
        kv_package = kv.to(gpu)
        package_scatter(row, kv_package, slot, 16, hnd, shift)
        torch.cuda.synchronize(gpu)
        got = bits(kv_dropin)

        want = kv.clone()
        torch_path.triton_rows_into_paged(src, want, slots, 16, hnd,
                                          (shift.cos, shift.sgn, shift.partner))
        want = bits(want)
        assert np.array_equal(got, want), (
            f"{int((got != want).sum())} of {want.size} elements differ from the Triton "
            f"kernel's arithmetic with the reference's tables")
        assert np.array_equal(bits(kv_package), got), "package scatter_shifted differs"
        if rotary == HEAD:
            ref = kv.clone()
            torch_path.shift_into_paged(src, ref, slots, 16, hnd,
                                        (shift.emb_cos.cpu(), shift.emb_sin.cpu()))
            assert np.array_equal(got, bits(ref)), "differs from the reference's torch path"
        # dimensions past the rotary width are the source's K bits
        d_rows = got[(slots // 16).numpy(), :, (slots % 16).numpy()] if hnd else \
            got[(slots // 16).numpy(), (slots % 16).numpy()]
        assert np.array_equal(d_rows[..., rotary:HEAD], bits(src)[..., rotary:HEAD])


def test_dropin_plain_scatter_and_empty(gpu):
    """``shift`` of None and delta 0 are plain scatters; n == 0 does nothing
    (shift_kernels.py:185-187)."""
    from marathon_amd.shift_kernels_hip import scatter_shifted

    src, kv, slots = _case(3, 40, True, torch.bfloat16)
    for shift in (None, reference_rope_shift(0, HEAD, inv_freq(64), gpu)):
        kv_dev = kv.to(gpu)
        scatter_shifted(src.to(gpu), kv_dev, slots.to(gpu), 16, True, shift)
        torch.cuda.synchronize(gpu)
        want = kv.clone()
        torch_path.shift_into_paged(src, want, slots, 16, True, None)
        assert np.array_equal(bits(kv_dev), bits(want))
    kv_dev = kv.to(gpu)
    scatter_shifted(src[:0].to(gpu), kv_dev, slots[:0].to(gpu), 16, True,
                    reference_rope_shift(5, HEAD, inv_freq(), gpu))
    torch.cuda.synchronize(gpu)
    assert np.array_equal(bits(kv_dev), bits(kv))
    with pytest.raises(AssertionError):
        scatter_shifted(src.to(gpu)[..., :128], kv_dev, slots.to(gpu), 16, True, None)


@pytest.mark.parametrize("device", ["gpu", "cpu"])
@pytest.mark.parametrize("hnd", [True, False])
def test_rope_shift_reference_tables_through_the_package(gpu, device, hnd):
    """``rope_shift(..., tables="reference")``: the reference's torch fp32 tables built
    on ``device``; the package's ``scatter_shifted`` with them is the reference's torch
    path bit for bit (0 ulp), every element."""
    from marathon_amd import rope_shift, scatter_shifted

    inv = inv_freq()
    where = gpu if device == "gpu" else torch.device("cpu")
    for n, delta in CASES:
        print(f"case rope_shift tables=reference on {device} hnd={hnd} n={n} delta={delta}",
              flush=True)
        src, kv, slots = _case(n + abs(delta) % 991, n, hnd, torch.bfloat16)
        shift = rope_shift(delta, HEAD, inv, where, tables="reference")
        if device == "cpu":  # tables as the CPU builds them, moved to the cache's device
            shift = type(shift)(shift.delta, shift.cos.to(gpu), shift.sgn.to(gpu),
                                shift.partner.to(gpu), shift.emb_cos, shift.emb_sin,
                                shift.inv_freq.to(gpu), shift.rotary)
        kv_dev = kv.to(gpu)
        scatter_shifted(src.to(gpu), kv_dev, slots.to(gpu), 16, hnd, shift)
        torch.cuda.synchronize(gpu)
        ref = kv.clone()
        torch_path.shift_into_paged(src, ref, slots, 16, hnd,
                                    (shift.emb_cos.cpu(), shift.emb_sin.cpu()))
        got, want = bits(kv_dev), bits(ref)
        assert np.array_equal(got, want), f"{int((got != want).sum())} elements differ"
