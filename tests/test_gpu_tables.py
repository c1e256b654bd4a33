"""The three routines that make a span's rotation tables agree bit for bit, over every
delta in [-131072, 131072] at theta 1e4 and 1e6 (rotary 128):

* the plan pass of the two-launch path (``plan_kernel``: double-precision ``sincos`` on
  the device),
* the small path (``mkv_shift_spans_small``: the same evaluation inside the shift kernel,
  ``lane_tables``),
* the host (``spans.span_tables``, float64 numpy), which the direct path takes.

The tables are read through the kernels' own outputs: an fp32 K row of ones in its first
half and zeros in its second, rotated by delta, comes out as ``RN(1 * c + 0 * sgn) = c``
in the first half and ``RN(0 * c + 1 * s) = s`` in the second -- the span's cos and sin
of every frequency, exactly.  One single-token span per delta, every path writing its own
flat destination.  (shift_kernels.py:73-84 for the tables; the exact values are pinned
against float64 closed forms and torch in tests/test_oracle.py.)

Beyond that range (shifts of up to 2^24 positions), 300,000 seeded deltas per theta
compare the plan pass with the host tables.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from marathon_amd.shift_kernels import inv_freq_for
from marathon_amd.spans import CacheSet, ShiftPlan, SmallShifts, span_array, span_tables
from oracle import kvshift_oracle as orc

pytestmark = pytest.mark.gpu

D, HEADS, LIM = 128, 2, 131072


def _rows(deltas: np.ndarray, first: int) -> list:
    return [(0, first + i, 0, 0, 1, int(dl), 0, 0) for i, dl in enumerate(deltas)]


@pytest.mark.parametrize("theta", [1e4, 1e6])
def test_plan_small_and_host_tables_agree_for_every_delta(gpu, theta):
    inv = inv_freq_for(D, theta)
    deltas = np.arange(-LIM, LIM + 1, dtype=np.int64)
    deltas = deltas[deltas != 0]  # delta 0 copies K: no table
    n = deltas.size
    src = torch.zeros(1, HEADS, 2 * D, dtype=torch.float32, device=gpu)
    src[0, :, : D // 2] = 1.0
    src_cs = CacheSet([src], "flat")
    dsts = {name: torch.zeros(n, HEADS, 2 * D, dtype=torch.float32, device=gpu)
            for name in ("two_launch", "small", "direct")}

    print(f"case tables theta={theta}: two-launch, {n} spans", flush=True)
    plan = ShiftPlan(span_array(_rows(deltas, 0)), src_cs, CacheSet([dsts["two_launch"]], "flat"),
                     inv_freq=inv, src_mode="flat", dst_mode="flat", direct=False)
    assert not plan.direct
    plan.launch()

    for name, per in (("small", 8), ("direct", 63)):
        print(f"case tables theta={theta}: {name}, {per} spans per step", flush=True)
        runner = SmallShifts(src_cs, CacheSet([dsts[name]], "flat"), inv_freq=inv,
                             src_mode="flat", dst_mode="flat")
        for lo in range(0, n, per):
            runner.run(_rows(deltas[lo:lo + per], lo), None, None)
    torch.cuda.synchronize(gpu)

    host = span_tables(deltas, inv, D)  # [n, 2, D]: cos, signed sin
    want = np.concatenate((host[:, 0, : D // 2], host[:, 1, D // 2:]), axis=1).view(np.uint32)
    c, s = orc.cos_sin(int(deltas[0]), inv.numpy())
    assert np.array_equal(want[0], np.concatenate((c, s)).view(np.uint32))
    for name, t in dsts.items():
        got = t[:, :, :D].cpu().numpy()
        assert np.array_equal(got[:, 0], got[:, 1]), name  # both heads
        got = got[:, 0].view(np.uint32)
        bad = np.nonzero((got != want).any(axis=1))[0]
        print(f"  {name}: {bad.size} of {n} deltas differ from the host tables", flush=True)
        assert bad.size == 0, (f"{name}: deltas {deltas[bad[:10]].tolist()} differ from the "
                               "host tables")


@pytest.mark.parametrize("theta", [1e4, 1e6])
def test_plan_and_host_tables_agree_for_far_deltas(gpu, theta):
    inv = inv_freq_for(D, theta)
    rng = np.random.default_rng(int(theta))
    mag = rng.integers(LIM + 1, 2 ** 24 + 1, size=300000)
    deltas = mag * rng.choice(np.array([-1, 1]), size=mag.size)
    n = deltas.size
    src = torch.zeros(1, HEADS, 2 * D, dtype=torch.float32, device=gpu)
    src[0, :, : D // 2] = 1.0
    dst = torch.zeros(n, HEADS, 2 * D, dtype=torch.float32, device=gpu)
    print(f"case far tables theta={theta}: two-launch, {n} spans", flush=True)
    plan = ShiftPlan(span_array(_rows(deltas, 0)), CacheSet([src], "flat"), CacheSet([dst], "flat"),
                     inv_freq=inv, src_mode="flat", dst_mode="flat", direct=False)
    plan.launch()
    torch.cuda.synchronize(gpu)
    host = span_tables(deltas, inv, D)
    want = np.concatenate((host[:, 0, : D // 2], host[:, 1, D // 2:]), axis=1).view(np.uint32)
    got = dst[:, :, :D].cpu().numpy()
    assert np.array_equal(got[:, 0], got[:, 1])
    got = got[:, 0].view(np.uint32)
    bad = np.nonzero((got != want).any(axis=1))[0]
    print(f"  {bad.size} of {n} deltas differ from the host tables", flush=True)
    assert bad.size == 0, deltas[bad[:10]].tolist()
