"""The C ABI from a C program: no Python and no torch in the process that shifts.

tests/c/shift_spans_example.c (built by ``build()`` with gcc against
include/marathon_kvshift.h and the HIP runtime) allocates device buffers, runs a
two-layer, two-span batched shift (flat store -> HND paged cache through a slot array)
with ``mkv_shift_spans`` and checks the ABI's error path.  It dumps every input and
output; here the output is compared with the oracle byte for byte.
"""

from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

from marathon_amd import _lib
from oracle import kvshift_oracle as orc

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "shift_spans_example")


def test_c_program_shift_matches_the_oracle(gpu, tmp_path):
    del gpu  # the C program opens the device itself
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} is not built (run __graft_entry__.build())")
    out = tmp_path / "shift.bin"
    print("case C program through the C ABI", flush=True)
    res = subprocess.run([EXE, str(out)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    raw = out.read_bytes()
    head = np.frombuffer(raw, np.int32, 12)
    layers, heads, d, bs, hist, blocks, n_spans, n_slots, rc, flags, abi, err_ok = map(int, head)
    assert (rc, flags, err_ok) == (_lib.MKV_OK, 0, 1)
    assert abi == _lib.MKV_ABI_VERSION
    at = 48

    def take(dtype, count):
        nonlocal at
        a = np.frombuffer(raw, dtype, count, at)
        at += a.nbytes
        return a

    inv = take(np.float32, d // 2)
    spans = take(_lib.SPAN_DTYPE, n_spans)
    slots = take(np.int64, n_slots)
    src = take(np.uint16, layers * hist * heads * 2 * d).reshape(layers, hist, heads, 2 * d)
    dshape = (layers, blocks, heads, bs, 2 * d)
    before = take(np.uint16, int(np.prod(dshape))).reshape(dshape)
    after = take(np.uint16, int(np.prod(dshape))).reshape(dshape)
    assert at == len(raw)

    src_side = orc.Side([[src[layer].copy() for layer in range(layers)]], "flat", 1, "flat", None)
    dst_side = orc.Side([[before[layer].copy() for layer in range(layers)]], "hnd", bs, "slots",
                        slots.copy())
    rows = [orc.Span(int(r["src_pos"]), int(r["dst_pos"]), int(r["n_tokens"]), int(r["delta"]),
                     int(r["src_index"]), int(r["dst_index"]), int(r["src_group"]),
                     int(r["dst_group"])) for r in spans]
    orc.shift_spans(rows, src_side, dst_side, inv, "bf16")
    for layer in range(layers):
        assert np.array_equal(after[layer], dst_side.caches[0][layer]), f"layer {layer}"
    assert not np.array_equal(after, before)
