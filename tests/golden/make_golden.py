"""Write the golden fixtures under tests/golden/ (run from the repo root).

Each fixture is one single-span shift at the reference kernel test's geometry
(tests/test_shift_kernels.py:46-78: 8 KV heads, head_size 128, block 16, a scattered
block table, a run starting at position 3) with seeded inputs, and two expected
outputs computed in this container:

* ``want_cr``    -- the oracle with correctly rounded cos/sin (what the kernels compute,
                    bit for bit);
* ``want_torch`` -- the reference's torch op sequence (oracle/torch_path.py) with
                    torch's CPU cos/sin tables, for bf16 full-rotary cases; the kernels
                    must land within 1 bf16 ulp of it.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import kvshift_oracle as orc  # noqa: E402
from oracle import torch_path  # noqa: E402

CASES = [
    # name, dtype, hnd, n, delta, rotary, scale, seed
    ("bf16_hnd_ragged_neg566", "bf16", True, 21, -566, 128, None, 1),
    ("bf16_nhd_full_10000", "bf16", False, 29, 10000, 128, None, 2),
    ("bf16_hnd_partial64_186", "bf16", True, 21, 186, 64, None, 3),
    ("fp8_hnd_1999", "fp8", True, 21, 1999, 128, 0.037, 4),
    ("fp16_nhd_neg1133", "f16", False, 21, -1133, 128, None, 5),
]


def make(name, dtype, hnd, n, delta, rotary, scale, seed):
    g = torch.Generator().manual_seed(seed)
    heads, d, bs, nblocks, start = 8, 128, 16, 2, 3
    if dtype == "fp8":
        src = (torch.randn(n, heads, 2 * d, generator=g) / scale).clamp(-448, 448)
        src = src.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    elif dtype == "f16":
        src = torch.randn(n, heads, 2 * d, generator=g).to(torch.float16).view(torch.int16)
        src = src.numpy().view(np.uint16)
    else:
        src = torch.randn(n, heads, 2 * d, generator=g).to(torch.bfloat16).view(torch.int16)
        src = src.numpy().view(np.uint16)
    shape = (nblocks, heads, bs, 2 * d) if hnd else (nblocks, bs, heads, 2 * d)
    kv = np.zeros(shape, src.dtype)
    table = torch.randperm(nblocks, generator=g).numpy()
    pos = np.arange(start, start + n)
    slots = table[pos // bs] * bs + pos % bs
    inv = orc.inv_freq(rotary, 1e6)
    want = kv.copy()
    orc.scatter_shifted(src, want, slots, bs, hnd, delta, inv, dtype,
                        k_scale=None if scale is None else np.float32(scale))
    out = dict(src=src, kv=kv, slots=slots.astype(np.int64), inv_freq=inv,
               block_size=np.int64(bs), hnd=np.bool_(hnd), delta=np.int64(delta),
               dtype=np.array(dtype), scale=np.float32(scale or 0.0), want_cr=want)
    if dtype == "bf16" and rotary == d:
        ref = torch.zeros(shape, dtype=torch.bfloat16)
        rows = torch.from_numpy(src.view(np.int16)).view(torch.bfloat16)
        emb = torch_path.rope_emb_tables(delta, torch.from_numpy(inv))
        torch_path.shift_into_paged(rows, ref, torch.from_numpy(slots), bs, hnd, emb)
        out["want_torch"] = ref.view(torch.int16).numpy().view(np.uint16)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)


if __name__ == "__main__":
    for case in CASES:
        make(*case)
        print("wrote", case[0])
