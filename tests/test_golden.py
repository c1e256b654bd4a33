"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py): the
oracle reproduces them on the CPU, and the HIP kernel reproduces them on the GPU."""

from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

from oracle import kvshift_oracle as orc

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = sorted(glob.glob(os.path.join(HERE, "*.npz")))
TORCH_OF = {"bf16": torch.bfloat16, "f16": torch.float16, "fp8": torch.float8_e4m3fn}
INT_OF = {"bf16": torch.int16, "f16": torch.int16, "fp8": torch.uint8}


def _load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_fixtures_exist():
    assert len(FIXTURES) >= 5


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p))
def test_oracle_reproduces_the_fixture(path):
    f = _load(path)
    dtype = str(f["dtype"])
    got = f["kv"].copy()
    scale = None if dtype != "fp8" else np.float32(f["scale"])
    orc.scatter_shifted(f["src"], got, f["slots"], int(f["block_size"]), bool(f["hnd"]),
                        int(f["delta"]), f["inv_freq"], dtype, k_scale=scale)
    assert np.array_equal(got, f["want_cr"])
    if "want_torch" in f:
        assert int(orc.ulp_distance_bf16(f["want_cr"], f["want_torch"]).max()) <= 1


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p))
def test_kernel_reproduces_the_fixture(gpu, path):
    from marathon_amd import rope_shift, scatter_shifted

    f = _load(path)
    dtype = str(f["dtype"])
    print(f"case golden {os.path.basename(path)}", flush=True)
    tdt, idt = TORCH_OF[dtype], INT_OF[dtype]
    src = torch.from_numpy(f["src"].view(np.int16) if idt == torch.int16 else f["src"])
    kv = torch.from_numpy(f["kv"].view(np.int16) if idt == torch.int16 else f["kv"])
    src = src.view(tdt).to(gpu)
    kv = kv.view(tdt).to(gpu)
    shift = rope_shift(int(f["delta"]), src.shape[-1] // 2, torch.from_numpy(f["inv_freq"]), gpu)
    kw = {"k_scale": float(f["scale"])} if dtype == "fp8" else {}
    scatter_shifted(src, kv, torch.from_numpy(f["slots"]).to(gpu), int(f["block_size"]),
                    bool(f["hnd"]), shift, **kw)
    torch.cuda.synchronize(gpu)
    got = kv.cpu().view(idt).numpy()
    got = got.view(np.uint16) if idt == torch.int16 else got
    assert np.array_equal(got, f["want_cr"])
    if "want_torch" in f:
        assert int(orc.ulp_distance_bf16(got, f["want_torch"]).max()) <= 1
