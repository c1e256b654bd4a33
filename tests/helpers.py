"""Helpers shared by the tests: bit views, seeded inputs, oracle bridges."""

from __future__ import annotations

import numpy as np
import torch

from oracle import kvshift_oracle as orc

TORCH_BITS = {
    torch.bfloat16: (torch.int16, np.uint16, "bf16"),
    torch.float16: (torch.int16, np.uint16, "f16"),
    torch.float32: (torch.int32, np.uint32, "f32"),
    torch.float8_e4m3fn: (torch.uint8, np.uint8, "fp8"),
}


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bit patterns of a tensor (copied to the CPU)."""
    iv, nv, _ = TORCH_BITS[t.dtype]
    return t.detach().cpu().contiguous().view(iv).numpy().view(nv).copy()


def dname(dtype: torch.dtype) -> str:
    return TORCH_BITS[dtype][2]


def inv_freq(rotary: int = 128, theta: float = 1e6) -> torch.Tensor:
    """The reference tests' inverse frequencies (tests/test_shift_kernels.py:28-29)."""
    return 1.0 / (theta ** (torch.arange(0, rotary, 2, dtype=torch.float32) / rotary))


def randn(shape, dtype, gen, scale: float = 1.0) -> torch.Tensor:
    if dtype == torch.float8_e4m3fn:
        x = torch.randn(shape, dtype=torch.float32, generator=gen) / scale
        return x.clamp(-448, 448).to(torch.float8_e4m3fn)
    return torch.randn(shape, dtype=torch.float32, generator=gen).to(dtype)


def oracle_side(cs, mode: str, index) -> orc.Side:
    """An oracle Side holding CPU bit copies of a marathon_amd CacheSet (split K and V
    planes as fused rows, K then V: the oracle's row format)."""
    caches = [[bits(cs.fused(g, layer)) for layer in range(cs.layers)]
              for g in range(cs.groups)]
    idx = None if index is None else index.detach().cpu().numpy()
    return orc.Side(caches, cs.layout, cs.block_size, mode, idx)


def oracle_spans(spans: np.ndarray) -> list:
    return [
        orc.Span(int(r["src_pos"]), int(r["dst_pos"]), int(r["n_tokens"]), int(r["delta"]),
                 int(r["src_index"]), int(r["dst_index"]), int(r["src_group"]),
                 int(r["dst_group"]))
        for r in spans
    ]


def ulp_bf16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return orc.ulp_distance_bf16(a, b)


def within_table_rounding(got: np.ndarray, ref: np.ndarray, src_k: np.ndarray,
                          rotary: int) -> np.ndarray:
    """Per element: ``got`` (correctly rounded cos/sin tables) and ``ref`` (the reference's
    torch fp32 tables, each within 1 fp32 ulp of them) differ by at most 1 bf16 ulp plus
    what the tables' rounding can move ``k*c + kp*s`` before the cast: 2 * (|k| + |kp|) *
    2^-24.  Where the two products nearly cancel, that term exceeds 1 ulp of the small
    result; everywhere else the bound is 1 ulp.  All arrays are bf16 bits ``[..., D]``."""
    g = orc.bf16_to_f32(got[..., :rotary]).astype(np.float64)
    r = orc.bf16_to_f32(ref[..., :rotary]).astype(np.float64)
    k = orc.bf16_to_f32(src_k[..., :rotary]).astype(np.float64)
    kp = np.roll(k, rotary // 2, axis=-1)
    big = np.maximum(np.abs(g), np.abs(r)).astype(np.float32)
    ulp = np.spacing(big).astype(np.float64) * 65536.0  # bf16 keeps 8 of fp32's 24 bits
    return np.abs(g - r) <= ulp + 2.0 * (np.abs(k) + np.abs(kp)) * 2.0**-24
