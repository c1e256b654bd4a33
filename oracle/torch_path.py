"""The reference's torch shift path, run on the CPU -- TEST INFRASTRUCTURE ONLY.

Restates the op sequence of ``scatter_shifted_torch`` (src/marathon/shift_kernels.py:
141-159) with the tables of ``rope_shift`` (:68-84): slice K, upcast to fp32, build
rotate_half with a ``cat``, ``k * emb_cos + rot * emb_sin`` as separate fp32 ops, cast
back to the cache dtype, ``cat`` K and V, and scatter with advanced indexing.  It is
kept op-for-op alike on purpose: it is the timed CPU baseline ("the reference's torch
CPU shift path") and the "reference rotation" the kernels are held to within 1 ulp.
"""

from __future__ import annotations

import torch


def rope_emb_tables(delta: int, inv_freq: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``emb_cos``/``emb_sin`` as rope_shift builds them on the CPU (shift_kernels.py:73, 83-84)."""
    ang = float(delta) * inv_freq.to(dtype=torch.float32)
    emb = torch.cat((ang, ang))
    return emb.cos(), emb.sin()


def rope_shift_tables(delta: int, head_size: int, inv_freq: torch.Tensor, device) -> dict:
    """The reference's ``rope_shift`` tables built with torch on ``device``
    (shift_kernels.py:68-84): ``cos``/``sgn`` [head_size] as its Triton kernel reads them
    and ``emb_cos``/``emb_sin`` [rotary] as its torch path reads them."""
    rotary = 2 * int(inv_freq.numel())
    assert rotary <= head_size, f"rotary {rotary} > head_size {head_size}"
    half = rotary // 2
    ang = float(delta) * inv_freq.to(device=device, dtype=torch.float32)
    emb = torch.cat((ang, ang))
    cos = torch.ones(head_size, dtype=torch.float32, device=device)
    cos[:rotary] = emb.cos()
    sin = emb.sin()
    sgn = torch.zeros(head_size, dtype=torch.float32, device=device)
    sgn[:half] = -sin[:half]
    sgn[half:rotary] = sin[half:rotary]
    partner = torch.arange(head_size, dtype=torch.int32, device=device)
    partner[:half] += half
    partner[half:rotary] -= half
    return {"cos": cos, "sgn": sgn, "partner": partner, "emb_cos": emb.cos(), "emb_sin": sin}


def triton_rows_into_paged(
    rows: torch.Tensor,
    cache: torch.Tensor,
    slot: torch.Tensor,
    block_size: int,
    hnd: bool,
    tables: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None,
) -> None:
    """One layer as the reference's Triton kernel computes it (shift_kernels.py:117-132),
    on the CPU: ``k * cos + k[partner] * sgn`` in fp32 with the ``[head_size]`` tables
    of ``rope_shift`` (cos, sgn, partner), as separate multiplies and one add, cast back
    to the cache dtype; V copied.  This is the reference's only path that handles
    partial rotary: its torch path multiplies the ``[head_size]`` keys by the
    ``[rotary]`` ``emb_cos`` and cannot broadcast them when rotary < head_size
    (:153-156).  For finite keys, the dimensions past ``rotary`` come out as
    ``k * 1 + k * 0 = k``.  ``tables`` of ``None`` is a delta-0 plain scatter."""
    d = rows.shape[-1] // 2
    keys = rows[..., :d]
    if tables is not None:
        cos, sgn, partner = (t.cpu() for t in tables)
        kf = keys.to(torch.float32)
        kp = kf[..., partner.long()]
        keys = (kf * cos + kp * sgn).to(cache.dtype)
    block, offset = slot // block_size, slot % block_size
    where = (block, slice(None), offset) if hnd else (block, offset)
    cache[where] = torch.cat((keys, rows[..., d:]), dim=-1)


def shift_into_paged(
    rows: torch.Tensor,
    cache: torch.Tensor,
    slot: torch.Tensor,
    block_size: int,
    hnd: bool,
    emb: tuple[torch.Tensor, torch.Tensor] | None,
) -> None:
    """One layer of the torch path: rotate K of ``rows`` [n, heads, 2D] and scatter.

    ``emb`` is ``(emb_cos, emb_sin)`` or ``None`` for a delta-0 plain scatter.
    """
    d = rows.shape[-1] // 2
    keys = rows[..., :d]
    if emb is not None:
        kf = keys.to(torch.float32)
        h = kf.shape[-1] // 2
        rotated_half = torch.cat((-kf[..., h:], kf[..., :h]), dim=-1)
        keys = (kf * emb[0] + rotated_half * emb[1]).to(cache.dtype)
    block, offset = slot // block_size, slot % block_size
    where = (block, slice(None), offset) if hnd else (block, offset)
    cache[where] = torch.cat((keys, rows[..., d:]), dim=-1)
