"""Bit-level numpy restatement of the shift path -- TEST INFRASTRUCTURE ONLY.

Each function cites the reference code it restates.  Cache contents are handled as
raw bit patterns (``uint16`` for bf16/fp16, ``uint32`` for fp32, ``uint8`` for fp8
e4m3fn) so that V can be compared bit for bit and K's rounding is explicit.

Pinned by (see ``tests/test_oracle.py``):

* ``inv_freq``                 -- closed form 1/theta^(2i/R) in float64, and the
  reference test helper's expression (tests/test_shift_kernels.py:28-29).
* ``angles`` / ``cos_sin``     -- float64 closed forms; torch's own fp32 cos/sin
  (``method="torch"``) agree within 1 fp32 ulp.
* ``f32_to_bf16`` / ``f32_to_f16`` -- torch's ``.to(bfloat16/float16)`` casts.
* ``e4m3_decode`` / ``e4m3_encode`` -- the format definition enumerated over all 256
  codes, and torch's ``float8_e4m3fn`` casts for in-range values.
* ``rotate_k``                 -- the reference test's table identity
  (tests/test_shift_kernels.py:32-43), the fresh-RoPE identity
  (tests/test_kvshift.py:48-55), invertibility, composition, norm preservation.
* ``slots``                    -- the reference's known answer
  (tests/test_shift_store.py:24-27) and brute force.
* ``scatter_shifted`` / ``shift_spans`` -- the reference's CPU scatter test geometry
  (tests/test_shift_kernels.py:93-134) against ``rerotate_keys``, its wrong-angle guard
  (:137-155), and the torch op sequence in :mod:`oracle.torch_path`.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

# ------------------------------------------------------------------ element codecs

BITS_DTYPE = {"bf16": np.uint16, "f16": np.uint16, "f32": np.uint32, "fp8": np.uint8}


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> float32 (exact: bf16 is the top half of an fp32)."""
    return (np.asarray(bits, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even; any NaN -> 0x7FC0.

    The rounding of every non-NaN value is torch's ``.to(torch.bfloat16)``, which is
    what ``scatter_shifted_torch`` applies to the rotated K (shift_kernels.py:156).  NaN
    payloads are implementation-defined there (c10's scalar cast gives 0x7FC0, the
    vectorized CPU cast keeps payload bits); the kernels and this oracle canonicalise to
    0x7FC0.
    """
    x = np.asarray(x, np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), r)


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    """float32 -> fp16 bits, round to nearest even (IEEE); any NaN -> 0x7E00."""
    x = np.asarray(x, np.float32)
    with np.errstate(over="ignore"):
        h = x.astype(np.float16).view(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7E00), h)


def f32_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, np.uint32).view(np.float32)


def f32_to_f32_bits(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, np.float32)
    return np.where(np.isnan(x), np.uint32(0x7FC00000), x.view(np.uint32))


def _e4m3_table() -> np.ndarray:
    """All 256 e4m3fn codes as float32, straight from the OCP format definition.

    sign | 4-bit exponent (bias 7) | 3-bit mantissa.  Exponent 0 is subnormal
    (m * 2^-9).  S.1111.111 is NaN.  There is no infinity; the largest value is
    S.1111.110 = 448.
    """
    out = np.empty(256, np.float32)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 7
        if e == 15 and m == 7:
            out[code] = np.nan
        elif e == 0:
            out[code] = s * m * 2.0**-9
        else:
            out[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return out


E4M3_TABLE = _e4m3_table()
E4M3_MAX = 448.0
_E4M3_POS = E4M3_TABLE[:127].astype(np.float64)  # codes 0..126: 0 .. 448, increasing


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    return E4M3_TABLE[np.asarray(codes, np.uint8)]


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn code, round to nearest, ties to the even code; NaN -> 0x7F.

    Magnitudes above 448 saturate to 448 (the callers clamp first, so this never
    fires on the shift path).  Found by nearest-value search over the code table --
    deliberately a different formulation from the kernel's bit arithmetic.
    """
    x = np.asarray(x, np.float32)
    nan = np.isnan(x)
    sign = np.where(np.signbit(x), np.uint8(0x80), np.uint8(0))
    a = np.minimum(np.abs(np.where(nan, 0.0, x)).astype(np.float64), E4M3_MAX)
    hi = np.searchsorted(_E4M3_POS, a, side="left")  # first value >= a
    hi = np.minimum(hi, 126)
    lo = np.maximum(hi - 1, 0)
    d_lo = a - _E4M3_POS[lo]
    d_hi = _E4M3_POS[hi] - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo)
    code = np.where(a == _E4M3_POS[hi], hi, code).astype(np.uint8)
    return np.where(nan, np.uint8(0x7F), code | sign).astype(np.uint8)


# --------------------------------------------------------------- rotation tables


def inv_freq(rotary: int, theta: float) -> np.ndarray:
    """Inverse RoPE frequencies, fp32, the connector's expression.

    ``1 / theta ** (arange(0, rotary, 2, fp32) / rotary)`` evaluated with torch on
    the CPU (src/marathon/vllm_shift_connector.py:194-199; the reference tests build
    the same vector at tests/test_shift_kernels.py:28-29).
    """
    import torch

    return (
        1.0 / (theta ** (torch.arange(0, rotary, 2, dtype=torch.float32) / rotary))
    ).numpy()


def angles(delta: int, inv: np.ndarray) -> np.ndarray:
    """fl32(float(delta) * inv_freq): shift_kernels.py:73, kvshift.py:58."""
    return np.float32(delta) * np.asarray(inv, np.float32)


def cos_sin(delta: int, inv: np.ndarray, method: str = "cr") -> tuple[np.ndarray, np.ndarray]:
    """cos/sin of the fp32 angles, fp32, one entry per frequency.

    ``method="cr"``: the exact cosine/sine of each fp32 angle rounded once to fp32
    (evaluated in float64) -- the values the HIP kernel uses.
    ``method="torch"``: torch's fp32 ``cos``/``sin`` of ``cat(ang, ang)`` on the CPU,
    i.e. the reference's own ``rope_shift(..., "cpu")`` tables (shift_kernels.py:76-84).
    """
    a = angles(delta, inv)
    if method == "cr":
        a64 = a.astype(np.float64)
        return np.cos(a64).astype(np.float32), np.sin(a64).astype(np.float32)
    if method == "torch":
        import torch

        t = torch.from_numpy(a.copy())
        emb = torch.cat((t, t))
        h = a.shape[0]
        return emb.cos().numpy()[:h].copy(), emb.sin().numpy()[:h].copy()
    raise ValueError(method)


def emb_tables(delta: int, inv: np.ndarray, method: str = "cr") -> tuple[np.ndarray, np.ndarray]:
    """``emb_cos``/``emb_sin`` of length rotary: ``cat(x, x)`` (shift_kernels.py:83-84)."""
    c, s = cos_sin(delta, inv, method)
    return np.concatenate((c, c)), np.concatenate((s, s))


def rope_tables(delta: int, head_size: int, inv: np.ndarray, method: str = "cr") -> dict:
    """The five ``RopeShift`` tables (shift_kernels.py:68-84) as numpy arrays."""
    rotary = 2 * int(np.asarray(inv).shape[0])
    assert rotary <= head_size, f"rotary {rotary} > head_size {head_size}"
    half = rotary // 2
    ec, es = emb_tables(delta, inv, method)
    cos = np.ones(head_size, np.float32)
    sgn = np.zeros(head_size, np.float32)
    cos[:rotary] = ec
    sgn[:half] = -es[:half]
    sgn[half:rotary] = es[half:rotary]
    partner = np.arange(head_size, dtype=np.int32)
    partner[:half] += half
    partner[half:rotary] -= half
    return {"cos": cos, "sgn": sgn, "partner": partner, "emb_cos": ec, "emb_sin": es}


# ------------------------------------------------------------------------- rotation


def rotate_f32(kf: np.ndarray, emb_cos: np.ndarray, emb_sin: np.ndarray) -> np.ndarray:
    """``kf * emb_cos + rotate_half(kf) * emb_sin`` in fp32, separate mul, mul, add.

    rotate_half(x) = cat(-x[..., h:], x[..., :h]) (kvshift.py:44-46); the product
    order and the single add follow scatter_shifted_torch (shift_kernels.py:153-156).
    """
    kf = np.asarray(kf, np.float32)
    h = kf.shape[-1] // 2
    rot = np.concatenate((-kf[..., h:], kf[..., :h]), axis=-1)
    # raw-bit inputs hold NaN and Inf on purpose: IEEE results, no warnings
    with np.errstate(invalid="ignore", over="ignore"):
        a = kf * emb_cos
        b = rot * emb_sin
        return a + b


def rerotate_keys(k: np.ndarray, delta: int, inv: np.ndarray, method: str = "cr") -> np.ndarray:
    """kvshift.rerotate_keys (kvshift.py:49-61) for fp32 keys: delta == 0 returns k."""
    if delta == 0:
        return np.asarray(k, np.float32)
    ec, es = emb_tables(delta, inv, method)
    return rotate_f32(k, ec, es)


def rotate_k_bits(
    k_bits: np.ndarray,
    delta: int,
    inv: np.ndarray,
    dtype: str,
    k_scale: float | None = None,
    method: str = "cr",
) -> np.ndarray:
    """Re-rotate K given as cache bit patterns ``[..., head_size]``; returns bits.

    delta == 0 returns K untouched (shift_kernels.py:152; the kernel's ``ROTATE``
    flag, :124, :187).  Dimensions at or above ``rotary`` pass through untouched
    (shift_kernels.py:74-75 gives them cos 1, sgn 0).  bf16/fp16/fp32: upcast, rotate in
    fp32, round to nearest even (shift_kernels.py:153-156).  fp8 e4m3fn (no reference
    -- the kernels' own rule): x = fl32(decode * s); rotate; q = fl32(y / s) clamped to
    +-448 (NaN kept), encoded round-to-nearest-even.
    """
    k_bits = np.asarray(k_bits)
    rotary = 2 * int(np.asarray(inv).shape[0])
    if delta == 0 or rotary == 0:
        return k_bits.copy()
    ec, es = emb_tables(delta, inv, method)
    head = k_bits[..., :rotary]
    if dtype == "bf16":
        y = rotate_f32(bf16_to_f32(head), ec, es)
        out_head = f32_to_bf16(y)
    elif dtype == "f16":
        y = rotate_f32(f16_to_f32(head), ec, es)
        out_head = f32_to_f16(y)
    elif dtype == "f32":
        y = rotate_f32(f32_bits_to_f32(head), ec, es)
        out_head = f32_to_f32_bits(y)
    elif dtype == "fp8":
        s = np.float32(k_scale)
        x = e4m3_decode(head) * s
        y = rotate_f32(x, ec, es)
        with np.errstate(invalid="ignore"):
            q = y / s
            q = np.where(q > E4M3_MAX, np.float32(E4M3_MAX), q)
            q = np.where(q < -E4M3_MAX, np.float32(-E4M3_MAX), q)
        out_head = e4m3_encode(q.astype(np.float32))
    else:
        raise ValueError(dtype)
    out = k_bits.copy()
    out[..., :rotary] = out_head
    return out


# --------------------------------------------------------------- slots and paging


def slots(block_ids, lo: int, hi: int, block_size: int) -> np.ndarray:
    """Flat slots of positions [lo, hi) through a block table (shift_store.py:56-60)."""
    pos = np.arange(lo, hi, dtype=np.int64)
    table = np.asarray(block_ids, dtype=np.int64)
    return table[pos // block_size] * block_size + pos % block_size


def paged_rows(kv: np.ndarray, slot: np.ndarray, block_size: int, layout: str):
    """Index tuple of the rows of ``slot`` in a cache of the given layout.

    ``hnd``: [blocks, heads, bs, 2D] -> kv[blk, :, off];  ``nhd``: [blocks, bs, heads,
    2D] -> kv[blk, off] (shift_kernels.py:157-159); ``flat``: [rows, heads, 2D].
    """
    slot = np.asarray(slot, np.int64)
    if layout == "flat":
        return (slot,)
    blk, off = slot // block_size, slot % block_size
    return (blk, slice(None), off) if layout == "hnd" else (blk, off)


def scatter_shifted(
    src_bits: np.ndarray,
    kv_bits: np.ndarray,
    slot: np.ndarray,
    block_size: int,
    hnd: bool,
    delta: int,
    inv: np.ndarray,
    dtype: str = "bf16",
    k_scale: float | None = None,
    method: str = "cr",
) -> None:
    """scatter_shifted (shift_kernels.py:141-159, :166-210) on bit arrays, in place."""
    n, _, two_d = src_bits.shape
    d = two_d // 2
    assert kv_bits.shape[-1] == two_d, f"src row {two_d} != kv row {kv_bits.shape[-1]}"
    if n == 0:
        return
    k = rotate_k_bits(src_bits[..., :d], delta, inv, dtype, k_scale, method)
    rows = np.concatenate((k, src_bits[..., d:]), axis=-1)
    kv_bits[paged_rows(kv_bits, slot, block_size, "hnd" if hnd else "nhd")] = rows


# ------------------------------------------------------------ batched span tables


@dataclass
class Side:
    """One side of a batched shift, in the oracle's terms.

    caches[group][layer] is a bit array: ``flat`` [rows, heads, 2D] or paged ``hnd`` /
    ``nhd``.  ``mode`` is how a span maps token positions to slots: ``flat``
    (slot = position), ``slots`` (int64 ``index[span_index + i]``) or ``table``
    (``index[span_index + pos // bs] * bs + pos % bs``).
    """

    caches: list
    layout: str
    block_size: int = 1
    mode: str = "flat"
    index: np.ndarray | None = None


@dataclass
class Span:
    src_pos: int
    dst_pos: int
    n_tokens: int
    delta: int
    src_index: int = 0
    dst_index: int = 0
    src_group: int = 0
    dst_group: int = 0


def span_slots(side: Side, pos0: int, index0: int, n: int) -> np.ndarray:
    if side.mode == "flat":
        return np.arange(pos0, pos0 + n, dtype=np.int64)
    if side.mode == "slots":
        return np.asarray(side.index[index0 : index0 + n], np.int64)
    if side.mode == "table":
        pos = np.arange(pos0, pos0 + n, dtype=np.int64)
        tbl = np.asarray(side.index, np.int64)
        return tbl[index0 + pos // side.block_size] * side.block_size + pos % side.block_size
    raise ValueError(side.mode)


def shift_spans(
    spans: list,
    src: Side,
    dst: Side,
    inv: np.ndarray,
    dtype: str = "bf16",
    k_scale=None,
    method: str = "cr",
) -> None:
    """Every span x every layer: the batched load, in place on ``dst.caches``.

    Semantics of one (span, layer) are exactly ``scatter_shifted`` on the rows the
    span's source slots select -- the connector's per-load, per-layer loop
    (vllm_shift_connector.py:505-518) and the prototype's per-segment stitch
    (kvshift.py:265-266) folded into one table.
    """
    layers = len(dst.caches[0])
    for sp in spans:
        if sp.n_tokens <= 0:
            continue
        s_slot = span_slots(src, sp.src_pos, sp.src_index, sp.n_tokens)
        d_slot = span_slots(dst, sp.dst_pos, sp.dst_index, sp.n_tokens)
        for layer in range(layers):
            s_cache = src.caches[sp.src_group][layer]
            d_cache = dst.caches[sp.dst_group][layer]
            rows = s_cache[paged_rows(s_cache, s_slot, src.block_size, src.layout)]
            d = rows.shape[-1] // 2
            scale = None if k_scale is None else float(k_scale[layer])
            k = rotate_k_bits(rows[..., :d], sp.delta, inv, dtype, scale, method)
            out = np.concatenate((k, rows[..., d:]), axis=-1)
            d_cache[paged_rows(d_cache, d_slot, dst.block_size, dst.layout)] = out


# ------------------------------------------------------------ float64 closed forms


def rope_f64(k: np.ndarray, pos: np.ndarray, inv: np.ndarray) -> np.ndarray:
    """Fresh NeoX RoPE in float64: k * cos(p * theta) + rotate_half(k) * sin(p * theta).

    ``k`` is ``[..., seq, head_dim]`` (full rotary), ``pos`` ``[seq]``.
    """
    k = np.asarray(k, np.float64)
    ang = np.asarray(pos, np.float64)[:, None] * np.asarray(inv, np.float64)[None, :]
    emb = np.concatenate((ang, ang), axis=-1)
    h = k.shape[-1] // 2
    rot = np.concatenate((-k[..., h:], k[..., :h]), axis=-1)
    return k * np.cos(emb) + rot * np.sin(emb)


def ulp_distance_bf16(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """Distance in bf16 ulps between two bf16 bit arrays (monotone integer mapping)."""

    def key(b):
        b = np.asarray(b, np.uint16).astype(np.int32)
        return np.where(b & 0x8000, 0x8000 - b, b)  # -0 and +0 both map to 0

    return np.abs(key(a_bits) - key(b_bits))
