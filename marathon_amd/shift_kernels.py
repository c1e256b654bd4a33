"""Fused re-rotate-and-scatter on MI355X: the host API of src/marathon/shift_kernels.py.

Same names, argument meanings and error behaviour as the reference module:

* :class:`RopeShift` / :func:`rope_shift` -- per-delta rotation tables
  (shift_kernels.py:50-84), built once per delta on the host and kept on the device;
  the single-span kernel reads ``cos`` and ``sgn`` as the reference's Triton kernel
  does (shift_kernels.py:96, :127).
* :func:`scatter_shifted` -- write ``src`` ``[n, heads, 2*head_size]`` into the paged
  ``kv`` at ``slots``, K re-rotated by delta, V copied bit for bit
  (shift_kernels.py:166-210).  One call is one HIP launch on the current stream.
* :func:`use_hip` -- the analogue of ``use_triton`` (shift_kernels.py:162-163).
* :func:`warmup` -- kept for the connector's call (vllm_shift_connector.py:404-405);
  the kernels are compiled ahead of time, so it only loads the library.

Divergence, on purpose: there is no torch fallback.  The reference's
``scatter_shifted`` falls back to ``scatter_shifted_torch`` off-GPU
(shift_kernels.py:180-181); here a tensor that is not on a HIP device raises, so a
measurement or a parity check can never run anything but the HIP kernel.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib

_DTYPES = {
    torch.bfloat16: _lib.MKV_BF16,
    torch.float16: _lib.MKV_F16,
    torch.float32: _lib.MKV_F32,
    torch.float8_e4m3fn: _lib.MKV_FP8_E4M3,
}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise TypeError(f"unsupported KV cache dtype {dtype}") from None


@dataclass(frozen=True)
class RopeShift:
    """Rotation for one delta on one device (shift_kernels.py:50-65).

    ``cos``/``sgn`` fp32 [head_size], ``partner`` int32 [head_size], ``emb_cos`` /
    ``emb_sin`` fp32 [rotary]: the same tables the reference builds.  ``inv_freq`` is the
    fp32 [rotary / 2] vector the kernel reads; ``rotary`` is 2 * len(inv_freq).
    """

    delta: int
    cos: torch.Tensor
    sgn: torch.Tensor
    partner: torch.Tensor
    emb_cos: torch.Tensor
    emb_sin: torch.Tensor
    inv_freq: torch.Tensor
    rotary: int


def inv_freq_for(head_dim: int, rope_theta: float, partial_rotary_factor: float = 1.0) -> torch.Tensor:
    """The connector's inverse frequencies (vllm_shift_connector.py:194-199), fp32, CPU."""
    rotary = int(head_dim * partial_rotary_factor)
    return 1.0 / (float(rope_theta) ** (torch.arange(0, rotary, 2, dtype=torch.float32) / rotary))


def shift_rotary(shift) -> int:
    """Rotated dimensions of a ``RopeShift``: the length of its ``emb_cos`` table, which
    ``rope_shift`` builds from the ``rotary / 2`` angles (shift_kernels.py:73, :83-84).
    Works for this package's ``RopeShift`` and for the reference's, which has no
    ``rotary`` field; a ``rotary`` field that disagrees with the table is refused."""
    if shift is None:
        return 0
    rotary = int(shift.emb_cos.numel())
    declared = getattr(shift, "rotary", None)
    if declared is not None and int(declared) != rotary:
        raise ValueError(f"RopeShift.rotary {declared} != len(emb_cos) {rotary}")
    return rotary


TABLES = ("exact", "reference")


def rope_shift(delta: int, head_size: int, inv_freq: torch.Tensor, device,
               tables: str = "exact") -> RopeShift:
    """Tables that move RoPE'd keys ``delta`` positions (shift_kernels.py:68-84).

    ``tables="exact"`` (the default): cos/sin of the fp32 angles ``fl32(delta *
    inv_freq)`` evaluated in double precision and rounded once to fp32, by the library's
    host routine (``mkv_rope_tables``) -- the routine the kernels run on the device, so
    the same bits.  ``tables="reference"``: the reference's own tables, built
    as its ``rope_shift`` builds them, with torch's fp32 ``cos``/``sin`` on ``device``;
    through :func:`scatter_shifted` these reproduce the reference's torch path
    (shift_kernels.py:141-159) bit for bit.
    """
    if tables not in TABLES:
        raise ValueError(f"tables must be one of {TABLES}, not {tables!r}")
    rotary = 2 * int(inv_freq.numel())
    assert rotary <= head_size, f"rotary {rotary} > head_size {head_size}"
    half = rotary // 2
    if tables == "reference":
        return _reference_tables(delta, head_size, inv_freq, device, rotary)
    inv = inv_freq.detach().to(device="cpu", dtype=torch.float32).numpy()
    # the library's host routine: the bits the plan pass and the small path compute
    t = _lib.rope_tables([int(delta)], inv, rotary)[0]  # [2, rotary]: cos, signed sine
    c = t[0, :half].copy()
    s = t[1, half:].copy()
    emb_c = np.concatenate((c, c))
    emb_s = np.concatenate((s, s))
    cos = np.ones(head_size, np.float32)
    sgn = np.zeros(head_size, np.float32)
    cos[:rotary] = emb_c
    sgn[:half] = -emb_s[:half]
    sgn[half:rotary] = emb_s[half:rotary]
    partner = np.arange(head_size, dtype=np.int32)
    partner[:half] += half
    partner[half:rotary] -= half

    def dev(a):
        return torch.from_numpy(a).to(device)

    return RopeShift(
        int(delta),
        dev(cos),
        dev(sgn),
        dev(partner),
        dev(emb_c),
        dev(emb_s),
        dev(inv.copy()),
        rotary,
    )


def _reference_tables(delta: int, head_size: int, inv_freq: torch.Tensor, device,
                      rotary: int) -> RopeShift:
    """The reference's table construction (shift_kernels.py:72-84), in torch fp32 on
    ``device``: one fp32 multiply per angle, then torch's fp32 ``cos``/``sin`` of
    ``cat(ang, ang)``."""
    half = rotary // 2
    inv = inv_freq.detach().to(device=device, dtype=torch.float32)
    ang = float(delta) * inv
    emb = torch.cat((ang, ang))
    emb_cos, emb_sin = emb.cos(), emb.sin()
    cos = torch.ones(head_size, dtype=torch.float32, device=device)
    sgn = torch.zeros(head_size, dtype=torch.float32, device=device)
    cos[:rotary] = emb_cos
    sgn[:half] = -emb_sin[:half]
    sgn[half:rotary] = emb_sin[half:rotary]
    partner = torch.arange(head_size, dtype=torch.int32, device=device)
    partner[:half] += half
    partner[half:rotary] -= half
    return RopeShift(int(delta), cos, sgn, partner, emb_cos, emb_sin, inv.contiguous(), rotary)


def use_hip(kv: torch.Tensor) -> bool:
    """True when ``kv`` lives on a HIP device, i.e. when :func:`scatter_shifted` runs."""
    return bool(kv.is_cuda)


def paged_strides(kv: torch.Tensor, hnd: bool) -> tuple[int, int, int]:
    """(block, head, in-block offset) element strides of a fused 4-D cache.

    HND ``[blocks, heads, bs, 2D]`` or NHD ``[blocks, bs, heads, 2D]``
    (shift_kernels.py:135-138).
    """
    s = kv.stride()
    return (s[0], s[1], s[2]) if hnd else (s[0], s[2], s[1])


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream(device: torch.device) -> int:
    """The hipStream_t of ``device``'s current stream, as an integer.  Read through
    torch's raw-stream accessor where this torch has it (0.06 us instead of the 1.9 us
    of building a ``torch.cuda.Stream`` object: a per-layer call pays this 40 times)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return int(_raw_stream(idx))
    return int(torch.cuda.current_stream(device).cuda_stream)


_current_device = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# fp32 K scales given as Python numbers, kept on their device: the reference's
# per-layer loop passes the same 40 scales on every load, so each is uploaded once
_SCALES: dict[tuple[int, int], torch.Tensor] = {}
# the K scales the fp8 requantisation divides by correctly rounded (include/marathon_kvshift.h)
_SCALE_MIN, _SCALE_MAX = np.float32(2.0 ** -90), np.float32(2.0 ** 100)
_SCALES_MAX = 4096


def _scale_tensor(k_scale, device) -> torch.Tensor:
    if isinstance(k_scale, torch.Tensor):
        t = k_scale.detach().reshape(-1)[:1]
        if t.device != device or t.dtype != torch.float32:
            t = t.to(device=device, dtype=torch.float32)
        return t.contiguous()
    value = np.float32(float(k_scale))
    if not _SCALE_MIN <= value <= _SCALE_MAX:
        raise ValueError(f"k_scale {float(k_scale)!r} outside [2^-90, 2^100]")
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (int(idx), int(value.view(np.uint32)))  # by bits
    t = _SCALES.get(key)
    if t is None:
        if len(_SCALES) >= _SCALES_MAX:
            _SCALES.clear()
        t = torch.tensor([value], dtype=torch.float32, device=torch.device("cuda", idx))
        _SCALES[key] = t
    return t


def scatter_shifted(
    src: torch.Tensor,
    kv: torch.Tensor,
    slots: torch.Tensor,
    block_size: int,
    hnd: bool,
    shift: RopeShift | None,
    *,
    k_scale=None,
    error_flags: torch.Tensor | None = None,
) -> None:
    """Write ``src`` (``[n, heads, 2*head_size]``) into ``kv``'s slots, K rotated by delta.

    ``slots`` are flat destination slots (block ``slot // block_size``, offset
    ``slot % block_size``); ``hnd`` selects the paged layout; ``shift`` of ``None`` (or
    delta 0) is a plain scatter (shift_kernels.py:166-179).  Asynchronous on the
    current stream.  ``k_scale`` (fp8 caches only) is the layer's K scale;
    ``error_flags`` an optional int32 device tensor that collects out-of-range bits.
    """
    if not kv.is_cuda:
        raise RuntimeError(
            "scatter_shifted: kv is not on a HIP device; marathon_amd has no CPU path"
        )
    n, heads, two_d = src.shape
    d = two_d // 2
    assert kv.shape[-1] == two_d, f"src row {two_d} != kv row {kv.shape[-1]}"
    if n == 0:
        return
    if src.dtype != kv.dtype:
        raise TypeError(f"src dtype {src.dtype} != kv dtype {kv.dtype}")
    # device indices as ints: a per-layer call runs these checks 40 times per shift
    dev = kv.get_device()
    if src.get_device() != dev:
        raise ValueError(f"src on {src.device}, kv on {kv.device}")
    ss, ks = src.stride(), kv.stride()
    if ss[2] != 1 or ks[3] != 1:
        raise ValueError("src and kv rows must be contiguous in the last dimension")
    code = dtype_code(kv.dtype)
    if slots.get_device() != dev or slots.dtype != torch.int64 or not slots.is_contiguous():
        slots = slots.to(device=kv.device, dtype=torch.int64, non_blocking=True).contiguous()
    if slots.numel() != n:
        raise ValueError(f"{slots.numel()} slots for {n} tokens")
    # the rotary width is the length of emb_cos (rope_shift builds it from the rotary/2
    # angles, shift_kernels.py:73, :83-84): host metadata, so a reference-built RopeShift
    # (no ``rotary`` field) of a partial-rotary model needs nothing more from the caller
    rotary = shift_rotary(shift)
    rotate = shift is not None and shift.delta != 0 and rotary > 0
    cos = sgn = scale = None
    if rotate:
        cos, sgn = shift.cos, shift.sgn
        if cos.get_device() != dev:
            cos, sgn = cos.to(kv.device), sgn.to(kv.device)
        if cos.numel() != d or sgn.numel() != d:
            raise ValueError(f"rotation tables of {cos.numel()} for head_size {d}")
        if code == _lib.MKV_FP8_E4M3:
            if k_scale is None:
                raise ValueError("fp8 KV cache needs k_scale")
            scale = _scale_tensor(k_scale, kv.device)
    blk_s, head_s, off_s = (ks[0], ks[1], ks[2]) if hnd else (ks[0], ks[2], ks[1])
    stream = _raw_stream(dev) if _raw_stream is not None else current_stream(kv.device)
    args = (
        src.data_ptr(),
        ss[0],
        ss[1],
        kv.data_ptr(),
        blk_s,
        head_s,
        off_s,
        kv.shape[0],
        slots.data_ptr(),
        n,
        heads,
        d,
        int(block_size),
        code,
        None if cos is None else cos.data_ptr(),
        None if sgn is None else sgn.data_ptr(),
        rotary if rotate else 0,
        None if scale is None else scale.data_ptr(),
        None if error_flags is None else error_flags.data_ptr(),
        ctypes.c_void_p(int(stream)),
    )
    fn = _lib.lib().mkv_scatter_shifted
    if dev == _current_device():
        rc = fn(*args)
    else:
        with torch.cuda.device(dev):  # the launch goes to the current device
            rc = fn(*args)
    _lib.check(rc)


def warmup(kv: torch.Tensor, block_size: int, hnd: bool) -> None:
    """Load the library before the first real load (shift_kernels.py:213-238).

    The reference pre-compiles its Triton specialisations here; HIP kernels are
    compiled ahead of time, so there is nothing to compile -- only the library load.
    """
    if use_hip(kv):
        _lib.lib()
