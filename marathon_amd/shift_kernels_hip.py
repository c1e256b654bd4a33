"""The reference-side drop-in: ``scatter_shifted`` bound to ``mkv_scatter_shifted``.

This file is what a maintainer adds to the reference as ``src/marathon/shift_kernels_hip.py``
and imports in place of ``shift_kernels.scatter_shifted`` at the connector's call site
(src/marathon/vllm_shift_connector.py:515).  It depends on nothing but ctypes, torch and
the library, so it runs unchanged inside the reference's package or from this one.

* ``scatter_shifted(src, kv, slots, block_size, hnd, shift)`` has the reference's
  signature and meaning (src/marathon/shift_kernels.py:166-210): the same row-size
  assertion, ``n == 0`` a no-op, ``shift`` of ``None`` or delta 0 a plain scatter,
  asynchronous on the current stream.
* ``shift`` is the reference's own ``RopeShift`` (shift_kernels.py:50-65: ``delta``,
  ``cos``, ``sgn``, ``partner``, ``emb_cos``, ``emb_sin``), built by its ``rope_shift``
  (:68-84) on the cache's device.  The kernel reads ``cos`` and ``sgn`` as the Triton
  kernel does (:96, :127).  The rotary width is ``shift.emb_cos.numel()``: ``rope_shift``
  builds ``emb_cos`` as ``cat(ang, ang).cos()`` of the ``rotary / 2`` angles (:73, :83-84),
  and the element count of a tensor is host metadata, so a partial-rotary model
  (``partial_rotary_factor`` < 1, vllm_shift_connector.py:194-199) rotates exactly its
  first ``rotary`` dimensions with no argument from the caller and no device sync.
* ``partner`` is not read: ``rope_shift`` always builds the rotate-half permutation
  ``i + rotary/2`` (i < rotary/2), ``i - rotary/2`` (rotary/2 <= i < rotary), ``i``
  beyond (:79-81), and the kernel takes the partner element from the lane that holds it.
* There is no CPU path: a ``kv`` that is not on a HIP device raises (the reference falls
  back to its torch path there, :180-181; a caller that wants that keeps the reference's
  ``scatter_shifted`` for CPU tensors).

The library is found at ``$MARATHON_KVSHIFT_LIB``, else next to this file in
``_lib/libmarathon_kvshift.so`` (where this package's build puts it).
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_LIB_PATH = os.environ.get("MARATHON_KVSHIFT_LIB") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "_lib", "libmarathon_kvshift.so"
)
_DT = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2, torch.float8_e4m3fn: 3}
_lock = threading.Lock()
_lib = None


def _library() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(_LIB_PATH):
                    raise RuntimeError(f"{_LIB_PATH} is missing (set MARATHON_KVSHIFT_LIB)")
                i32, i64, vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p
                cdll = ctypes.CDLL(_LIB_PATH, mode=ctypes.RTLD_LOCAL)
                f = cdll.mkv_scatter_shifted
                f.restype = ctypes.c_int
                f.argtypes = [
                    vp, i64, i64,            # src, token stride, head stride (elements)
                    vp, i64, i64, i64, i64,  # kv, block / head / offset strides, num blocks
                    vp, i64,                 # slots (int64, device), n_tokens
                    i32, i32, i32, i32,      # heads, head_size, block_size, dtype
                    vp, vp, i32,             # cos, sgn (device fp32 [head_size]), rotary
                    vp, vp, vp,              # k_scale (fp8), error_flags, stream
                ]
                cdll.mkv_last_error.restype = ctypes.c_char_p
                _lib = cdll
    return _lib


def scatter_shifted(src, kv, slots, block_size, hnd, shift, *, k_scale=None):
    """Write ``src`` (``[n, heads, 2*head_size]``) into ``kv``'s slots, K rotated by delta.

    Drop-in for src/marathon/shift_kernels.py:166-210.  ``k_scale`` (a device fp32
    tensor holding the layer's K scale) is needed only for an fp8 e4m3 cache, which the
    reference does not have.
    """
    if not kv.is_cuda:
        raise RuntimeError("scatter_shifted: kv is not on a HIP device (no CPU path here)")
    n, heads, two_d = src.shape
    d = two_d // 2
    assert kv.shape[-1] == two_d, f"src row {two_d} != kv row {kv.shape[-1]}"
    if n == 0:
        return
    if src.dtype != kv.dtype:
        raise TypeError(f"src dtype {src.dtype} != kv dtype {kv.dtype}")
    if slots.device != kv.device or slots.dtype != torch.int64 or not slots.is_contiguous():
        slots = slots.to(device=kv.device, dtype=torch.int64, non_blocking=True).contiguous()
    rotary = shift.emb_cos.numel() if shift is not None else 0
    rotate = shift is not None and shift.delta != 0 and rotary > 0
    s = kv.stride()
    blk_s, head_s, off_s = (s[0], s[1], s[2]) if hnd else (s[0], s[2], s[1])
    if rotate and kv.dtype == torch.float8_e4m3fn and k_scale is None:
        raise ValueError("an fp8 KV cache needs k_scale")
    rc = _library().mkv_scatter_shifted(
        src.data_ptr(), src.stride(0), src.stride(1),
        kv.data_ptr(), blk_s, head_s, off_s, kv.shape[0],
        slots.data_ptr(), n, heads, d, block_size, _DT[kv.dtype],
        shift.cos.data_ptr() if rotate else None,
        shift.sgn.data_ptr() if rotate else None,
        rotary if rotate else 0,
        k_scale.data_ptr() if (rotate and k_scale is not None) else None,
        None,
        torch.cuda.current_stream(kv.device).cuda_stream,
    )
    if rc != 0:
        raise RuntimeError(_library().mkv_last_error().decode(errors="replace"))
