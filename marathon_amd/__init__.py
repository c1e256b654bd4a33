"""marathon_amd: the shift-connector KV reuse path of acrosley/marathon on MI355X.

Host API (mirrors src/marathon/shift_kernels.py and src/marathon/shift_store.py):
``rope_shift``, ``RopeShift``, ``scatter_shifted``, ``use_hip``, ``warmup``,
``ShiftStore``, ``SessionTable``, ``slots``, ``plan_load``, ``plan_save``; the
block-layout :class:`BlockShiftStore` (preallocated pool, per-position validity); batched
launches through :class:`marathon_amd.spans.ShiftPlan`; the worker-side load path in
:mod:`marathon_amd.connector`.  Everything that touches KV runs in hand-written gfx950
kernels (``csrc/kvshift.hip``) behind the C ABI in ``include/marathon_kvshift.h``.
"""

from .block_store import BlockShiftStore
from .shift_kernels import RopeShift, inv_freq_for, rope_shift, scatter_shifted, use_hip, warmup
from .shift_store import (
    DEFAULT_STORE_TOKENS,
    SLAB,
    LoadDecision,
    SessionTable,
    ShiftStore,
    plan_load,
    plan_save,
    slots,
)

__all__ = [
    "RopeShift",
    "inv_freq_for",
    "rope_shift",
    "scatter_shifted",
    "use_hip",
    "warmup",
    "DEFAULT_STORE_TOKENS",
    "SLAB",
    "LoadDecision",
    "SessionTable",
    "ShiftStore",
    "BlockShiftStore",
    "plan_load",
    "plan_save",
    "slots",
]
