"""CPU oracle for the shift-connector KV reuse path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes on this path, so the
HIP kernels can be checked against it:

* :mod:`oracle.kvshift_oracle` -- numpy, bit-level: inverse frequencies, rotation
  tables, rotate-half re-rotation in the reference's fp32 op order, round-to-nearest-even
  back to bf16/fp16, the fp8 e4m3fn dequant -> rotate -> requant rule, slot mapping and
  the paged scatter for single spans, multi-span and batched span tables.
* :mod:`oracle.torch_path` -- the reference's torch op sequence for the shift
  (slice, upcast, cat-based rotate_half, mul/mul/add, cast, cat, index_put), run on the
  CPU.  It is the timed CPU baseline and the "reference rotation" the tests compare
  the kernels against (within 1 bf16 ulp).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only to check results or as the baseline -- never
as the thing measured or shipped.  The product (``marathon_amd``) never imports it and
has no CPU fallback.

Parity status of each function is listed in the module docstrings; every function
here is pinned by at least one check in ``tests/test_oracle.py`` (known answers from the
reference's own tests, torch library routines on closed forms, invariants, or brute
force), so no function of the oracle is "parity unpinned".
"""
