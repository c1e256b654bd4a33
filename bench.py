"""Benchmark: fused KV-shift throughput on one MI355X.

Workload (one "step" = one whole shift, one launch): the Qwen3-14B-shaped multi-span
shift -- 40 layers, 8 KV heads, head_dim 128, bf16, a 30,720-token history with 8
reused spans (seed 3: 22,141 tokens, deltas in [-2048, 2048] incl. 0, no boundary on a
multiple of 16), read from the session store's block layout (each 16-token block a K
plane then a V plane, as the block store holds it) through a shuffled block table and
written into an HND paged cache through a slot mapping.  Inputs are resident
in HBM before timing.  Bytes are algorithmic: each K and V element read once and
written once (2 * tokens * layers * 8 * 256 * 2 B), reported in decimal GB/s.

Prints one JSON line.  Also measured, in the same line:
* ``roofline``: bytes per launch / mean launch time from HIP events on the launch
  stream, against the 8 TB/s HBM peak; ``traffic`` from the committed rocprofv3
  FETCH_SIZE/WRITE_SIZE profile of this kernel and workload, when present.
* ``cpu_baseline``: the reference's torch shift path (its op sequence, restated in
  ``oracle/torch_path.py``) on the host CPU over the headline workload itself (all 40
  layers and 8 spans), best of 5 after a warm-up, on every CPU the process may use; the
  Qwen3-0.6B-shaped CPU case (28 layers x 4,096 tokens, delta +37) is reported beside
  it, with the HIP path's time for that same shift (``qwen3_0_6b_shift_hip``).
* ``reference_shape``: the reference benchmark's own shape (30,720 tokens x 40 layers,
  delta 186, flat store -> HND paged cache, scattered block table), for comparison with
  its published 6.54 ms on an RTX 5090, as one batched launch.
* ``reference_loop``: the reference benchmark's own loop through the drop-in API: 40
  per-layer ``scatter_shifted`` calls per shift at 4,096, 12,288 and 30,720 tokens, the
  rows of its published table.
* ``tp_shares``: the headline shift at 4, 2 and 1 KV heads (one GPU's share at TP 2, 4,
  8), bf16 and fp8.
* ``session_batches``: the batched-sessions shift with 16 sessions, in fp8, and at one
  KV head (bf16 and fp8).
* ``size_sweep``: one batched shift of 512 to 32,768 tokens x 40 layers, to show where
  the fixed cost of a call stops mattering.
* ``ceilings``: a plain elementwise copy of the same bytes, and the headline with its
  block tables made the identity: what the GPU streams with nothing scattered.
* ``dst_layouts``: the headline shift into fused NHD caches and into caches that keep K
  and V in separate planes, beside the fused HND headline.
* ``src_layouts``: the headline shift, bf16 and fp8, from the store's K/V planes and
  from store blocks whose rows hold K then V per head.
* ``connector_step`` / ``save_step``: the connector's load and save calls end to end.
* ``plan_variants``: A/B of the token records' order (span order against destination
  page order) and of the single-launch direct path against the two-launch path.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_GBS = 8000.0  # MI355X HBM3E, decimal GB/s
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "shift_kernel_bf16_qwen3-14b-multispan_traffic.json")


def build_defines() -> str:
    """The tuning-knob definitions the library was built with ("" = the defaults)."""
    from marathon_amd.build import DEFINES_FILE

    try:
        with open(DEFINES_FILE) as f:
            return f.read().strip()
    except OSError:
        return "unknown"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def warm_up(launch, seconds: float = 0.25) -> None:
    """Launch repeatedly for ``seconds`` (the side sections' shifts take 0.1-12 ms;
    timed straight after building a workload, the first launches run on an idle GPU and
    read up to 12% slow)."""
    import torch

    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        launch()
        torch.cuda.synchronize()


def time_plan(plan, steps: int, warmup: int, stream):
    import torch

    for _ in range(warmup):
        plan.launch(stream.cuda_stream)
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record(stream)
        plan.launch(stream.cuda_stream)
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    return wall, per


def spot_check(wl, rows: int = 96, seed: int = 0) -> int:
    """Compare ``rows`` sampled (layer, token) rows of the output with the oracle."""
    import numpy as np
    import torch

    from oracle import kvshift_oracle as orc

    rng = np.random.default_rng(seed)
    inv = wl.inv_freq.numpy()
    src_tab = wl.meta["src_table"]
    sbs = wl.src.block_size
    dst_slots = wl.dst_index.numpy()
    spans = wl.spans
    checked = 0
    for _ in range(rows):
        s = int(rng.integers(len(spans)))
        sp = spans[s]
        i = int(rng.integers(int(sp["n_tokens"])))
        layer = int(rng.integers(wl.layers))
        pos = int(sp["src_pos"]) + i
        sblk, soff = int(src_tab[pos // sbs]), pos % sbs
        slot = int(dst_slots[int(sp["dst_index"]) + i])
        dblk, doff = slot // 16, slot % 16
        src_row = wl.src.fused(0, layer, (sblk, soff)).cpu()  # [heads, 2D], K then V
        got = wl.dst.caches[0][layer][dblk, :, doff].cpu()  # HND: [heads, 2D]
        sb = src_row.view(torch.int16).numpy().view(np.uint16)
        gb = got.view(torch.int16).numpy().view(np.uint16)
        want_k = orc.rotate_k_bits(sb[:, :128], int(sp["delta"]), inv, "bf16")
        if not (np.array_equal(gb[:, :128], want_k) and np.array_equal(gb[:, 128:], sb[:, 128:])):
            raise AssertionError(f"bench output differs from the oracle at span {s} token {i} layer {layer}")
        checked += 1
    return checked


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def host_cores() -> dict:
    """CPUs this process may run on (its affinity set), next to what the OS reports."""
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 1
    return {"os_cpu_count": os.cpu_count(), "usable": usable}


def _loadavg() -> list | None:
    try:
        return [round(x, 2) for x in os.getloadavg()]
    except OSError:
        return None


def _spread(seconds: list) -> dict:
    """min / median / max of timed passes, in ms."""
    import numpy as np

    ms = np.array(seconds) * 1e3
    return {"n": len(seconds), "min": round(float(ms.min()), 2),
            "median": round(float(np.median(ms)), 2), "max": round(float(ms.max()), 2)}


def _k_vs_torch_path(small: dict, gpu_out: dict) -> dict:
    """K of the Qwen3-0.6B shift written by the HIP path, against the reference's torch
    path on the CPU (``small["kv"]`` after the timed passes), over every element of the
    shifted rows of all 28 layers: with this package's correctly rounded tables (count
    and fraction more than 1 bf16 ulp apart, max ulp), and with the reference's own
    tables (``rope_shift(..., tables="reference")``: elements that differ at all)."""
    import numpy as np
    import torch

    from oracle import kvshift_oracle as orc

    sl = small["slots"].numpy()
    blk, off = sl // 16, sl % 16
    beyond = differ_ref = total = 0
    worst = 0
    for layer, ref in enumerate(small["kv"]):
        want = ref.view(torch.int16).numpy().view(np.uint16)[blk, :, off][..., :128]
        exact = gpu_out["exact"][layer].view(torch.int16).numpy().view(np.uint16)[blk, :, off][..., :128]
        refd = gpu_out["reference"][layer].view(torch.int16).numpy().view(np.uint16)[blk, :, off][..., :128]
        u = orc.ulp_distance_bf16(exact, want)
        beyond += int((u > 1).sum())
        worst = max(worst, int(u.max()))
        differ_ref += int((refd != want).sum())
        total += want.size
    return {"elements": total, "exact_tables_beyond_1ulp": beyond,
            "exact_tables_fraction_beyond_1ulp": float(f"{beyond / total:.3e}"),
            "exact_tables_max_ulp": worst, "reference_tables_elements_differing": differ_ref}


def cpu_baseline(reps: int = 5, gpu_small: dict | None = None,
                 small_gpu_out: dict | None = None) -> dict:
    """The reference torch shift path on the host CPU, on the headline workload itself:
    the Qwen3-14B multi-span shift (40 layers, 8 spans, 22,141 tokens), every layer and
    every span, read from the reference's flat store (shift_store.py:225-236, rows of a
    span are one contiguous view) and scattered into an HND paged cache through its
    slots.  Best of ``reps`` passes after one warm-up pass; also the Qwen3-0.6B case
    (28 layers x 4,096 tokens, delta +37), the reference's own CPU-sized shift, with
    the HIP path's time for the same shift (``gpu_small``) beside it.

    torch runs on every CPU this process may use (its affinity set; equal to
    ``os.cpu_count()`` unless the process is confined to fewer), as the reference's
    benchmark protocol asks (``torch.set_num_threads`` before timing)."""
    import numpy as np
    import torch

    cores = host_cores()
    torch.set_num_threads(cores["usable"])

    from marathon_amd import workloads as W
    from marathon_amd.shift_kernels import inv_freq_for
    from marathon_amd.shift_store import slots as slot_map
    from oracle import torch_path

    layers, heads, d, bs = 40, 8, 128, 16
    lay = W.qwen3_14b_multispan_layout()
    gen = torch.Generator().manual_seed(3)
    first = torch.randn(lay.src_history, heads, 2 * d, dtype=torch.bfloat16, generator=gen)
    stores = [first] + [first.clone() for _ in range(layers - 1)]  # distinct memory
    blocks = -(-lay.dst_history // bs) + 8
    caches = [torch.zeros(blocks, heads, bs, 2 * d, dtype=torch.bfloat16) for _ in range(layers)]
    table = np.random.default_rng(3).permutation(blocks).tolist()
    inv = inv_freq_for(d, 1e6)
    spans = []
    for s0, d0, n, dl in zip(lay.src_start, lay.dst_start, lay.length, lay.delta):
        s0, d0, n, dl = int(s0), int(d0), int(n), int(dl)
        emb = torch_path.rope_emb_tables(dl, inv) if dl != 0 else None
        spans.append((s0, n, slot_map(table, d0, d0 + n, bs), emb))
    load_before = _loadavg()
    passes = []
    for i in range(reps + 1):
        t0 = time.perf_counter()
        for store, cache in zip(stores, caches):
            for s0, n, sl, emb in spans:
                torch_path.shift_into_paged(store[s0:s0 + n], cache, sl, bs, True, emb)
        dt = time.perf_counter() - t0
        if i:
            passes.append(dt)
    best = min(passes)
    tokens = int(lay.length.sum())
    moved = 2 * tokens * layers * heads * 2 * d * 2
    del stores, caches

    # the reference's own CPU-sized case
    small = W.qwen3_0_6b_cpu_shift()
    emb_small = torch_path.rope_emb_tables(small["delta"], small["inv_freq"])
    passes_small = []
    for i in range(reps + 1):
        t0 = time.perf_counter()
        for src, kv in zip(small["src"], small["kv"]):
            torch_path.shift_into_paged(src, kv, small["slots"], 16, True, emb_small)
        dt = time.perf_counter() - t0
        if i:
            passes_small.append(dt)
    best_small = min(passes_small)
    load_after = _loadavg()
    moved_small = 2 * sum(t.numel() * t.element_size() for t in small["src"])
    small_row = {
        "GB_s": round(moved_small / best_small / 1e9, 3),
        "ms_per_shift": round(best_small * 1e3, 2),
        "passes_ms": _spread(passes_small),
    }
    if small_gpu_out is not None:
        small_row["k_vs_torch_path"] = _k_vs_torch_path(small, small_gpu_out)
    if gpu_small:
        small_row["hip"] = gpu_small
        small_row["hip_speedup_batched"] = round(best_small * 1e3 / gpu_small["batched_ms"], 1)
    return {
        "value": round(moved / best / 1e9, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "os_cpu_count": cores["os_cpu_count"],
        "usable_cpus": cores["usable"],
        "kind": "port",
        "sample": f"the reference torch shift path (oracle/torch_path.py) on the CPU over the "
        f"whole Qwen3-14B multi-span shift: {layers} layers x 8 spans, {tokens:,} tokens, flat "
        f"store -> HND paged cache; best of {reps} passes after 1 warm-up; "
        f"{best * 1e3:.1f} ms per shift; {torch.get_num_threads()} torch threads "
        f"(os.cpu_count() {cores['os_cpu_count']}, {cores['usable']} usable); "
        f"CPU: {_cpu_model()}",
        "ms_per_shift": round(best * 1e3, 2),
        "passes_ms": _spread(passes),
        "host_loadavg_1_5_15min": {"before": load_before, "after": load_after},
        "qwen3_0_6b_4096_tokens": small_row,
    }


def qwen3_0_6b_hip(dev, steps: int, warmup: int, stream, iters: int = 5,
                   keep_outputs: bool = False):
    """The Qwen3-0.6B-shaped shift the CPU baseline also times (28 layers, a flat store of
    4,096 tokens per layer, one span shifted by +37 into 259 of 512 seeded HND blocks),
    on the HIP path: one batched launch (HIP events on the launch stream, mean over
    ``steps``) and the reference's call pattern of 28 per-layer ``scatter_shifted``
    calls (host wall clock, best of ``iters``).  A sampled row is checked against the
    oracle."""
    import numpy as np
    import torch

    from marathon_amd import workloads as W
    from marathon_amd.shift_kernels import rope_shift, scatter_shifted
    from marathon_amd.spans import CacheSet, ShiftPlan, span_array
    from oracle import kvshift_oracle as orc

    wl = W.qwen3_0_6b_cpu_shift()
    delta, n = wl["delta"], wl["src"][0].shape[0]
    src = [t.to(dev) for t in wl["src"]]
    kv = [t.to(dev) for t in wl["kv"]]
    slots = wl["slots"].to(dev)
    plan = ShiftPlan(span_array([(0, 0, 0, 0, n, delta, 0, 0)]), CacheSet(src, "flat"),
                     CacheSet(kv, "hnd", 16), inv_freq=wl["inv_freq"], src_mode="flat",
                     dst_mode="slots", dst_index=wl["slots"])
    warm_up(lambda: plan.launch(stream.cuda_stream))
    _, per = time_plan(plan, max(steps, 50), warmup, stream)
    ms = float(np.mean(per))
    shift = rope_shift(delta, 128, wl["inv_freq"], dev)

    def loop():
        for s_, k_ in zip(src, kv):
            scatter_shifted(s_, k_, slots, 16, True, shift)

    warm_up(loop)
    best = float("inf")
    for _ in range(iters):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        loop()
        torch.cuda.synchronize()
        best = min(best, (time.perf_counter() - t0) * 1e3)
    t = int(np.random.default_rng(1).integers(n))
    slot = int(wl["slots"][t])
    sb = wl["src"][-1][t].view(torch.int16).numpy().view(np.uint16)
    gb = kv[-1][slot // 16, :, slot % 16].cpu().view(torch.int16).numpy().view(np.uint16)
    if not (np.array_equal(gb[:, :128], orc.rotate_k_bits(sb[:, :128], delta,
                                                         wl["inv_freq"].numpy(), "bf16"))
            and np.array_equal(gb[:, 128:], sb[:, 128:])):
        raise AssertionError("Qwen3-0.6B shift differs from the oracle")
    moved = plan.algorithmic_bytes
    out = {
        "shape": "28 layers x 4,096 tokens x 8 heads x 128, bf16, delta +37, flat store -> "
        "HND paged (259 of 512 seeded blocks)",
        "bytes": moved,
        "batched_ms": round(ms, 4),
        "batched_GB_s": round(moved / (ms / 1e3) / 1e9, 1),
        "per_layer_loop_ms": round(best, 4),
        "per_layer_loop_GB_s": round(moved / (best / 1e3) / 1e9, 1),
    }
    outputs = None
    if keep_outputs:
        # the caches as the per-layer loop left them (this package's tables), then the
        # same loop with the reference's own torch fp32 tables built on the CPU, as the
        # CPU torch path uses them; compared with that path after the CPU leg has run
        torch.cuda.synchronize()
        outputs = {"exact": [t.cpu() for t in kv]}
        ref = rope_shift(delta, 128, wl["inv_freq"], "cpu", tables="reference")
        ref = type(ref)(ref.delta, ref.cos.to(dev), ref.sgn.to(dev), ref.partner,
                        ref.emb_cos, ref.emb_sin, ref.inv_freq, ref.rotary)
        for s_, k_ in zip(src, kv):
            scatter_shifted(s_, k_, slots, 16, True, ref)
        torch.cuda.synchronize()
        outputs["reference"] = [t.cpu() for t in kv]
    del src, kv, plan
    torch.cuda.empty_cache()
    return (out, outputs) if keep_outputs else out


def reference_shape(dev, steps: int, warmup: int, stream) -> dict:
    """The reference micro-benchmark's shape (scripts/bench_shift_copy.py:24-53)."""
    import numpy as np
    import torch

    from marathon_amd.shift_kernels import inv_freq_for
    from marathon_amd.spans import CacheSet, ShiftPlan, span_array

    n, layers, heads, d, bs = 30720, 40, 8, 128, 16
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    blocks = -(-n // bs) + 8
    src = [torch.randn(n, heads, 2 * d, dtype=torch.bfloat16, device=dev, generator=gen)
           for _ in range(layers)]
    kv = [torch.zeros(blocks, heads, bs, 2 * d, dtype=torch.bfloat16, device=dev)
          for _ in range(layers)]
    table = torch.randperm(blocks, device=dev, generator=gen)
    pos = torch.arange(n, device=dev)
    slot = table[pos // bs] * bs + pos % bs
    plan = ShiftPlan(span_array([(0, 0, 0, 0, n, 186, 0, 0)]), CacheSet([src], "flat"),
                     CacheSet([kv], "hnd", bs), inv_freq=inv_freq_for(d, 1e6),
                     src_mode="flat", dst_mode="slots", dst_index=slot)
    warm_up(lambda: plan.launch(stream.cuda_stream))
    wall, per = time_plan(plan, steps, warmup, stream)
    ms = float(np.mean(per))
    out = {
        "shape": "30,720 tokens x 40 layers x 8 heads x 128, bf16, delta 186, flat store -> "
        "HND paged (scripts/bench_shift_copy.py)",
        "ms": round(ms, 4),
        "GB_s": round(plan.algorithmic_bytes / (ms / 1e3) / 1e9, 1),
        "reference_rtx5090_ms": 6.54,
    }
    del src, kv, plan
    torch.cuda.empty_cache()
    return out


def reference_loop(dev, iters: int = 5) -> dict:
    """The reference micro-benchmark's own loop through the drop-in API
    (scripts/bench_shift_copy.py:24-53): for each of 40 layers, one ``scatter_shifted``
    call from a ``[n, 8, 256]`` bf16 store slice into an HND paged cache through a
    scattered slot mapping, delta 186.  Host wall clock around the 40 calls
    (synchronised on both sides), best of ``iters`` passes after a warm-up; bytes are
    the source read once plus the destination written once.  One row per token count
    of its published table (docs/findings.md:644-646, RTX 5090).  Beside each, the same
    loop of 40 launches of torch's elementwise kernel over the same bytes."""
    import numpy as np
    import torch

    from marathon_amd.shift_kernels import inv_freq_for, rope_shift, scatter_shifted
    from oracle import kvshift_oracle as orc

    layers, heads, d, bs = 40, 8, 128, 16
    inv = inv_freq_for(d, 1e6)
    shift = rope_shift(186, d, inv, dev)
    published = {4096: 1.01, 12288: 2.80, 30720: 6.54}
    out = {"what": "40 per-layer scatter_shifted calls per shift (the reference's call "
           "pattern), best of %d after a 0.25 s warm-up, host wall clock" % iters}
    for n, ref_ms in published.items():
        gen = torch.Generator(device=dev)
        gen.manual_seed(n)
        blocks = -(-n // bs) + 8
        src = [torch.randn(n, heads, 2 * d, dtype=torch.bfloat16, device=dev, generator=gen)
               for _ in range(layers)]
        kv = [torch.zeros(blocks, heads, bs, 2 * d, dtype=torch.bfloat16, device=dev)
              for _ in range(layers)]
        table = torch.randperm(blocks, device=dev, generator=gen)
        pos = torch.arange(n, device=dev)
        slots = table[pos // bs] * bs + pos % bs
        best = host = float("inf")

        def one_shift():
            for s, k in zip(src, kv):
                scatter_shifted(s, k, slots, bs, True, shift)

        warm_up(one_shift)
        for i in range(iters + 1):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for s, k in zip(src, kv):
                scatter_shifted(s, k, slots, bs, True, shift)
            t1 = time.perf_counter()
            torch.cuda.synchronize()
            ms = (time.perf_counter() - t0) * 1e3
            if i:
                best = min(best, ms)
                host = min(host, (t1 - t0) * 1e3)
        # one sampled row of the last layer against the oracle
        t = int(np.random.default_rng(n).integers(n))
        slot = int(slots[t])
        sb = src[-1][t].cpu().view(torch.int16).numpy().view(np.uint16)
        gb = kv[-1][slot // bs, :, slot % bs].cpu().view(torch.int16).numpy().view(np.uint16)
        if not (np.array_equal(gb[:, :d], orc.rotate_k_bits(sb[:, :d], 186, inv.numpy(), "bf16"))
                and np.array_equal(gb[:, d:], sb[:, d:])):
            raise AssertionError(f"reference loop output differs from the oracle at n={n}")
        moved = 2 * sum(s.numel() * s.element_size() for s in src)
        # the same 40-launch loop through torch's elementwise kernel, the same bytes
        # (each layer's rows read once, written once into a tensor of their size): the
        # floor that one launch per layer sets on this GPU
        outs = [torch.empty_like(s) for s in src]

        def torch_loop():
            for s, o in zip(src, outs):
                torch.neg(s, out=o)

        warm_up(torch_loop)
        best_torch = float("inf")
        for i in range(iters + 1):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            torch_loop()
            torch.cuda.synchronize()
            if i:
                best_torch = min(best_torch, (time.perf_counter() - t0) * 1e3)
        # and through the hand-written stream copy (tests/hip/copy_ceiling.hip, sc1 nt
        # stores): the fastest 40-launch loop over these bytes found for this GPU
        cl = _ceiling_lib()
        st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        nb = src[0].numel() * src[0].element_size()

        def copy_loop():
            for s, o in zip(src, outs):
                if cl.ceil_stream_copy(s.data_ptr(), o.data_ptr(), nb, 1, st) != 0:
                    raise RuntimeError("ceil_stream_copy refused its arguments")

        warm_up(copy_loop)
        best_copy = float("inf")
        for i in range(iters + 1):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            copy_loop()
            torch.cuda.synchronize()
            if i:
                best_copy = min(best_copy, (time.perf_counter() - t0) * 1e3)
        if not torch.equal(outs[-1], src[-1]):
            raise AssertionError("stream copy loop output differs from its source")
        out[f"tokens_{n}"] = {
            "ms": round(best, 4),
            "GB_s": round(moved / (best / 1e3) / 1e9, 1),
            "GiB_s": round(moved / (best / 1e3) / 2**30, 1),
            "us_per_token": round(best * 1e3 / n, 4),
            "host_enqueue_ms": round(host, 4),
            "torch_neg_loop_ms": round(best_torch, 4),
            "torch_neg_loop_GB_s": round(moved / (best_torch / 1e3) / 1e9, 1),
            "stream_copy_loop_ms": round(best_copy, 4),
            "stream_copy_loop_frac_of_peak": round(moved / (best_copy / 1e3) / 1e9 / PEAK_GBS, 4),
            "frac_of_peak": round(moved / (best / 1e3) / 1e9 / PEAK_GBS, 4),
            "reference_rtx5090_ms": ref_ms,
        }
        del src, kv, slots, table, outs
        torch.cuda.empty_cache()
    return out


def other_workloads(dev, steps: int, warmup: int, stream) -> dict:
    """Informational: the other GPU workloads, one launch per step each."""
    import numpy as np
    import torch

    from marathon_amd import workloads as W

    out = {}
    for name, make in (("qwen3_8b_single_span_bf16", lambda: W.qwen3_8b_single_span(dev)),
                       ("qwen3_14b_multispan_fp8", lambda: W.qwen3_14b_multispan_fp8(dev)),
                       ("batched_32_sessions_bf16", lambda: W.batched_sessions(dev))):
        log(f"timing {name}")
        wl = make()
        plan = wl.plan()
        warm_up(lambda: plan.launch(stream.cuda_stream))
        _, per = time_plan(plan, steps, warmup, stream)
        ms = float(np.mean(per))
        out[name] = {
            "tokens": wl.tokens,
            "layers": wl.layers,
            "spans": int(len(wl.spans)),
            "ms": round(ms, 4),
            "GB_s": round(plan.algorithmic_bytes / (ms / 1e3) / 1e9, 1),
            "frac_of_peak": round(plan.algorithmic_bytes / (ms / 1e3) / 1e9 / PEAK_GBS, 4),
        }
        del wl, plan
        torch.cuda.empty_cache()
    return out


def session_batches(dev, steps: int, warmup: int, stream) -> dict:
    """Informational: the batched-sessions shift (config 5's layout: each session its
    own store, one shared HND destination pool, 36 layers) in its other forms: 16
    sessions, fp8 e4m3, and one GPU's share under tensor parallelism 8 (1 KV head) in
    bf16 and fp8.  One launch per step each."""
    import numpy as np
    import torch

    from marathon_amd import workloads as W

    out = {}
    for name, make in (
            ("sessions_16_bf16", lambda: W.batched_sessions(dev, sessions=16)),
            ("sessions_32_fp8", lambda: W.batched_sessions(dev, dtype=torch.float8_e4m3fn)),
            ("sessions_32_tp8_bf16", lambda: W.batched_sessions(dev, heads=1)),
            ("sessions_32_tp8_fp8",
             lambda: W.batched_sessions(dev, heads=1, dtype=torch.float8_e4m3fn))):
        log(f"timing {name}")
        wl = make()
        plan = wl.plan()
        warm_up(lambda: plan.launch(stream.cuda_stream))
        _, per = time_plan(plan, steps, warmup, stream)
        ms = float(np.median(per))
        gbs = plan.algorithmic_bytes / (ms / 1e3) / 1e9
        out[name] = {"sessions": int(wl.src.groups), "heads": int(wl.dst.heads),
                     "tokens": wl.tokens, "layers": wl.layers, "ms": round(ms, 4),
                     "GB_s": round(gbs, 1), "frac_of_peak": round(gbs / PEAK_GBS, 4)}
        del wl, plan
        torch.cuda.empty_cache()
    return out


def tp_shares(dev, steps: int, warmup: int, stream) -> dict:
    """Informational: one GPU's share of the headline shift under tensor parallelism
    over KV heads (4, 2 and 1 heads of 8), bf16 and fp8, one launch per step."""
    import numpy as np
    import torch

    from marathon_amd import workloads as W

    out = {}
    for heads in (4, 2, 1):
        for name, make in (("bf16", lambda h: W.qwen3_14b_multispan(dev, heads=h)),
                           ("fp8", lambda h: W.qwen3_14b_multispan_fp8(dev, heads=h))):
            wl = make(heads)
            plan = wl.plan()
            warm_up(lambda: plan.launch(stream.cuda_stream))
            _, per = time_plan(plan, max(steps, 50), warmup, stream)
            ms = float(np.median(per))
            gbs = plan.algorithmic_bytes / (ms / 1e3) / 1e9
            row = {"heads": heads, "ms": round(ms, 4), "GB_s": round(gbs, 1),
                   "frac_of_peak": round(gbs / PEAK_GBS, 4)}
            if name == "bf16":
                row["rows_checked"] = spot_check(wl, rows=32, seed=heads)
            out[f"tp{8 // heads}_{name}"] = row
            del wl, plan
            torch.cuda.empty_cache()
    return out


def size_sweep(dev, steps: int, warmup: int, stream) -> dict:
    """Informational: one batched shift of n tokens x 40 layers (a flat store span into
    an HND paged cache through shuffled slots, delta 186) for n from 512 to 32,768: how
    the fixed costs of a call (the plan kernel, two launches, ramp-up and drain) weigh
    on small shifts.  Beside each: the same bytes through the hand-written stream copy
    and the same rows through the hand-written paged copy (one block id per token, then
    the data), each one launch timed the same way."""
    import numpy as np
    import torch

    from marathon_amd.shift_kernels import inv_freq_for
    from marathon_amd.spans import CacheSet, ShiftPlan, span_array

    layers, heads, d, bs = 40, 8, 128, 16
    out = {}
    cl = _ceiling_lib()
    for n in (512, 2048, 8192, 32768):
        gen = torch.Generator(device=dev)
        gen.manual_seed(n)
        blocks = -(-n // bs) + 8
        src = [torch.randn(n, heads, 2 * d, dtype=torch.bfloat16, device=dev, generator=gen)
               for _ in range(layers)]
        kv = [torch.zeros(blocks, heads, bs, 2 * d, dtype=torch.bfloat16, device=dev)
              for _ in range(layers)]
        table = torch.randperm(blocks, device=dev, generator=gen)
        pos = torch.arange(n, device=dev)
        slot = table[pos // bs] * bs + pos % bs
        plan = ShiftPlan(span_array([(0, 0, 0, 0, n, 186, 0, 0)]), CacheSet([src], "flat"),
                         CacheSet([kv], "hnd", bs), inv_freq=inv_freq_for(d, 1e6),
                         src_mode="flat", dst_mode="slots", dst_index=slot)
        warm_up(lambda: plan.launch(stream.cuda_stream))
        _, per = time_plan(plan, max(steps, 50), warmup, stream)
        ms = float(np.median(per))
        gbs = plan.algorithmic_bytes / (ms / 1e3) / 1e9
        # the same bytes through one launch of the hand-written stream copy, timed the
        # same way (HIP events around each launch, median): the ceiling at this size
        half = plan.algorithmic_bytes // 2
        a = torch.empty(half, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        st = ctypes.c_void_p(stream.cuda_stream)
        cms = _time_launch(lambda: cl.ceil_stream_copy(a.data_ptr(), b.data_ptr(), half, 1, st),
                           max(steps, 50), stream)
        del a, b
        pms = _sweep_paged_copy(cl, plan, table, n, max(steps, 50), stream)
        moved = plan.algorithmic_bytes
        out[f"tokens_{n}"] = {"ms": round(ms, 4), "GB_s": round(gbs, 1),
                              "frac_of_peak": round(gbs / PEAK_GBS, 4),
                              "us_per_token": round(ms * 1e3 / n, 5),
                              "stream_copy_ms": round(cms, 4),
                              "stream_copy_frac_of_peak": round(
                                  moved / (cms / 1e3) / 1e9 / PEAK_GBS, 4),
                              "paged_copy_ms": round(pms, 4),
                              "paged_copy_frac_of_peak": round(
                                  moved / (pms / 1e3) / 1e9 / PEAK_GBS, 4)}
        del src, kv, plan
        torch.cuda.empty_cache()
    return out


def _sweep_paged_copy(cl, plan, table, n: int, runs: int, stream) -> float:
    """The size sweep's rows (n tokens x every layer, the flat source read as 16-token
    blocks in order, the destination through the sweep's block table) moved by the
    hand-written paged copy, which reads one block id per token and then the data, with
    no rotation and no span or slot metadata.  Returns the median ms of ``runs``
    launches, after checking eight sampled rows."""
    import torch

    dev = plan.dst.first.device
    eb = plan.dst.first.element_size()
    heads, d, layers = plan.dst.heads, plan.dst.head_size, plan.dst.layers
    s_k, s_v, _, _, _ = plan.src.device_tables(dev)
    d_k, d_v, _, _, _ = plan.dst.device_tables(dev)
    row, s_head, _ = plan.src.strides  # flat rows: token stride, head stride
    d_block, d_head, d_off = plan.dst.strides
    ident = torch.arange(n // 16, dtype=torch.int32, device=dev)
    tab = table.to(torch.int32)
    torch.cuda.synchronize()
    st = ctypes.c_void_p(stream.cuda_stream)
    args = (s_k, s_v, d_k, d_v, layers, ident.data_ptr(), ident.numel(), n // 16,
            tab.data_ptr(), tab.numel(), plan.dst.first.shape[0], n, heads, d * eb,
            16 * row * eb, s_head * eb, row * eb, d_block * eb, d_head * eb, d_off * eb, st)

    def launch():
        if cl.ceil_paged_copy(*args) != 0:
            raise RuntimeError("ceil_paged_copy refused the size sweep's arguments")

    ms = _time_launch(launch, runs, stream)
    for k in range(8):
        pos, layer = (k * 977 + 5) % n, (k * 13) % layers
        blk = int(tab[pos // 16])
        want = plan.src.caches[0][layer][pos]
        got = plan.dst.caches[0][layer][blk, :, pos % 16]
        if not torch.equal(want.view(torch.uint8), got.contiguous().view(torch.uint8)):
            raise AssertionError(f"size sweep paged copy: row {pos} layer {layer}")
    return ms


def ceilings(dev, steps: int, warmup: int, stream) -> dict:
    """Informational: what this GPU streams with nothing scattered, beside the headline.

    * ``elementwise_copy``: torch's elementwise kernel (``neg``) over 3.6 GB of bf16,
      reading it once and writing it once (the headline moves 7.26 GB the same way).
    * ``headline_identity_tables``: the headline shift through the same kernel, with the
      source block table and the destination slots made the identity, so every span is
      one contiguous run on each side.  The gap between this and the headline is what
      scattered 64 KB blocks cost.  ``headline_fp8_identity_tables``: the same for the
      fp8 shift (32 KB blocks).
    * ``headline_zero_delta`` / ``headline_fp8_zero_delta``: the headline shift (shuffled
      tables) with every span's delta set to 0, so K is copied like V: the same gather and
      scatter with no rotation.  The gap between this and the headline is what the
      rotation costs.
    """
    import numpy as np
    import torch

    from marathon_amd import workloads as W

    out = {}
    n = 22141 * 40 * 8 * 256  # the headline's K and V elements (tokens x layers x heads x 2D)
    a = torch.zeros(n, dtype=torch.bfloat16, device=dev)
    b = torch.empty_like(a)
    warm_up(lambda: torch.neg(a, out=b))
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    for i in range(steps):
        starts[i].record(stream)
        torch.neg(a, out=b)
        ends[i].record(stream)
    torch.cuda.synchronize()
    ms = float(np.median([s_.elapsed_time(e) for s_, e in zip(starts, ends)]))
    moved = 2 * a.numel() * a.element_size()
    out["elementwise_copy"] = {"bytes": moved, "ms": round(ms, 4),
                               "GB_s": round(moved / (ms / 1e3) / 1e9, 1),
                               "frac_of_peak": round(moved / (ms / 1e3) / 1e9 / PEAK_GBS, 4)}
    del a, b
    torch.cuda.empty_cache()

    for name, make in (("headline_identity_tables", W.qwen3_14b_multispan),
                       ("headline_fp8_identity_tables", W.qwen3_14b_multispan_fp8)):
        wl = make(dev)
        wl.src_index = torch.arange(wl.src.first.shape[0], dtype=torch.int32)
        wl.dst_index = torch.cat([torch.arange(int(r["dst_pos"]),
                                               int(r["dst_pos"]) + int(r["n_tokens"]),
                                               dtype=torch.int64) for r in wl.spans])
        if int(wl.dst_index.max()) >= wl.dst.first.shape[0] * 16:
            raise AssertionError("identity slots exceed the destination cache")
        plan = wl.plan()
        warm_up(lambda: plan.launch(stream.cuda_stream))
        _, per = time_plan(plan, max(steps, 50), warmup, stream)
        ms = float(np.median(per))
        gbs = plan.algorithmic_bytes / (ms / 1e3) / 1e9
        out[name] = {"ms": round(ms, 4), "GB_s": round(gbs, 1),
                     "frac_of_peak": round(gbs / PEAK_GBS, 4)}
        del wl, plan
        torch.cuda.empty_cache()

    for name, make in (("headline_zero_delta", W.qwen3_14b_multispan),
                       ("headline_fp8_zero_delta", W.qwen3_14b_multispan_fp8)):
        wl = make(dev)
        wl.spans["delta"] = 0
        plan = wl.plan()
        warm_up(lambda: plan.launch(stream.cuda_stream))
        _, per = time_plan(plan, max(steps, 50), warmup, stream)
        ms = float(np.median(per))
        gbs = plan.algorithmic_bytes / (ms / 1e3) / 1e9
        out[name] = {"ms": round(ms, 4), "GB_s": round(gbs, 1),
                     "frac_of_peak": round(gbs / PEAK_GBS, 4)}
        del wl, plan
        torch.cuda.empty_cache()
    return out


CEILING_LIB = os.path.join(ROOT, "tests", "_lib", "libcopy_ceiling.so")


def _ceiling_lib():
    """The copy kernels of tests/hip/copy_ceiling.hip (built by ``build()``): benchmark
    infrastructure, not the product library."""
    import ctypes

    if not os.path.exists(CEILING_LIB):
        raise RuntimeError(f"{CEILING_LIB} is missing: run __graft_entry__.build()")
    lib = ctypes.CDLL(CEILING_LIB)
    i32, i64, vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p
    lib.ceil_stream_copy.argtypes = [vp, vp, i64, i32, vp]
    lib.ceil_stream_copy_persistent.argtypes = [vp, vp, i64, i32, vp]
    lib.ceil_paged_copy.argtypes = [vp, vp, vp, vp, i32, vp, i64, i64, vp, i64, i64, i64, i32,
                                    i32, i64, i64, i64, i64, i64, i64, vp]
    lib.ceil_paged_copy_lanes.argtypes = [vp, vp, vp, vp, i32, vp, i64, i64, vp, i64, i64, i64,
                                          i32, i32, i64, i64, i64, i64, i64, i64, i32, vp]
    lib.ceil_paged_copy_ex.argtypes = [vp, vp, vp, vp, i32, vp, i64, i64, vp, i64, i64, i64,
                                       i32, i32, i64, i64, i64, i64, i64, i64, i32, vp, vp]
    return lib


def _time_launch(launch, steps: int, stream) -> float:
    """Median ms of ``launch()`` over ``steps`` launches, HIP events on ``stream``."""
    import numpy as np
    import torch

    warm_up(launch)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    for i in range(steps):
        starts[i].record(stream)
        launch()
        ends[i].record(stream)
    torch.cuda.synchronize()
    return float(np.median([s_.elapsed_time(e) for s_, e in zip(starts, ends)]))


def copy_ceilings(dev, steps: int, warmup: int, stream) -> dict:
    """Hand-written copies of the headline's bytes (tests/hip/copy_ceiling.hip), the
    practical ceiling the shift kernel is held to:

    * ``stream_copy_*``: one contiguous 3.63 GB buffer into another (the headline's
      7.26 GB read once and written once), 16 bytes per thread, one-shot grid, XCD-aware
      order, non-temporal loads; stores non-temporal (``nt``) or device-scope streaming
      (``sc1 nt``, the shift kernel's stores).  ``*_persistent_*``: the same copy by a
      fixed grid of 1,024 / 2,048 / 8,192 workgroups walking the buffer.
    * ``paged_copy_*``: the headline's 22,141 tokens x 40 layers from the session store's
      blocks into the HND paged cache, through the headline's own shuffled block tables
      (``shuffled``) or identity tables (``identity``), with no rotation and no token
      metadata beyond the two block ids: bf16 from the store's K/V planes (64 KB blocks),
      fp8 from its fused rows (32 KB blocks), as the headline and its fp8 twin read them.
    * ``paged_copy_*_runs_of_G_blocks``: the same copy with both block tables shuffled in
      runs of G consecutive blocks, up to one 2 MB translation page per run.
    * ``paged_copy_*_kv_split``: the same copy with K and V moved by separate waves (a
      wave pair per row group); ``*_k_after_read``: each K store held behind one
      dependent read of a small table after its data arrives, as the shift's rotation
      holds K behind its cos/sin table.
    * ``paged_copy_*_1head_shuffled_*``: the same copy of one GPU's share under tensor
      parallelism 8 (1 KV head), each lane finding its own (token, head) row as the
      shift kernel's per-lane path does, with ``sc1 nt`` buffer or ``nt`` global stores.

    Every copy is checked after timing: the stream copy whole, the paged copy on sampled
    rows."""
    import ctypes

    import numpy as np
    import torch

    from marathon_amd import workloads as W

    lib = _ceiling_lib()
    st = ctypes.c_void_p(stream.cuda_stream)
    runs = max(steps, 50)
    out = {}
    nbytes = 22141 * 40 * 8 * 256 * 2  # the headline's K and V bytes, read once
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    a = torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), dtype=torch.int32, device=dev,
                      generator=gen)
    b = torch.empty_like(a)
    for name, scope in (("stream_copy_nt", 0), ("stream_copy_sc1_nt", 1)):
        b.zero_()

        def launch(scope=scope):
            if lib.ceil_stream_copy(a.data_ptr(), b.data_ptr(), nbytes, scope, st) != 0:
                raise RuntimeError("ceil_stream_copy refused its arguments")

        ms = _time_launch(launch, runs, stream)
        if not torch.equal(a, b):
            raise AssertionError(f"{name}: the copy differs from its source")
        gbs = 2 * nbytes / (ms / 1e3) / 1e9
        out[name] = {"bytes": 2 * nbytes, "ms": round(ms, 4), "GB_s": round(gbs, 1),
                     "frac_of_peak": round(gbs / PEAK_GBS, 4)}
    # the same copy by a persistent grid (workgroups walking the buffer in grid strides)
    for wgs in (1024, 2048, 8192):
        name = f"stream_copy_sc1_nt_persistent_{wgs}_workgroups"
        b.zero_()

        def launch(wgs=wgs):
            if lib.ceil_stream_copy_persistent(a.data_ptr(), b.data_ptr(), nbytes, wgs, st) != 0:
                raise RuntimeError("ceil_stream_copy_persistent refused its arguments")

        ms = _time_launch(launch, runs, stream)
        if not torch.equal(a, b):
            raise AssertionError(f"{name}: the copy differs from its source")
        gbs = 2 * nbytes / (ms / 1e3) / 1e9
        out[name] = {"bytes": 2 * nbytes, "ms": round(ms, 4), "GB_s": round(gbs, 1),
                     "frac_of_peak": round(gbs / PEAK_GBS, 4), "workgroups": wgs}
    del a, b
    torch.cuda.empty_cache()

    rng = np.random.default_rng(0)
    for dname, make in (("bf16", W.qwen3_14b_multispan), ("fp8", W.qwen3_14b_multispan_fp8)):
        wl = make(dev)
        tables = {
            "shuffled": (np.asarray(wl.meta["src_table"], np.int32),
                         np.asarray(wl.meta["dst_table"], np.int32)),
            "identity": (np.arange(wl.src.first.shape[0], dtype=np.int32),
                         np.arange(wl.dst.first.shape[0], dtype=np.int32)),
        }
        for tname, (st_np, dt_np) in tables.items():
            out[f"paged_copy_{dname}_{tname}"] = _paged_copy(
                lib, wl, st_np, dt_np, None, runs, stream, rng, f"paged_copy_{dname}_{tname}")
            name = f"paged_copy_{dname}_{tname}_kv_split"
            out[name] = _paged_copy(lib, wl, st_np, dt_np, None, runs, stream, rng, name,
                                    ex=(1, False))
        st_np, dt_np = tables["shuffled"]
        for suffix, ex in (("k_after_read", (0, True)), ("kv_split_k_after_read", (1, True))):
            name = f"paged_copy_{dname}_shuffled_{suffix}"
            out[name] = _paged_copy(lib, wl, st_np, dt_np, None, runs, stream, rng, name, ex=ex)
        # both tables permuted in runs of G consecutive blocks (G = 1: every block on its
        # own; the largest G makes a run one 2 MB translation page): how the cost of
        # scattered blocks fades as the runs grow
        blk_bytes = 16 * wl.dst.heads * 2 * wl.dst.head_size * wl.dst.first.element_size()
        page_blocks = (2 << 20) // blk_bytes
        perm = np.random.default_rng(7)
        for g in (1, 4, page_blocks):
            st_np = _run_permutation(wl.src.first.shape[0], g, perm)
            dt_np = _run_permutation(wl.dst.first.shape[0], g, perm)
            name = f"paged_copy_{dname}_runs_of_{g}_blocks"
            out[name] = _paged_copy(lib, wl, st_np, dt_np, None, runs, stream, rng, name)
        del wl
        torch.cuda.empty_cache()
    # one GPU's share under tensor parallelism 8 (1 KV head): rows of 256 B (bf16) or
    # 128 B (fp8), a wave's rows spanning tokens, each lane resolving its own row
    for dname, make in (("bf16", W.qwen3_14b_multispan), ("fp8", W.qwen3_14b_multispan_fp8)):
        wl = make(dev, heads=1)
        st_np = np.asarray(wl.meta["src_table"], np.int32)
        dt_np = np.asarray(wl.meta["dst_table"], np.int32)
        for sname, scope in (("sc1_nt", 1), ("nt", 0)):
            name = f"paged_copy_{dname}_1head_shuffled_{sname}"
            out[name] = _paged_copy(lib, wl, st_np, dt_np, scope, runs, stream, rng, name)
        del wl
        torch.cuda.empty_cache()
    return out


def _run_permutation(n: int, run: int, rng):
    """A block table over n blocks that keeps runs of ``run`` consecutive blocks together
    and shuffles the runs (the last run may be short)."""
    import numpy as np

    starts = np.arange(0, n, run)[rng.permutation(-(-n // run))]
    return np.concatenate([np.arange(a, min(a + run, n)) for a in starts]).astype(np.int32)


def _paged_copy(lib, wl, st_np, dt_np, lanes_scope, runs: int, stream, rng, name: str,
                ex=None) -> dict:
    """Time one paged copy of the workload's 22,141 tokens x every layer from its store
    blocks into its paged cache through the given block tables, and check 32 sampled
    rows.  ``lanes_scope`` None: ``ceil_paged_copy`` (a wave's rows in one token);
    0 or 1: ``ceil_paged_copy_lanes`` with ``nt`` or ``sc1 nt`` stores.  ``ex``
    (kv_split, k_after_read): ``ceil_paged_copy_ex`` instead."""
    import ctypes

    import torch

    dev = wl.dst.first.device
    n = 22141
    st = ctypes.c_void_p(stream.cuda_stream)
    eb = wl.dst.first.element_size()
    heads, d, layers = wl.dst.heads, wl.dst.head_size, wl.layers
    s_k, s_v, _, _, _ = wl.src.device_tables(dev)
    d_k, d_v, _, _, _ = wl.dst.device_tables(dev)
    torch.cuda.synchronize()
    s_str = [x * eb for x in wl.src.strides]
    d_str = [x * eb for x in wl.dst.strides]
    src_blocks, dst_blocks = wl.src.first.shape[0], wl.dst.first.shape[0]
    need = -(-n // 16)
    assert need <= len(st_np) and need <= len(dt_np)
    st_dev = torch.from_numpy(st_np).to(dev)
    dt_dev = torch.from_numpy(dt_np).to(dev)
    args = (s_k, s_v, d_k, d_v, layers, st_dev.data_ptr(), st_dev.numel(), src_blocks,
            dt_dev.data_ptr(), dt_dev.numel(), dst_blocks, n, heads, d * eb, *s_str, *d_str)

    zeros = torch.zeros(16, dtype=torch.int32, device=dev)  # the K stores' read table

    def launch():
        if ex is not None:
            rc = lib.ceil_paged_copy_ex(*args, ex[0], zeros.data_ptr() if ex[1] else None, st)
        elif lanes_scope is None:
            rc = lib.ceil_paged_copy(*args, st)
        else:
            rc = lib.ceil_paged_copy_lanes(*args, lanes_scope, st)
        if rc != 0:
            raise RuntimeError(f"{name}: the copy kernel returned {rc}")

    ms = _time_launch(launch, runs, stream)
    for _ in range(32):  # sampled rows: the destination row is the source row
        pos, layer = int(rng.integers(n)), int(rng.integers(layers))
        sb, db, off = int(st_np[pos // 16]), int(dt_np[pos // 16]), pos % 16
        want = wl.src.fused(0, layer, (sb, off))  # [heads, 2D]
        got = wl.dst.caches[0][layer][db, :, off]
        if not torch.equal(want.contiguous().view(torch.uint8),
                           got.contiguous().view(torch.uint8)):
            raise AssertionError(f"{name}: row {pos} layer {layer}")
    moved = 2 * n * layers * heads * 2 * d * eb
    gbs = moved / (ms / 1e3) / 1e9
    return {"bytes": moved, "ms": round(ms, 4), "GB_s": round(gbs, 1),
            "frac_of_peak": round(gbs / PEAK_GBS, 4),
            "blocks_kb": 16 * heads * 2 * d * eb / 1024}


def dst_layouts(dev, steps: int, warmup: int, stream) -> dict:
    """Informational: the headline shift into each paged-cache layout the connector
    takes -- fused HND (the headline), fused NHD, and K/V split into planes as
    ``[2, blocks, 16, heads, D]`` and ``[blocks, 2, 16, heads, D]``."""
    import numpy as np
    import torch

    from marathon_amd import workloads as W
    from marathon_amd.spans import CacheSet, ShiftPlan

    wl = W.qwen3_14b_multispan(dev)
    nblk, layers = wl.dst.first.shape[0], wl.layers
    heads, d = wl.dst.heads, wl.dst.head_size
    dst_hnd = wl.dst
    wl.dst = None

    def run(dst):
        plan = ShiftPlan(wl.spans, wl.src, dst, inv_freq=wl.inv_freq, src_mode=wl.src_mode,
                         src_index=wl.src_index, dst_mode=wl.dst_mode, dst_index=wl.dst_index)
        warm_up(lambda: plan.launch(stream.cuda_stream))
        _, per = time_plan(plan, max(steps, 50), warmup, stream)
        ms = float(np.median(per))
        gbs = plan.algorithmic_bytes / (ms / 1e3) / 1e9
        return {"ms": round(ms, 4), "GB_s": round(gbs, 1), "frac_of_peak": round(gbs / PEAK_GBS, 4)}

    out = {"fused_hnd": run(dst_hnd)}
    del dst_hnd
    torch.cuda.empty_cache()
    nhd = [torch.zeros(nblk, 16, heads, 2 * d, dtype=torch.bfloat16, device=dev)
           for _ in range(layers)]
    out["fused_nhd"] = run(CacheSet([nhd], "nhd", 16))
    del nhd
    torch.cuda.empty_cache()
    for axis, name in ((0, "split_2_blocks_bs_heads_d"), (1, "split_blocks_2_bs_heads_d")):
        shape = (2, nblk, 16, heads, d) if axis == 0 else (nblk, 2, 16, heads, d)
        caches = [torch.zeros(shape, dtype=torch.bfloat16, device=dev) for _ in range(layers)]
        out[name] = run(CacheSet([[c.select(axis, 0) for c in caches]], "nhd", 16,
                                 v_caches=[[c.select(axis, 1) for c in caches]]))
        del caches
        torch.cuda.empty_cache()
    del wl
    torch.cuda.empty_cache()
    return out


def src_layouts(dev, steps: int, warmup: int, stream) -> dict:
    """Informational: the headline shift (bf16 and fp8) from each block layout of the
    session store -- K and V planes per block, ``[blocks, 2, 16, heads, D]``, and rows of
    K then V per head, ``[blocks, 16, heads, 2D]`` -- the same values, blocks and tables;
    the two launches alternate over 5 rounds (the best round's median of each).  The
    block store keeps planes for 2- and 4-byte elements and rows for fp8."""
    import torch

    from marathon_amd import workloads as W

    out = {}
    for dt, make in (("bf16", W.qwen3_14b_multispan), ("fp8", W.qwen3_14b_multispan_fp8)):
        wls = {layout: make(dev, src_layout=layout) for layout in ("planes", "fused")}
        plans = {layout: wl.plan() for layout, wl in wls.items()}
        for plan in plans.values():
            warm_up(lambda: plan.launch(stream.cuda_stream))
        best = _ab(plans, max(steps, 50), warmup, stream, rounds=5)
        for layout, ms in best.items():
            gbs = plans[layout].algorithmic_bytes / (ms / 1e3) / 1e9
            out[f"{layout}_{dt}"] = {"ms": round(ms, 4), "GB_s": round(gbs, 1),
                                     "frac_of_peak": round(gbs / PEAK_GBS, 4)}
        del wls, plans
        torch.cuda.empty_cache()
    return out


def src_block_sizes(dev, steps: int, warmup: int, stream) -> dict:
    """Tokens per session-store block, the store's own choice (the destination keeps
    vLLM's 16-token blocks): the Qwen3-14B multi-span shift in bf16 and fp8, and its fp8
    one-KV-head share (tensor parallelism 8), from store blocks of 16, 32 and 64 tokens
    through shuffled tables; the launches alternate over 5 rounds (the best round's
    median of each), and sampled rows of each are checked against the oracle."""
    import torch

    from marathon_amd import workloads as W

    out = {}
    cases = (("bf16", W.qwen3_14b_multispan, {}), ("fp8", W.qwen3_14b_multispan_fp8, {}),
             ("fp8_1_head", W.qwen3_14b_multispan_fp8, {"heads": 1}))
    for name, make, kw in cases:
        wls = {blk: make(dev, src_block=blk, **kw) for blk in (16, 32, 64)}
        plans = {blk: wl.plan() for blk, wl in wls.items()}
        for plan in plans.values():
            warm_up(lambda: plan.launch(stream.cuda_stream))
        best = _ab(plans, max(steps, 50), warmup, stream, rounds=5)
        for blk, ms in best.items():
            gbs = plans[blk].algorithmic_bytes / (ms / 1e3) / 1e9
            row = {"ms": round(ms, 4), "GB_s": round(gbs, 1),
                   "frac_of_peak": round(gbs / PEAK_GBS, 4),
                   "store_block_kb": blk * wls[blk].dst.heads * 2 * 128
                   * wls[blk].dst.first.element_size() // 1024}
            if name == "bf16":
                row["rows_checked"] = spot_check(wls[blk], rows=32, seed=blk)
            out[f"{name}_store_block_{blk}"] = row
        del wls, plans
        torch.cuda.empty_cache()
    return out


def _same_output(a_plan, b_plan, caches) -> bool:
    """Run two plans of one workload into zeroed caches; whether every byte matches."""
    import torch

    for c in caches:
        c.zero_()
    a_plan.launch()
    torch.cuda.synchronize()
    first = [c.clone() for c in caches]
    for c in caches:
        c.zero_()
    b_plan.launch()
    torch.cuda.synchronize()
    return all(torch.equal(x.view(torch.uint8), y.view(torch.uint8))
               for x, y in zip(first, caches))


def _ab(plans: dict, steps: int, warmup: int, stream, rounds: int = 3) -> dict:
    """Median launch time of each plan (HIP events), each plan's launches back to back,
    the plans alternating over ``rounds``; the best round's median per plan."""
    import numpy as np

    best = {name: float("inf") for name in plans}
    for _ in range(rounds):
        for name, plan in plans.items():
            _, per = time_plan(plan, steps, warmup, stream)
            best[name] = min(best[name], float(np.median(per)))
    return best


def plan_variants(dev, steps: int, warmup: int, stream) -> dict:
    """A/B of the plan options, each pair on one workload with byte-identical output.

    * ``record_order``: the two-launch path's token records in span order against
      destination-page order (records sorted by the 2 MB page of the destination row),
      sorted on the host (``dst_page``: the plan's ``token_order``, no extra launch) and
      on the device (``dst_page_device``: an ordered plan pass and one more small
      launch), on the fp8 and bf16 Qwen3-14B multi-span shifts, the fp8 one from 64-token
      store blocks, and one GPU's fp8 share at 1 KV head; ``host_order_ms`` is what
      computing the host order adds to building the plan.
    * ``direct``: the single-launch path (token prefix and rotation tables from the
      host, no plan pass or workspace) against the two-launch path, for one span of
      16 to 2,048 tokens x 40 layers (flat store -> HND paged cache through shuffled
      slots, delta 186).  ``ShiftPlan`` takes the direct path by default up to
      ``DIRECT_MAX_TOKEN_LAYERS`` token-layers.
    * ``span_count``: one shift of 16,384 tokens x 40 layers cut into 1, 64 or 4,096
      spans (the plan pass builds the span prefix in every workgroup).
    """
    import torch

    from marathon_amd import spans as S
    from marathon_amd import workloads as W
    from marathon_amd.shift_kernels import inv_freq_for

    out = {"record_order": {}, "direct": {"default_max_token_layers":
                                          S.DIRECT_MAX_TOKEN_LAYERS}}
    for name, make in (("qwen3_14b_multispan_fp8", lambda: W.qwen3_14b_multispan_fp8(dev)),
                       ("qwen3_14b_multispan_fp8_store_block_64",
                        lambda: W.qwen3_14b_multispan_fp8(dev, src_block=64)),
                       ("qwen3_14b_multispan_bf16", lambda: W.qwen3_14b_multispan(dev)),
                       ("qwen3_14b_multispan_fp8_1_head",
                        lambda: W.qwen3_14b_multispan_fp8(dev, heads=1))):
        log(f"record order A/B: {name}")
        wl = make()
        build_ms = {}
        for order in ("none", "dst_page") * 3:  # the first builds carry one-time costs
            t0 = time.perf_counter()
            wl.plan(direct=False, order=order)
            ms_ = (time.perf_counter() - t0) * 1e3
            build_ms[order] = min(build_ms.get(order, ms_), ms_)
        plans = {"none": wl.plan(direct=False, order="none"),
                 "dst_page": wl.plan(direct=False, order="dst_page"),
                 "dst_addr": wl.plan(direct=False, order="dst_addr"),
                 "dst_page_device": wl.plan(direct=False, order="dst_page_device")}
        assert plans["dst_page"].order == "dst_page_host"
        same = all(_same_output(plans["none"], plans[k], wl.dst.caches[0])
                   for k in ("dst_page", "dst_addr", "dst_page_device"))
        warm_up(lambda: plans["none"].launch(stream.cuda_stream))
        ms = _ab(plans, max(steps, 30), warmup, stream, rounds=4)
        gb = plans["none"].algorithmic_bytes
        out["record_order"][name] = {
            **{f"{k}_ms": round(v, 4) for k, v in ms.items()},
            **{f"{k}_frac_of_peak": round(gb / (v / 1e3) / 1e9 / PEAK_GBS, 4)
               for k, v in ms.items()},
            "dst_page_gain_pct": round(100 * (ms["none"] / ms["dst_page"] - 1), 2),
            "dst_addr_gain_pct": round(100 * (ms["none"] / ms["dst_addr"] - 1), 2),
            "dst_page_device_gain_pct": round(100 * (ms["none"] / ms["dst_page_device"] - 1), 2),
            "host_order_ms": round(build_ms["dst_page"] - build_ms["none"], 3),
            "bit_identical": same,
        }
        del wl, plans
        torch.cuda.empty_cache()

    layers, heads, d, bs = 40, 8, 128, 16
    for n in (16, 64, 256, 512, 2048):
        gen = torch.Generator(device=dev)
        gen.manual_seed(n)
        blocks = -(-n // bs) + 8
        src = [torch.randn(n, heads, 2 * d, dtype=torch.bfloat16, device=dev, generator=gen)
               for _ in range(layers)]
        kv = [torch.zeros(blocks, heads, bs, 2 * d, dtype=torch.bfloat16, device=dev)
              for _ in range(layers)]
        table = torch.randperm(blocks, device=dev, generator=gen)
        pos = torch.arange(n, device=dev)
        slot = table[pos // bs] * bs + pos % bs
        src_set, dst_set = S.CacheSet([src], "flat"), S.CacheSet([kv], "hnd", bs)

        def make(direct):
            return S.ShiftPlan(S.span_array([(0, 0, 0, 0, n, 186, 0, 0)]), src_set, dst_set,
                               inv_freq=inv_freq_for(d, 1e6), src_mode="flat",
                               dst_mode="slots", dst_index=slot, direct=direct)

        plans = {"direct": make(True), "two_launch": make(False)}
        if not plans["direct"].direct:
            raise AssertionError("the direct path refused an eligible shift")
        same = _same_output(plans["direct"], plans["two_launch"], kv)
        warm_up(lambda: plans["direct"].launch(stream.cuda_stream))
        ms = _ab(plans, max(steps, 50), warmup, stream)
        gb = plans["direct"].algorithmic_bytes
        out["direct"][f"tokens_{n}"] = {
            "token_layers": n * layers,
            **{f"{k}_ms": round(v, 4) for k, v in ms.items()},
            **{f"{k}_frac_of_peak": round(gb / (v / 1e3) / 1e9 / PEAK_GBS, 4)
               for k, v in ms.items()},
            "bit_identical": same,
        }
        del src, kv, plans, src_set, dst_set
        torch.cuda.empty_cache()

    # the plan pass builds the span prefix in every workgroup: the same 16,384 tokens
    # x 40 layers cut into 1, 64 and 4,096 (the limit of one descriptor) spans, each
    # span with its own delta, flat store -> HND paged cache through shuffled slots
    n = 16384
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    blocks = -(-n // bs) + 8
    src = [torch.randn(n, heads, 2 * d, dtype=torch.bfloat16, device=dev, generator=gen)
           for _ in range(layers)]
    kv = [torch.zeros(blocks, heads, bs, 2 * d, dtype=torch.bfloat16, device=dev)
          for _ in range(layers)]
    table = torch.randperm(blocks, device=dev, generator=gen)
    pos = torch.arange(n, device=dev)
    slot = table[pos // bs] * bs + pos % bs
    src_set, dst_set = S.CacheSet([src], "flat"), S.CacheSet([kv], "hnd", bs)
    out["span_count"] = {"what": "16,384 tokens x 40 layers (bf16) in 1, 64 or 4,096 spans, "
                         "two-launch path; median launch time"}
    plans = {}
    for count in (1, 64, 4096):
        per = n // count
        rows = [(k * per, 0, 0, k * per, per, 186 + (k % 97), 0, 0) for k in range(count)]
        plans[f"spans_{count}"] = S.ShiftPlan(
            S.span_array(rows), src_set, dst_set, inv_freq=inv_freq_for(d, 1e6),
            src_mode="flat", dst_mode="slots", dst_index=slot, direct=False)
    warm_up(lambda: plans["spans_1"].launch(stream.cuda_stream))
    ms = _ab(plans, max(steps, 30), warmup, stream)
    gb = plans["spans_1"].algorithmic_bytes
    for name, v in ms.items():
        out["span_count"][name] = {"ms": round(v, 4),
                                   "frac_of_peak": round(gb / (v / 1e3) / 1e9 / PEAK_GBS, 4)}
    del src, kv, plans, src_set, dst_set
    torch.cuda.empty_cache()
    return out


def connector_step(dev, steps: int, warmup: int) -> dict:
    """Worker load steps through the connector: a session held in the block-layout store,
    loaded by ``ShiftLoader.start_load_kv`` with device-side slots (block tables, not
    slot lists) into an HND paged cache.  Times the whole call from Python (store
    checks, span table, one pinned upload, plan + shift kernels) to the stream's
    completion, next to the kernels alone on the same plan.  The steps: the Qwen3-14B
    multi-span workload's eight spans in bf16 and in fp8 e4m3 (per-layer K scales, as
    vLLM's ``_k_scale``), into a shuffled destination block table (a long-running
    engine's) and into an ascending one (a fresh engine's); and one 29,232-token bf16
    load, the size of the reference's in-engine measurement (docs/findings.md:664-666:
    34.4 ms copy_ms, 6.2 ms of it the kernel)."""
    import numpy as np
    import torch

    from marathon_amd import BlockShiftStore
    from marathon_amd import workloads as W
    from marathon_amd.connector import Load, ShiftLoader
    from marathon_amd.shift_kernels import inv_freq_for

    layers, heads, d, bs = 40, 8, 128, 16
    lay = W.qwen3_14b_multispan_layout()
    history = lay.src_history
    names = [f"layer{i}" for i in range(layers)]
    blocks = -(-max(lay.dst_history, history) // bs) + 8
    table = np.random.default_rng(1).permutation(blocks).astype(np.int32)
    out = {"what": "ShiftLoader.start_load_kv from a BlockShiftStore session into an HND "
           "paged cache (40 layers), block tables on the device; medians over steps",
           "reference_in_engine_copy_ms_29232_tokens": 34.4,
           "reference_kernel_ms_29232_tokens": 6.2}
    # a long-running engine's block tables are fragmented (shuffled here); a fresh
    # engine hands a request ascending blocks (the *_contiguous_dst cases)
    fresh = np.arange(blocks, dtype=np.int32)
    multi = lambda tab=table: [Load.from_blocks("s", tab, int(dst), int(dst) + int(n), int(dl))
                               for dst, n, dl in zip(lay.dst_start, lay.length, lay.delta)]
    for dtype, cases in (
        (torch.bfloat16, {"qwen3_14b_8_spans": multi,
                          "qwen3_14b_8_spans_contiguous_dst": lambda: multi(fresh),
                          "one_load_29232_tokens":
                              lambda: [Load.from_blocks("s", table, 0, 29232, -186)]}),
        (torch.float8_e4m3fn, {"qwen3_14b_8_spans_fp8": multi,
                               "qwen3_14b_8_spans_fp8_contiguous_dst": lambda: multi(fresh)}),
    ):
        gen = torch.Generator(device=dev)
        gen.manual_seed(0)
        fp8 = dtype == torch.float8_e4m3fn
        k_scales = {}
        if fp8:
            ks, _ = W.fp8_layer_scales(4, layers)  # the fp8 multi-span shift's scales
            k_scales = {name: float(k) for name, k in zip(names, ks)}
        store = BlockShiftStore(budget_tokens=32768, device=str(dev), block_size=bs)
        assert store.reserve("s", 0, history)
        for name in names:
            buf = store.write_target("s", name, 0, history, (heads, 2 * d), dtype, dev)
            x = torch.randn(buf.shape, dtype=torch.float32, device=dev, generator=gen)
            buf.copy_((x / k_scales[name]).clamp_(-448.0, 448.0) if fp8 else x)
            del x
        kv = {name: torch.zeros(blocks, heads, bs, 2 * d, dtype=dtype, device=dev)
              for name in names}
        loader = ShiftLoader(store, bs, inv_freq_for(d, 1e6), k_scales=k_scales)
        loader.register_kv_caches(kv)
        for case, loads in cases.items():
            for _ in range(warmup):
                loader.start_load_kv(loads())
            torch.cuda.synchronize()
            host, e2e = [], []
            for _ in range(steps):
                batch = loads()
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                loader.start_load_kv(batch)
                t1 = time.perf_counter()
                torch.cuda.synchronize()
                e2e.append((time.perf_counter() - t0) * 1e3)
                host.append((t1 - t0) * 1e3)
            plan = loader.last_plan
            _, per = time_plan(plan, steps, warmup, torch.cuda.current_stream(dev))
            time.sleep(0.005)  # an idle gap that separates the cases in a kernel trace
            kms = float(np.mean(per))
            out[case] = {
                "dtype": "fp8_e4m3" if fp8 else "bf16",
                "tokens": plan.tokens,
                "ms_end_to_end": round(float(np.median(e2e)), 4),
                "host_ms": round(float(np.median(host)), 4),
                "kernel_ms": round(kms, 4),
                "kernel_GB_s": round(plan.algorithmic_bytes / (kms / 1e3) / 1e9, 1),
                "kernel_frac_of_peak": round(plan.algorithmic_bytes / (kms / 1e3) / 1e9
                                             / PEAK_GBS, 4),
            }
        del store, kv, loader
        torch.cuda.empty_cache()
    return out


def save_step(dev, steps: int, warmup: int) -> dict:
    """The save path (paged cache -> block-layout store) through ``ShiftSaver.save_all``:
    an edit turn's one-shot ``save="full"`` re-gather of a 29,232-token prompt over 40
    layers, and a decode step's one-token save (vllm_shift_connector.py:296-330,
    :539-553).  Block tables on the device; whole call to stream completion, next to the
    kernels alone."""
    import numpy as np
    import torch

    from marathon_amd import BlockShiftStore
    from marathon_amd.connector import Save, ShiftSaver

    layers, heads, d, bs, n = 40, 8, 128, 16, 29232
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    blocks = -(-n // bs) + 8
    names = [f"layer{i}" for i in range(layers)]
    kv = {name: torch.randn(blocks, heads, bs, 2 * d, dtype=torch.bfloat16, device=dev,
                            generator=gen) for name in names}
    # the same cache in fp8 e4m3 (a save copies bytes: no K scale is involved)
    kv8 = {name: (t.float() * 16).clamp(-448, 448).to(torch.float8_e4m3fn)
           for name, t in kv.items()}
    table = np.random.default_rng(2).permutation(blocks).astype(np.int32)
    store = BlockShiftStore(budget_tokens=32768, device=str(dev), block_size=bs)
    store8 = BlockShiftStore(budget_tokens=32768, device=str(dev), block_size=bs)
    saver = ShiftSaver(store, bs)
    saver8 = ShiftSaver(store8, bs)
    out = {"what": "ShiftSaver.save_all from an HND paged cache (40 layers, bf16; fp8 e4m3 "
           "where named) into a BlockShiftStore session, block tables on the device; "
           "medians over steps"}
    cases = {"full_prompt_29232_tokens": (kv, saver, lambda: [Save.from_blocks("s", table, 0, n)]),
             "decode_step_1_token": (kv, saver,
                                     lambda: [Save.from_blocks("s", table, n - 1, n)]),
             "full_prompt_29232_tokens_fp8": (kv8, saver8,
                                              lambda: [Save.from_blocks("s", table, 0, n)]),
             "decode_step_1_token_fp8": (kv8, saver8,
                                         lambda: [Save.from_blocks("s", table, n - 1, n)])}
    for case, (kv_c, saver_c, saves) in cases.items():
        for _ in range(warmup):
            saver_c.save_all(kv_c, saves())
        torch.cuda.synchronize()
        e2e, host = [], []
        for _ in range(steps):
            batch = saves()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            saver_c.save_all(kv_c, batch)
            t1 = time.perf_counter()
            torch.cuda.synchronize()
            e2e.append((time.perf_counter() - t0) * 1e3)
            host.append((t1 - t0) * 1e3)
        plan = saver_c.last_plan
        _, per = time_plan(plan, steps, warmup, torch.cuda.current_stream(dev))
        kms = float(np.mean(per))
        out[case] = {
            "tokens": plan.tokens,
            "ms_end_to_end": round(float(np.median(e2e)), 4),
            "host_ms": round(float(np.median(host)), 4),
            "kernel_ms": round(kms, 4),
            "kernel_GB_s": round(plan.algorithmic_bytes / (kms / 1e3) / 1e9, 1),
        }
    # vLLM's per-layer hook for a decode step: 40 save_kv_layer calls, each its own
    # launch (as the reference saves), or deferred to one launch in wait_for_save
    for case, deferred in (("decode_step_40_layer_hooks", False),
                           ("decode_step_40_layer_hooks_deferred", True)):
        hook = ShiftSaver(store, bs, deferred=deferred)

        def one_step():
            saves = [Save.from_blocks("s", table, n - 1, n)]
            for name in names:
                hook.save_kv_layer(name, kv[name], saves)
            hook.wait_for_save()

        for _ in range(warmup):
            one_step()
        torch.cuda.synchronize()
        e2e = []
        for _ in range(steps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            one_step()
            torch.cuda.synchronize()
            e2e.append((time.perf_counter() - t0) * 1e3)
        out[case] = {"tokens": 1, "ms_end_to_end": round(float(np.median(e2e)), 4)}
    del store, kv, saver, store8, kv8, saver8
    torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-reference-shape", action="store_true")
    ap.add_argument("--no-reference-loop", action="store_true",
                    help="skip the reference benchmark's per-layer scatter_shifted loop")
    ap.add_argument("--no-other-workloads", "--no-other-configs", dest="no_other_workloads",
                    action="store_true",
                    help="skip the informational timings of the Qwen3-8B single-span, fp8 "
                    "multi-span and batched-session workloads")
    ap.add_argument("--no-tp-shares", action="store_true",
                    help="skip the timings of one GPU's share at 4, 2 and 1 KV heads")
    ap.add_argument("--no-session-batches", action="store_true",
                    help="skip the batched-sessions shift's other forms (16 sessions, fp8, "
                    "one KV head)")
    ap.add_argument("--no-size-sweep", action="store_true",
                    help="skip the batched shifts of 512 to 32,768 tokens")
    ap.add_argument("--no-ceilings", action="store_true",
                    help="skip the plain elementwise copy and the identity-table headline")
    ap.add_argument("--no-dst-layouts", action="store_true",
                    help="skip the headline shift into the other paged-cache layouts")
    ap.add_argument("--no-src-layouts", action="store_true",
                    help="skip the headline shift from the store's other block layout")
    ap.add_argument("--no-src-block-sizes", action="store_true",
                    help="skip the A/B of 16-, 32- and 64-token store blocks")
    ap.add_argument("--no-connector-step", action="store_true",
                    help="skip the end-to-end connector load and save step timings")
    ap.add_argument("--no-plan-variants", action="store_true",
                    help="skip the A/B of record order and of the direct path")
    ap.add_argument("--only", default="",
                    help="comma-separated informational sections to run (e.g. "
                    "'plan_variants'; 'headline' for none); every other one, the CPU "
                    "baseline included, is skipped")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 1 GiB device copy (for PMC counter scaling)")
    args = ap.parse_args()
    if args.only:
        keep = {x.strip() for x in args.only.split(",") if x.strip()}
        sections = {"reference_shape", "reference_loop", "other_workloads", "tp_shares",
                    "session_batches", "size_sweep", "ceilings", "dst_layouts", "src_layouts", "src_block_sizes",
                    "connector_step", "plan_variants", "cpu_baseline"}
        if keep - sections - {"headline"}:  # "headline": the headline line alone
            ap.error(f"--only: unknown sections {sorted(keep - sections)}")
        for name in sections - keep:
            setattr(args, "no_" + name, True)
    if args.gpus != 1:
        print(
            "bench.py measures one GPU: the shift needs no collective and this library runs on "
            "a single MI355X (per-rank sharding is by KV head / layer / session with no "
            "exchange).  Run with --gpus 1.",
            file=sys.stderr,
        )
        return 2

    import numpy as np
    import torch

    from marathon_amd import workloads as W

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    log("building the Qwen3-14B multi-span workload (40 layers, 30,720-token history, 8 spans)")
    wl = W.qwen3_14b_multispan(dev)
    plan = wl.plan()
    torch.cuda.synchronize()
    log(f"spans={len(wl.spans)} tokens={wl.tokens} bytes={plan.algorithmic_bytes}")

    if args.copy_calibration:
        # a plain elementwise kernel of known traffic: reads 1 GiB, writes 1 GiB (a
        # same-dtype copy_ would go to the DMA engine and show no kernel counters)
        a = torch.zeros(1 << 28, dtype=torch.float32, device=dev)
        b = torch.empty_like(a)
        for _ in range(3):
            torch.neg(a, out=b)
        torch.cuda.synchronize()
        log("copy calibration: 3 x elementwise 1 GiB -> 1 GiB kernel done")
        del a, b

    wall, per = time_plan(plan, args.steps, args.warmup, stream)
    checked = spot_check(wl)
    log(f"spot check: {checked} sampled rows bit-identical to the oracle")
    ms_step = wall / args.steps * 1e3
    bytes_step = plan.algorithmic_bytes
    value = bytes_step * args.steps / wall / 1e9
    ev_ms = float(np.mean(per))
    achieved = bytes_step / (ev_ms / 1e3) / 1e9
    metadata = plan.metadata_bytes
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("traffic_bytes_per_launch")

    extra = {}
    side_steps = max(5, min(args.steps, 20))  # the informational sections
    del wl, plan  # the headline workload's caches make room for the other sections
    torch.cuda.empty_cache()
    if not args.no_reference_shape:
        log("reference benchmark shape (30,720 x 40, delta 186)")
        extra["reference_shape"] = reference_shape(dev, side_steps, args.warmup, stream)
    if not args.no_reference_loop:
        log("reference benchmark loop (40 x scatter_shifted, 4,096 / 12,288 / 30,720 tokens)")
        extra["reference_loop"] = reference_loop(dev)
    if not args.no_other_workloads:
        extra["other_workloads"] = other_workloads(dev, side_steps, args.warmup,
                                                   stream)
    if not args.no_tp_shares:
        log("tensor-parallel shares of the headline shift (4, 2, 1 KV heads)")
        extra["tp_shares"] = tp_shares(dev, side_steps, args.warmup, stream)
    if not args.no_session_batches:
        log("batched sessions: 16 sessions, fp8, one KV head")
        extra["session_batches"] = session_batches(dev, side_steps, args.warmup, stream)
    if not args.no_size_sweep:
        log("size sweep: one batched shift of 512 to 32,768 tokens x 40 layers")
        extra["size_sweep"] = size_sweep(dev, side_steps, args.warmup, stream)
    if not args.no_ceilings:
        log("ceilings: elementwise copy, the headline with identity tables")
        extra["ceilings"] = ceilings(dev, side_steps, args.warmup, stream)
        log("ceilings: hand-written stream and paged copies of the headline's bytes")
        extra["ceilings"].update(copy_ceilings(dev, side_steps, args.warmup, stream))
    if not args.no_dst_layouts:
        log("destination layouts (fused HND / NHD, split K/V planes)")
        extra["dst_layouts"] = dst_layouts(dev, side_steps, args.warmup, stream)
    if not args.no_src_layouts:
        log("store block layouts (K/V planes, fused rows), bf16 and fp8")
        extra["src_layouts"] = src_layouts(dev, side_steps, args.warmup, stream)
    if not args.no_src_block_sizes:
        log("store block sizes (16, 32, 64 tokens), bf16, fp8, fp8 one head")
        extra["src_block_sizes"] = src_block_sizes(dev, side_steps, args.warmup, stream)
    if not args.no_connector_step:
        log("connector load step (block store, device-side slots)")
        extra["connector_step"] = connector_step(dev, side_steps, args.warmup)
        log("connector save step (paged -> block store)")
        extra["save_step"] = save_step(dev, side_steps, args.warmup)
    if not args.no_plan_variants:
        log("plan variants: record order and direct path A/B")
        extra["plan_variants"] = plan_variants(dev, side_steps, args.warmup, stream)
    small = cpu = None
    if not args.no_cpu_baseline:
        log("Qwen3-0.6B shift on the HIP path (the CPU baseline's small case)")
        small, small_out = qwen3_0_6b_hip(dev, side_steps, args.warmup, stream,
                                          keep_outputs=True)
        log("cpu baseline (reference torch path on the host, the Qwen3-14B multi-span shift)")
        cpu = cpu_baseline(gpu_small=small, small_gpu_out=small_out)
        del small_out

    tokens = int(bytes_step // (2 * 40 * 8 * 256 * 2))
    line = {
        "metric": "fused KV-shift HBM GB/s (% of 8 TB/s peak) and ms per 30k-token shift, 1 GPU",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "arithmetic": "K rotated in fp32 (mul, mul, add, no FMA) and rounded to bf16 (RNE); "
        "V copied as raw bytes",
        "data": "synthetic: K/V ~ N(0,1) bf16 drawn on device (seed 3), shuffled block tables",
        "config": {
            "workload": "qwen3-14b multi-span shift: 40 layers, 8 kv heads, head_dim 128, "
            "30,720-token history, 8 spans (seed 3), session store blocks (K and V "
            "planes, shuffled table) -> HND paged cache (slots)",
            "tokens_shifted": tokens,
            "layers": 40,
            "spans": 8,
            "bytes_per_step": bytes_step,
        },
        "build_defines": build_defines(),
        "frac_of_peak": round(value / PEAK_GBS, 4),
        "tokens_per_s": round(tokens / (ms_step / 1e3), 1),
        "us_per_token": round(ms_step * 1e3 / tokens, 5),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_GBS, 4),
            "traffic": traffic,
            "kernel_ms": round(ev_ms, 4),
            # not in `achieved`: span and index arrays, rotation tables, token records
            "metadata_bytes": metadata,
        },
        "cpu_baseline": cpu,
        "qwen3_0_6b_shift_hip": small,
        "parity": f"{checked} sampled rows bit-identical to the oracle after timing",
        # config 1's K (every shifted element, 28 layers) against the reference's torch
        # path on the CPU: this package's tables and the reference's own
        "k_vs_torch_path_qwen3_0_6b": None if cpu is None else
        cpu["qwen3_0_6b_4096_tokens"].get("k_vs_torch_path"),
        **extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
