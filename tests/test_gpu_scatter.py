"""Single-span ``scatter_shifted`` on the GPU against the oracle and the reference path.

Geometry follows the reference's kernel test (tests/test_shift_kernels.py:46-90): 8 KV
heads, head_size 128, block 16, 64 blocks, a scattered ``randperm`` block table, a run
starting at position 3, n in {64, 37} (ragged), both paged layouts, the same deltas.
The bar here is stricter than the reference's own: bit-identical to the oracle (same
fp32 op order, same correctly rounded cos/sin), and within 1 bf16 ulp of the reference's
torch op sequence with torch's CPU tables.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from marathon_amd import rope_shift, scatter_shifted
from oracle import kvshift_oracle as orc
from oracle import torch_path
from tests.helpers import bits, dname, inv_freq, randn, ulp_bf16

pytestmark = pytest.mark.gpu

DELTAS = [-3000, -4, 0, 4, 186, 10000]


def _case(seed, n, hnd, dtype=torch.bfloat16, heads=8, d=128, bs=16, nblocks=64, start=3):
    g = torch.Generator().manual_seed(seed)
    src = randn((n, heads, 2 * d), dtype, g, 0.05)
    shape = (nblocks, heads, bs, 2 * d) if hnd else (nblocks, bs, heads, 2 * d)
    kv = randn(shape, dtype, g, 0.05)
    table = torch.randperm(nblocks, generator=g)[: -(-(n + start) // bs) + 1]
    pos = torch.arange(start, start + n)
    slots = table[pos // bs] * bs + pos % bs
    return src, kv, slots


def _run_gpu(dev, src, kv, slots, bs, hnd, shift, **kw):
    kv_dev = kv.to(dev)
    scatter_shifted(src.to(dev), kv_dev, slots.to(dev), bs, hnd, shift, **kw)
    torch.cuda.synchronize(dev)
    return kv_dev


@pytest.mark.parametrize("delta", DELTAS)
@pytest.mark.parametrize("hnd", [True, False])
@pytest.mark.parametrize("n", [64, 37])
def test_bf16_matches_oracle_and_reference_path(gpu, delta, hnd, n):
    print(f"case bf16 delta={delta} hnd={hnd} n={n}", flush=True)
    src, kv, slots = _case(delta * 7 + n, n, hnd)
    inv = inv_freq()
    got = bits(_run_gpu(gpu, src, kv, slots, 16, hnd, rope_shift(delta, 128, inv, gpu)))

    want = bits(kv)
    orc.scatter_shifted(bits(src), want, slots.numpy(), 16, hnd, delta, inv.numpy(), "bf16")
    assert np.array_equal(got, want), f"{int((got != want).sum())} elements differ from the oracle"

    # the reference's torch op sequence with torch's own CPU tables
    ref = kv.clone()
    emb = torch_path.rope_emb_tables(delta, inv) if delta else None
    torch_path.shift_into_paged(src, ref, slots, 16, hnd, emb)
    ref_bits = bits(ref)
    assert int(ulp_bf16(got, ref_bits).max()) <= 1
    # and the reference test's own bounds (tests/test_shift_kernels.py:75-78)
    gf = orc.bf16_to_f32(got)
    rf = orc.bf16_to_f32(ref_bits)
    assert float(np.abs(gf - rf).max()) <= 2**-7 * float(src.float().abs().max())
    assert float((ulp_bf16(got, ref_bits) > 1).mean()) < 1e-3


@pytest.mark.parametrize("tables_on", ["cpu", "gpu"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("hnd", [True, False])
def test_reference_tables_reproduce_the_reference_path_bit_for_bit(gpu, tables_on, dtype, hnd):
    """The drop-in as a caller keeping the reference's ``rope_shift`` would use it: the
    reference's own tables (torch fp32 cos/sin, built on the CPU or, as the connector
    builds them, on the GPU; shift_kernels.py:68-84) through ``mkv_scatter_shifted``
    give exactly the bits of the reference's torch op sequence with the same tables
    (shift_kernels.py:141-159): 0 ulp, every element, every delta."""
    from marathon_amd import RopeShift

    inv = inv_freq()
    for n, delta in ((64, -3000), (37, -4), (64, 4), (37, 186), (64, 10000), (37, -566)):
        print(f"case reference tables on {tables_on} {dtype} hnd={hnd} n={n} delta={delta}",
              flush=True)
        src, kv, slots = _case(abs(delta) + n, n, hnd, dtype)
        t = torch_path.rope_shift_tables(delta, 128, inv, "cpu" if tables_on == "cpu" else gpu)
        shift = RopeShift(delta, t["cos"].to(gpu), t["sgn"].to(gpu), None, t["emb_cos"],
                          t["emb_sin"], inv.to(gpu), 128)
        got = bits(_run_gpu(gpu, src, kv, slots, 16, hnd, shift))
        ref = kv.clone()
        torch_path.shift_into_paged(src, ref, slots, 16, hnd,
                                    (t["emb_cos"].cpu(), t["emb_sin"].cpu()))
        want = bits(ref)
        assert np.array_equal(got, want), (
            f"{int((got != want).sum())} of {want.size} elements differ from the torch path")


def test_zero_length_load_is_a_noop(gpu):
    kv = torch.randn(4, 8, 16, 256, dtype=torch.bfloat16, device=gpu)
    before = kv.clone()
    src = torch.empty(0, 8, 256, dtype=torch.bfloat16, device=gpu)
    slots = torch.empty(0, dtype=torch.int64, device=gpu)
    scatter_shifted(src, kv, slots, 16, True, rope_shift(4, 128, inv_freq(), gpu))
    torch.cuda.synchronize(gpu)
    assert torch.equal(kv, before)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("delta", [-1133, 0, 6759])
def test_other_float_dtypes_match_oracle(gpu, dtype, delta):
    print(f"case {dtype} delta={delta}", flush=True)
    src, kv, slots = _case(11 + delta, 45, False, dtype=dtype)
    inv = inv_freq()
    got = bits(_run_gpu(gpu, src, kv, slots, 16, False, rope_shift(delta, 128, inv, gpu)))
    want = bits(kv)
    orc.scatter_shifted(bits(src), want, slots.numpy(), 16, False, delta, inv.numpy(), dname(dtype))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("d,rotary", [(128, 64), (256, 64), (64, 64), (256, 256)])
def test_partial_rotary_and_other_head_sizes(gpu, d, rotary):
    print(f"case d={d} rotary={rotary}", flush=True)
    src, kv, slots = _case(5 + d + rotary, 50, True, d=d)
    inv = inv_freq(rotary)
    got = bits(_run_gpu(gpu, src, kv, slots, 16, True, rope_shift(-566, d, inv, gpu)))
    want = bits(kv)
    orc.scatter_shifted(bits(src), want, slots.numpy(), 16, True, -566, inv.numpy(), "bf16")
    assert np.array_equal(got, want)


@pytest.mark.parametrize("heads", [1, 2, 5, 8, 16])
def test_head_counts(gpu, heads):
    """TP shards hold 8/TP heads (one at TP=8); odd counts exercise ragged waves."""
    print(f"case heads={heads}", flush=True)
    src, kv, slots = _case(100 + heads, 41, heads % 2 == 0, heads=heads)
    inv = inv_freq()
    hnd = heads % 2 == 0
    got = bits(_run_gpu(gpu, src, kv, slots, 16, hnd, rope_shift(17, 128, inv, gpu)))
    want = bits(kv)
    orc.scatter_shifted(bits(src), want, slots.numpy(), 16, hnd, 17, inv.numpy(), "bf16")
    assert np.array_equal(got, want)


@pytest.mark.parametrize("bs", [1, 8, 32, 24])
def test_block_sizes(gpu, bs):
    print(f"case block_size={bs}", flush=True)
    src, kv, slots = _case(200 + bs, 70, False, bs=bs, nblocks=max(16, 160 // bs))
    inv = inv_freq()
    got = bits(_run_gpu(gpu, src, kv, slots, bs, False, rope_shift(-17, 128, inv, gpu)))
    want = bits(kv)
    orc.scatter_shifted(bits(src), want, slots.numpy(), bs, False, -17, inv.numpy(), "bf16")
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dtype,heads,d,rotary,hnd", [
    (torch.bfloat16, 2, 512, 512, True),       # a K row fills a whole wave (64 chunks)
    (torch.float32, 4, 256, 256, False),       # fp32: a K row fills a whole wave
    (torch.bfloat16, 64, 128, 128, True),      # one token is 8 passes of a workgroup
    (torch.float16, 32, 64, 64, False),        # 8 rows per wave, 2 passes per token
    (torch.float8_e4m3fn, 8, 64, 64, False),   # fp8: 16 rows per wave span two tokens
    (torch.float8_e4m3fn, 3, 256, 128, True),  # fp8: ragged heads, partial rotary
])
def test_geometry_limits(gpu, dtype, heads, d, rotary, hnd):
    """The largest head size (512), rows that fill a whole wave, many heads (one token
    over several passes) and waves whose rows span tokens, in every element type."""
    print(f"case geometry {dtype} heads={heads} d={d} rotary={rotary} hnd={hnd}", flush=True)
    g = torch.Generator().manual_seed(heads * 1000 + d + rotary)
    scale, n, nblocks, delta = 0.05, 37, 16, -301
    src = randn((n, heads, 2 * d), dtype, g, scale)
    shape = (nblocks, heads, 16, 2 * d) if hnd else (nblocks, 16, heads, 2 * d)
    kv = randn(shape, dtype, g, scale)
    table = torch.randperm(nblocks, generator=g)
    pos = torch.arange(7, 7 + n)
    slots = table[pos // 16] * 16 + pos % 16
    inv = inv_freq(rotary)
    fp8 = dtype == torch.float8_e4m3fn
    got = bits(_run_gpu(gpu, src, kv, slots, 16, hnd, rope_shift(delta, d, inv, gpu),
                        **({"k_scale": scale} if fp8 else {})))
    want = bits(kv)
    orc.scatter_shifted(bits(src), want, slots.numpy(), 16, hnd, delta, inv.numpy(),
                        dname(dtype), **({"k_scale": np.float32(scale)} if fp8 else {}))
    assert np.array_equal(got, want), f"{int((got != want).sum())} elements differ"


@pytest.mark.parametrize("dtype,heads,d,rotary,hnd", [
    (torch.bfloat16, 1, 128, 128, True),       # 4 tokens per wave pass
    (torch.bfloat16, 2, 128, 128, False),      # 2 tokens per pass
    (torch.bfloat16, 1, 64, 64, False),        # 8 tokens per pass
    (torch.bfloat16, 2, 64, 32, True),         # 4 tokens per pass, partial rotary
    (torch.float16, 2, 128, 128, True),
    (torch.float32, 1, 128, 64, False),        # fp32: 2 rows per wave, 2 tokens
    (torch.float8_e4m3fn, 1, 128, 128, True),  # fp8: 8 tokens per pass
    (torch.float8_e4m3fn, 2, 128, 64, False),  # fp8: 4 tokens per pass, partial rotary
    (torch.float8_e4m3fn, 4, 128, 128, True),  # fp8: 2 tokens per pass
])
@pytest.mark.parametrize("n", [37, 300])
def test_multi_token_passes(gpu, dtype, heads, d, rotary, hnd, n):
    """Head counts that divide a wave's rows: a wave pass covers several whole tokens.
    Ragged tails (37 and 300 tokens are not multiples of any tile) and every element
    type, against the oracle."""
    print(f"case multi-token {dtype} heads={heads} d={d} rotary={rotary} hnd={hnd} n={n}",
          flush=True)
    g = torch.Generator().manual_seed(heads * 7919 + d + rotary + n)
    scale, nblocks, delta = 0.05, 24, 1187
    src = randn((n, heads, 2 * d), dtype, g, scale)
    shape = (nblocks, heads, 16, 2 * d) if hnd else (nblocks, 16, heads, 2 * d)
    kv = randn(shape, dtype, g, scale)
    table = torch.randperm(nblocks, generator=g)
    pos = torch.arange(9, 9 + n)
    slots = table[pos // 16] * 16 + pos % 16
    inv = inv_freq(rotary)
    fp8 = dtype == torch.float8_e4m3fn
    got = bits(_run_gpu(gpu, src, kv, slots, 16, hnd, rope_shift(delta, d, inv, gpu),
                        **({"k_scale": scale} if fp8 else {})))
    want = bits(kv)
    orc.scatter_shifted(bits(src), want, slots.numpy(), 16, hnd, delta, inv.numpy(),
                        dname(dtype), **({"k_scale": np.float32(scale)} if fp8 else {}))
    assert np.array_equal(got, want), f"{int((got != want).sum())} elements differ"


@pytest.mark.parametrize("delta", [131071, -1048577, 16777219, 2**31 - 1, -(2**31)])
def test_extreme_deltas_match_oracle(gpu, delta):
    """int32 extremes and deltas beyond 2^24 (rounded to fp32 before the product, as
    torch rounds the reference's Python scalar): bit-exact against the oracle."""
    print(f"case extreme delta={delta}", flush=True)
    src, kv, slots = _case(abs(delta) % 1000, 53, True)
    inv = inv_freq()
    got = bits(_run_gpu(gpu, src, kv, slots, 16, True, rope_shift(delta, 128, inv, gpu)))
    want = bits(kv)
    orc.scatter_shifted(bits(src), want, slots.numpy(), 16, True, delta, inv.numpy(), "bf16")
    assert np.array_equal(got, want), f"{int((got != want).sum())} elements differ"


def test_source_view_into_a_store_buffer(gpu):
    """The connector hands the kernel ``buf[start:start+n]`` of a store buffer."""
    g = torch.Generator().manual_seed(3)
    buf = randn((300, 8, 256), torch.bfloat16, g)
    src = buf[123:123 + 77]
    _, kv, slots = _case(4, 77, True)
    inv = inv_freq()
    buf_dev = buf.to(gpu)
    kv_dev = kv.to(gpu)
    scatter_shifted(buf_dev[123:200], kv_dev, slots.to(gpu), 16, True, rope_shift(186, 128, inv, gpu))
    torch.cuda.synchronize(gpu)
    want = bits(kv)
    orc.scatter_shifted(bits(src), want, slots.numpy(), 16, True, 186, inv.numpy(), "bf16")
    assert np.array_equal(bits(kv_dev), want)


@pytest.mark.parametrize("delta", [-2048, 0, 37, 1999])
def test_fp8_single_span(gpu, delta):
    print(f"case fp8 delta={delta}", flush=True)
    g = torch.Generator().manual_seed(40 + delta)
    scale = 0.037
    src = randn((53, 8, 256), torch.float8_e4m3fn, g, scale)
    kv = randn((16, 8, 16, 256), torch.float8_e4m3fn, g, scale)
    table = torch.randperm(16, generator=g)
    pos = torch.arange(5, 58)
    slots = table[pos // 16] * 16 + pos % 16
    inv = inv_freq()
    got = bits(_run_gpu(gpu, src, kv, slots, 16, True, rope_shift(delta, 128, inv, gpu),
                        k_scale=scale))
    want = bits(kv)
    orc.scatter_shifted(bits(src), want, slots.numpy(), 16, True, delta, inv.numpy(), "fp8",
                        k_scale=np.float32(scale))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("delta", [-1, 7, 1999])
def test_fp8_every_code_in_k_and_its_partner(gpu, delta):
    """All 256 e4m3fn codes -- NaN (0x7F, 0xFF), +-0, subnormals, +-448 -- as K elements
    and as their rotate-half partners, bit-exact against the oracle's rule."""
    print(f"case fp8 all codes delta={delta}", flush=True)
    g = torch.Generator().manual_seed(77 + delta)
    n, heads, d = 64, 8, 128
    codes = torch.arange(256, dtype=torch.int64)
    k = codes[torch.randint(0, 256, (n, heads, d), generator=g)]
    # guarantee every (code, partner code) pairing of a sample set appears
    k[0, 0, :64] = codes[:64]
    k[0, 0, 64:] = codes[64:128]
    k[1, 0, :64] = codes[128:192]
    k[1, 0, 64:] = codes[192:]
    v = codes[torch.randint(0, 256, (n, heads, d), generator=g)]
    src = torch.cat((k, v), -1).to(torch.uint8).view(torch.float8_e4m3fn)
    kv = torch.zeros(8, heads, 16, 2 * d, dtype=torch.uint8).view(torch.float8_e4m3fn)
    slots = torch.randperm(128, generator=g)[:n]
    scale = 0.0625
    inv = inv_freq()
    got = bits(_run_gpu(gpu, src, kv, slots, 16, True, rope_shift(delta, d, inv, gpu),
                        k_scale=scale))
    want = bits(kv)
    orc.scatter_shifted(bits(src), want, slots.numpy(), 16, True, delta, inv.numpy(), "fp8",
                        k_scale=np.float32(scale))
    assert np.array_equal(got, want), f"{int((got != want).sum())} bytes differ"


def test_bf16_special_values(gpu):
    """NaN, +-inf, +-0, denormals and the largest finite values in K, bit-exact."""
    print("case bf16 special values", flush=True)
    g = torch.Generator().manual_seed(5)
    n, heads, d = 32, 8, 128
    src = torch.randn(n, heads, 2 * d, generator=g).to(torch.bfloat16)
    specials = torch.tensor([float("nan"), float("inf"), -float("inf"), 0.0, -0.0, 1e-40, -1e-40,
                             3.3e38, -3.3e38, 9.2e-41], dtype=torch.float32).to(torch.bfloat16)
    flat = src.view(-1, 2 * d)
    idx = torch.randint(0, flat.shape[0], (200,), generator=g)
    col = torch.randint(0, d, (200,), generator=g)
    flat[idx, col] = specials[torch.arange(200) % len(specials)]
    kv = torch.zeros(4, 16, heads, 2 * d, dtype=torch.bfloat16)
    slots = torch.randperm(64, generator=g)[:n]
    inv = inv_freq()
    got = bits(_run_gpu(gpu, src, kv, slots, 16, False, rope_shift(-566, d, inv, gpu)))
    want = bits(kv)
    orc.scatter_shifted(bits(src), want, slots.numpy(), 16, False, -566, inv.numpy(), "bf16")
    assert np.array_equal(got, want), f"{int((got != want).sum())} elements differ"
