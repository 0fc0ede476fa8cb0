"""GPU parity of the KV-cache writer (pa_cache_write) against the CPU oracle.

The bar is bit-exact: the writer is integer/byte work plus IEEE fp32
division and round-half-even, so every stored byte and scale must equal
oracle.write_kv / quantize_kv (the reference's quantisation,
pagedattn/cache.py:33-48) on the same rows.
"""

from __future__ import annotations

import pytest
import torch

from helpers import max_abs, seeded_q
from oracle import reference as oracle
from pagedattn import LLAMA3_8B, ModelShape, allocate, reshape_and_cache
from pagedattn.hip_decode import paged_decode_hip

pytestmark = pytest.mark.gpu


def _raw(t):
    return t.view(torch.uint8) if t.element_size() == 1 else t


def _cpu_copy(c):
    import dataclasses

    return dataclasses.replace(
        c, k_cache=c.k_cache.cpu().clone(), v_cache=c.v_cache.cpu().clone(),
        k_scale=None if c.k_scale is None else c.k_scale.cpu().clone(),
        v_scale=None if c.v_scale is None else c.v_scale.cpu().clone(),
        block_table=c.block_table.cpu(), seq_lens=c.seq_lens.cpu())


@pytest.mark.parametrize("kv_dtype,scale_dtype", [("fp16", torch.float16), ("fp8_e5m2", torch.float16),
                                                  ("int8", torch.float16), ("int8", torch.float32)])
@pytest.mark.parametrize("hkv,d", [(8, 128), (2, 64), (4, 32), (1, 256)])
def test_write_matches_oracle_bytes(kv_dtype, scale_dtype, hkv, d):
    shape = ModelShape(hkv * 2, hkv, d, "w")
    c = allocate(shape, 3, [100, 37, 5], kv_dtype=kv_dtype, scale_dtype=scale_dtype, seed=41,
                 device="cuda", slack_blocks=4)
    ref = _cpu_copy(c)
    g = torch.Generator().manual_seed(42)
    n = 40
    key = (torch.randn((n, hkv, d), generator=g) * 4).half()
    value = torch.randn((n, hkv, d), generator=g).half()
    key[3] = 0  # an all-zero row: the int8 scale takes the 1e-6 floor
    nb = c.k_cache.shape[0]
    slots = torch.randperm(nb * 16, generator=g)[:n].to(torch.int64)
    slots[[0, 7]] = -1                      # padding slots are skipped
    slots[9] = nb * 16 + 5                  # past the pool: skipped
    reshape_and_cache(key.cuda(), value.cuda(), c, slots.cuda())
    oracle.write_kv(key, value, ref, slots)
    torch.cuda.synchronize()
    assert torch.equal(_raw(c.k_cache.cpu()), _raw(ref.k_cache))
    assert torch.equal(_raw(c.v_cache.cpu()), _raw(ref.v_cache))
    if kv_dtype == "int8":
        assert torch.equal(c.k_scale.cpu(), ref.k_scale)
        assert torch.equal(c.v_scale.cpu(), ref.v_scale)


def test_e5m2_cast_of_every_fp16_value():
    """All 65,536 fp16 bit patterns through the writer equal torch's cast
    (round to nearest even, overflow to inf, NaN stays NaN)."""
    shape = ModelShape(1, 1, 128, "all")
    c = allocate(shape, 1, [512], kv_dtype="fp8_e5m2", seed=43, device="cuda", shuffle=False)
    pats = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.float16)
    rows = pats.view(512, 1, 128)
    slots = torch.arange(512, dtype=torch.int64)
    reshape_and_cache(rows.cuda(), rows.cuda(), c, slots.cuda())
    torch.cuda.synchronize()
    got = c.k_cache.cpu().view(torch.uint8).reshape(-1)
    want = pats.to(torch.float8_e5m2).view(torch.uint8)
    nan = torch.isnan(pats)
    assert torch.equal(got[~nan], want[~nan])
    # NaN inputs give an e5m2 NaN (exponent all ones, mantissa non-zero)
    gn = got[nan].to(torch.int32)
    assert bool(((gn & 0x7C) == 0x7C).all()) and bool(((gn & 0x3) != 0).all())


@pytest.mark.parametrize("kv_dtype", ["fp16", "fp8_e5m2", "int8"])
def test_write_then_decode(kv_dtype):
    """Append one token per sequence with the writer, then decode: matches the
    oracle on the oracle-written cache (the serving step: write, attend)."""
    lens = [15, 16, 100, 1]
    c = allocate(LLAMA3_8B, 4, lens, kv_dtype=kv_dtype, seed=44, device="cuda", slack_blocks=8)
    # give every sequence room for one more token, in a free block if it
    # needs a new one
    bt = c.block_table.clone()
    used = {int(bt[b, j]) for b, t in enumerate(lens) for j in range(-(-t // 16))}
    free = [i for i in range(c.k_cache.shape[0]) if i not in used]
    slots = []
    for b, t in enumerate(lens):
        if t % 16 == 0:
            bt[b, t // 16] = free.pop()
        slots.append(int(bt[b, t // 16]) * 16 + t % 16)
    assert bt.shape[1] * 16 > max(lens)
    c.block_table = bt
    ref = _cpu_copy(c)
    g = torch.Generator().manual_seed(45)
    key = torch.randn((4, 8, 128), generator=g).half()
    value = torch.randn((4, 8, 128), generator=g).half()
    slot_t = torch.tensor(slots, dtype=torch.int64)
    reshape_and_cache(key.cuda(), value.cuda(), c, slot_t.cuda())
    oracle.write_kv(key, value, ref, slot_t)
    c.seq_lens = c.seq_lens + 1
    ref.seq_lens = ref.seq_lens + 1
    q = seeded_q(4, 32, 128, 45, device="cuda")
    got = paged_decode_hip(q, c)
    torch.cuda.synchronize()
    want = oracle.reference_decode(q, ref, out_dtype=torch.float32)
    assert max_abs(got, want) < 2e-3


def test_bf16_rows_into_bf16_cache():
    c = allocate(LLAMA3_8B, 1, [64], kv_dtype="bf16", seed=46, device="cuda", slack_blocks=2)
    ref = _cpu_copy(c)
    g = torch.Generator().manual_seed(47)
    key = torch.randn((5, 8, 128), generator=g).to(torch.bfloat16)
    value = torch.randn((5, 8, 128), generator=g).to(torch.bfloat16)
    slots = torch.tensor([0, 17, -1, 40, 95], dtype=torch.int64)
    reshape_and_cache(key.cuda(), value.cuda(), c, slots.cuda())
    oracle.write_kv(key, value, ref, slots)
    torch.cuda.synchronize()
    assert torch.equal(c.k_cache.cpu(), ref.k_cache) and torch.equal(c.v_cache.cpu(), ref.v_cache)


@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
def test_int8_quotients_on_and_next_to_half_integers(scale_dtype):
    """Rows whose x / scale land exactly on half-integers (ties to even) and
    one fp16 step away from them: the writer's rounding equals torch's IEEE
    division + round-half-even there too."""
    shape = ModelShape(2, 1, 128, "h")
    c = allocate(shape, 1, [256], kv_dtype="int8", scale_dtype=scale_dtype, seed=48, device="cuda",
                 shuffle=False)
    ref = _cpu_copy(c)
    rows = []
    for amax in (127.0, 254.0, 100.0, 3.0, 1000.0):
        scale = torch.tensor(amax / 127.0, dtype=torch.float32).to(scale_dtype).float().item()
        k = torch.arange(-63, 64, dtype=torch.float32)          # 127 half-integers
        xs = ((k + 0.5) * scale).half()
        for step in (0, 1, -1):                                  # on, and one fp16 step off
            v = xs.view(torch.int16) + step
            v = torch.where(xs == 0, xs.view(torch.int16), v)
            row = torch.cat([v.view(torch.float16), torch.tensor([amax], dtype=torch.float16)])
            rows.append(row)
    key = torch.stack(rows).view(-1, 1, 128)
    value = key.flip(0).contiguous()
    n = key.shape[0]
    slots = torch.arange(n, dtype=torch.int64)
    reshape_and_cache(key.cuda(), value.cuda(), c, slots.cuda())
    oracle.write_kv(key, value, ref, slots)
    torch.cuda.synchronize()
    assert torch.equal(_raw(c.k_cache.cpu()), _raw(ref.k_cache))
    assert torch.equal(_raw(c.v_cache.cpu()), _raw(ref.v_cache))
    assert torch.equal(c.k_scale.cpu(), ref.k_scale) and torch.equal(c.v_scale.cpu(), ref.v_scale)


@pytest.mark.parametrize("kv_dtype", ["fp16", "int8"])
def test_repeated_writes_through_the_argument_cache(kv_dtype):
    """Steps of one geometry reuse a validated argument struct with new
    key/value/slot pointers: every step's bytes equal the oracle's. A cache
    whose tensors were replaced is validated and written again, and a slot
    tensor of another dtype is refused even after cached calls."""
    import dataclasses

    c = allocate(LLAMA3_8B, 2, [64, 40], kv_dtype=kv_dtype, seed=49, device="cuda", slack_blocks=8)
    ref = _cpu_copy(c)
    g = torch.Generator().manual_seed(50)
    nb = c.k_cache.shape[0]
    perm = torch.randperm(nb * 16, generator=g).to(torch.int64)
    for step in range(4):
        key = torch.randn((6, 8, 128), generator=g).half()
        value = torch.randn((6, 8, 128), generator=g).half()
        slots = perm[6 * step:6 * step + 6].clone()
        reshape_and_cache(key.cuda(), value.cuda(), c, slots.cuda())
        oracle.write_kv(key, value, ref, slots)
    torch.cuda.synchronize()
    assert torch.equal(_raw(c.k_cache.cpu()), _raw(ref.k_cache))
    assert torch.equal(_raw(c.v_cache.cpu()), _raw(ref.v_cache))

    # new tensors in a copy of the cache object: written there, not into c
    c2 = dataclasses.replace(c, k_cache=c.k_cache.clone(), v_cache=c.v_cache.clone(),
                             k_scale=None if c.k_scale is None else c.k_scale.clone(),
                             v_scale=None if c.v_scale is None else c.v_scale.clone())
    ref2 = _cpu_copy(c2)
    key = torch.randn((6, 8, 128), generator=g).half()
    slots = perm[40:46].clone()
    reshape_and_cache(key.cuda(), key.cuda(), c2, slots.cuda())
    oracle.write_kv(key, key, ref2, slots)
    torch.cuda.synchronize()
    assert torch.equal(_raw(c2.k_cache.cpu()), _raw(ref2.k_cache))
    assert torch.equal(_raw(c.k_cache.cpu()), _raw(ref.k_cache))  # c untouched
    with pytest.raises(ValueError, match="int64"):
        reshape_and_cache(key.cuda(), key.cuda(), c2, slots.to(torch.int32).cuda())
