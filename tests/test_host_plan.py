"""The host-built launch tables of the flat split (pa_flat_host_plan, the
tables pa_decode derives from seq_lens_host) against the oracle's flat
ranges (oracle.flat_segments).

No counterpart in the reference. The tables must describe exactly the
ranges the kernels find by scanning seq_lens on the GPU: for every range its
first sequence, first 32-token tile and tile count, and the list of the
sequences the merge writes (those cut by a range boundary, with their first
slot b + j0 and slot count, and the empty ones, with count 0). Runs on the
CPU: the call builds the tables on the host and launches nothing.
"""

from __future__ import annotations

import ctypes
import random

import pytest
import torch

from oracle import reference as oracle
from pagedattn import _abi

FAKE = 0x10000  # 16-byte aligned, never dereferenced: the call only plans


def _args(lens, flat, cost, max_blocks=1 << 12, block_size=16):
    b = len(lens)
    a = _abi.PaDecodeArgs()
    a.q = a.k_cache = a.v_cache = a.out = a.block_table = a.seq_lens = FAKE
    a.part_out = a.part_lse = FAKE
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim = b, 32, 8, 128
    a.block_size, a.num_blocks, a.max_blocks, a.num_splits = block_size, 64, max_blocks, 1
    a.stride_qb, a.stride_qh = 32 * 128, 128
    a.stride_kn, a.stride_kt, a.stride_kh = block_size * 8 * 128, 8 * 128, 128
    a.stride_ob, a.stride_oh = 32 * 128, 128
    a.stride_pb, a.stride_ph, a.stride_lb, a.stride_lh = 32 * 128, 128, 32, 1
    a.stride_btb = max_blocks
    a.kv_dtype, a.scale_dtype, a.io_dtype = _abi.PA_KV_FP16, _abi.PA_SCALE_NONE, _abi.PA_IO_FP16
    a.sm_scale = 128 ** -0.5
    a.flat_splits, a.flat_seq_cost = flat, cost
    host = torch.tensor(lens, dtype=torch.int32)
    a.seq_lens_host = host.data_ptr()
    return a, host


def _plan(lens, flat, cost, with_flags=False, **kw):
    a, host = _args(lens, flat, cost, **kw)
    ranges = (ctypes.c_int32 * (3 * flat))()
    items = (ctypes.c_int32 * (3 * max(1, len(lens))))()
    n = ctypes.c_int32(0)
    flags = ctypes.c_int32(-1)
    rc = _abi.load().pa_flat_host_plan(ctypes.byref(a), ranges, items, ctypes.byref(n), ctypes.byref(flags))
    del host
    got = (rc, [tuple(ranges[3 * j:3 * j + 3]) for j in range(flat)],
           [tuple(items[3 * i:3 * i + 3]) for i in range(n.value)])
    return got + (flags.value,) if with_flags else got


def _expected(lens, flat, cost, max_tokens):
    clamped = [max(0, min(t, max_tokens)) for t in lens]
    segs, _ = oracle.flat_segments(clamped, flat, seq_cost=cost)
    ranges = [(0, 0, 0)] * flat
    pieces = {}
    for j, b, lo, hi in segs:
        t0, t1 = lo // 32, -(-hi // 32)
        if ranges[j][2] == 0:
            ranges[j] = (b, t0, t1 - t0)
        else:
            ranges[j] = (ranges[j][0], ranges[j][1], ranges[j][2] + t1 - t0)
        pieces.setdefault(b, []).append(j)
    items = []
    for b, t in enumerate(clamped):
        if t == 0:
            items.append((b, 0, 0))
        elif len(pieces[b]) > 1:
            items.append((b, b + pieces[b][0], len(pieces[b])))
    return ranges, items


CASES = [
    ([300, 1, 4096, 0, 17, 33, 64, 1000], 7, 0),
    ([300, 1, 4096, 0, 17, 33, 64, 1000], 64, 1),
    ([300, 1, 4096, 0, 17, 33, 64, 1000], 256, 3),
    ([4096] * 64, 128, 0),          # C2: every range boundary on a sequence boundary
    ([0, 0, 0], 8, 2),              # only empty sequences
    ([32, 32], 8, 3),               # ranges that cover charges only
    ([40000, 3, 700], 40, 0),       # one sequence over many ranges
]


@pytest.mark.parametrize("lens,flat,cost", CASES)
def test_host_plan_matches_oracle(lens, flat, cost):
    rc, ranges, items = _plan(lens, flat, cost)
    assert rc == _abi.PA_OK, _abi.load().pa_last_error()
    want_r, want_i = _expected(lens, flat, cost, (1 << 12) * 16)
    assert ranges == want_r
    assert items == want_i


def test_host_plan_random_batches():
    rng = random.Random(7)
    for _ in range(300):
        b = rng.randint(1, 200)
        lens = [rng.choice([0, rng.randint(1, 64), rng.randint(1, 3000), rng.randint(1, 20000)])
                for _ in range(b)]
        flat = rng.choice([1, 2, 5, 37, 128, 256])
        cost = rng.choice([0, 0, 1, 2, 7])
        rc, ranges, items, flags = _plan(lens, flat, cost, with_flags=True)
        want_r, want_i = _expected(lens, flat, cost, (1 << 12) * 16)
        assert rc == _abi.PA_OK
        assert ranges == want_r, (lens, flat, cost)
        assert items == want_i, (lens, flat, cost)
        # the merge list goes to the kernel only when it fits its table
        assert bool(flags & _abi.PA_HOST_PLAN_MERGE) == (len(want_i) <= _abi.PA_HOST_TABLE_MAX)
        assert flags & _abi.PA_HOST_PLAN_RANGES


def test_host_plan_clamps_to_the_block_table():
    """Lengths past the block table count as its capacity, negative ones as
    empty, as the kernels clamp them."""
    lens = [5000, -3, 100, 70000]
    rc, ranges, items = _plan(lens, 9, 1, max_blocks=64)  # 1024 tokens per row
    assert rc == _abi.PA_OK
    want_r, want_i = _expected(lens, 9, 1, 64 * 16)
    assert ranges == want_r and items == want_i


def test_host_plan_limits():
    """Tables beyond the kernel-argument tables are still reported whole; the
    flags say which of them pa_decode would pass to the kernels."""
    lens = [100] * 10
    flat = _abi.PA_HOST_TABLE_MAX + 1
    rc, ranges, items, flags = _plan(lens, flat, 0, with_flags=True)
    assert rc == _abi.PA_OK
    assert flags == _abi.PA_HOST_PLAN_MERGE  # more ranges than the table holds: the kernels scan
    want_r, want_i = _expected(lens, flat, 0, (1 << 12) * 16)
    assert ranges == want_r and items == want_i
    lens = [0] * (_abi.PA_HOST_TABLE_MAX + 1)
    rc, ranges, items, flags = _plan(lens, 4, 0, with_flags=True)
    assert rc == _abi.PA_OK
    assert flags == _abi.PA_HOST_PLAN_RANGES  # more merge entries than the table holds
    assert items == [(b, 0, 0) for b in range(len(lens))]
    a, host = _args([100] * 10, 0, 0)
    ranges = (ctypes.c_int32 * 3)()
    items = (ctypes.c_int32 * 30)()
    n = ctypes.c_int32(0)
    assert _abi.load().pa_flat_host_plan(ctypes.byref(a), ranges, items, ctypes.byref(n), None) == \
        _abi.PA_ERR_INVALID


def test_merge_slot_count_spans_every_range():
    """One sequence cut by every one of PA_MAX_FLAT_SPLITS ranges: its merge
    entry counts all of them (the count once lived in 16 bits, where 65,536
    read as 0 and the merge wrote zeros for the sequence)."""
    flat = _abi.PA_MAX_FLAT_SPLITS
    tokens = flat * 32  # one 32-token tile per range
    rc, ranges, items, flags = _plan([tokens], flat, 0, with_flags=True, max_blocks=tokens // 256,
                                     block_size=256)
    assert rc == _abi.PA_OK, _abi.load().pa_last_error()
    assert items == [(0, 0, flat)]
    assert ranges == [(0, j, 1) for j in range(flat)]
    assert flags == _abi.PA_HOST_PLAN_MERGE  # the merge list is passed, the ranges are scanned
    # past the limit the launch is refused before any table is built
    a, host = _args([tokens], flat + 1, 0, max_blocks=tokens // 256, block_size=256)
    r = (ctypes.c_int32 * (3 * (flat + 1)))()
    it = (ctypes.c_int32 * 3)()
    n = ctypes.c_int32(0)
    assert _abi.load().pa_flat_host_plan(ctypes.byref(a), r, it, ctypes.byref(n), None) == _abi.PA_ERR_INVALID
