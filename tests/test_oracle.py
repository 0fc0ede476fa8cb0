"""CPU pinning of the oracle (oracle/reference.py) -- no GPU needed.

The reference stores no golden vectors (its tests compute a live fp32 oracle,
tests/test_correctness.py:59-122), so the torch oracle is pinned by:
  * an independent float64 C restatement that walks pages (oracle/pa_oracle.c),
    itself checked bit-for-bit on the fp16 / e5m2 decoders and the fp16
    rounding against numpy and torch's conversions;
  * closed forms (T = 1, q = 0, constant V, one dominant logit);
  * torch SDPA's math backend on the gathered cache (reference.py:57-72);
  * invariants (block-table permutation, split count, page size);
  * quantisation identities (cache.py:33-62);
  * committed fixtures under tests/golden/ (written by the C oracle);
  * planted mistakes: mutated copies of the oracle must fail these checks.
"""

from __future__ import annotations

import math
import pathlib
import types

import numpy as np
import pytest
import torch

from helpers import golden_case
from oracle import c_oracle
from oracle import reference as oracle
from pagedattn import LLAMA3_8B, MHA_DEBUG, ModelShape, allocate
from pagedattn.cache import PagedKVCache

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def _cache(shape, lens, kv_dtype="fp16", block_size=16, seed=0, scale_dtype=torch.float16,
           shuffle=True, slack=0):
    return allocate(shape, len(lens), lens, block_size=block_size, kv_dtype=kv_dtype,
                    device="cpu", seed=seed, scale_dtype=scale_dtype, shuffle=shuffle,
                    slack_blocks=slack)


def _q(b, hq, d, seed):
    g = torch.Generator().manual_seed(1000 + seed)
    return torch.randn((b, hq, d), dtype=torch.float16, generator=g)


def _dense_cache(shape, k_dense, v_dense, block_size=16, seed=0):
    """PagedKVCache holding dense fp16 K/V [B, T, Hkv, D] under a permuted pool."""
    b, t, h, d = k_dense.shape
    nb_seq = -(-t // block_size)
    pool = b * nb_seq + 3
    perm = torch.randperm(pool, generator=torch.Generator().manual_seed(seed))
    k = torch.zeros((pool, block_size, h, d), dtype=torch.float16)
    v = torch.zeros_like(k)
    bt = torch.zeros((b, nb_seq), dtype=torch.int32)
    for bi in range(b):
        for j in range(nb_seq):
            phys = int(perm[bi * nb_seq + j])
            bt[bi, j] = phys
            lo, hi = j * block_size, min((j + 1) * block_size, t)
            k[phys, : hi - lo] = k_dense[bi, lo:hi]
            v[phys, : hi - lo] = v_dense[bi, lo:hi]
    return PagedKVCache(shape, block_size, "fp16", k, v, None, None, bt,
                        torch.full((b,), t, dtype=torch.int32))


# --------------------------------------------------------------------------
# the C oracle's own number decoders, against numpy / torch
# --------------------------------------------------------------------------

def test_c_half_decoder_all_patterns():
    bits = np.arange(1 << 16, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float64)
    got = np.array([c_oracle.half_to_double(int(b)) for b in bits])
    finite = np.isfinite(want)
    assert np.array_equal(got[finite], want[finite])
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))


def test_c_e5m2_decoder_all_bytes_and_shift_identity():
    by = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    want = by.view(torch.float8_e5m2).to(torch.float64).numpy()
    got = np.array([c_oracle.e5m2_to_double(int(b)) for b in range(256)])
    fin = np.isfinite(want)
    assert np.array_equal(got[fin], want[fin])
    assert np.array_equal(np.isnan(got), np.isnan(want))
    # e5m2 -> fp16 is the byte shifted into the high half (cache.py:27-28)
    shifted = (by.to(torch.int32) << 8).to(torch.int16).view(torch.float16).to(torch.float64).numpy()
    assert np.array_equal(shifted[fin], want[fin])


def test_c_round_half_matches_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 5, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                  1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11]),
    ])
    want = x.astype(np.float16).astype(np.float64)
    got = np.array([c_oracle.round_half(float(v)) for v in x])
    assert np.array_equal(got, want)


# --------------------------------------------------------------------------
# torch oracle against the float64 C oracle
# --------------------------------------------------------------------------

CASES = [
    # shape, lens, kv_dtype, block_size, scale dtype
    (LLAMA3_8B, [1, 17, 300], "fp16", 16, torch.float16),
    (ModelShape(14, 2, 64, "qwen"), [32, 192, 77, 5], "fp16", 16, torch.float16),
    (MHA_DEBUG, [65, 130], "fp16", 32, torch.float16),
    (ModelShape(8, 2, 32, "d32"), [40, 257], "fp8_e5m2", 16, torch.float16),
    (LLAMA3_8B, [200, 33], "fp8_e5m2", 64, torch.float16),
    (ModelShape(16, 2, 64, "g8"), [129, 3], "int8", 16, torch.float16),
    (ModelShape(64, 8, 128, "70b"), [70], "int8", 16, torch.float32),
    (ModelShape(24, 1, 256, "d256"), [50, 1], "int8", 32, torch.float32),
    (LLAMA3_8B, [90, 7], "bf16", 16, torch.float16),
    (ModelShape(14, 2, 64, "qwen"), [33], "bf16", 32, torch.float16),
]


@pytest.mark.parametrize("shape,lens,kv_dtype,block_size,scale_dtype", CASES)
def test_torch_oracle_matches_c_oracle(shape, lens, kv_dtype, block_size, scale_dtype):
    c = _cache(shape, lens, kv_dtype, block_size, seed=len(lens), scale_dtype=scale_dtype, slack=5)
    q = _q(len(lens), shape.num_q_heads, shape.head_dim, 1)
    ref32 = oracle.reference_decode(q, c, out_dtype=torch.float32)
    ref64 = c_oracle.decode(q, c)
    assert (ref32.double() - ref64).abs().max().item() < 2e-5
    # the reference's own output cast (reference.py:49)
    assert oracle.reference_decode(q, c).dtype == torch.float16


@pytest.mark.parametrize("sm_scale", [0.0, 0.01, 0.3])
def test_sm_scale_override(sm_scale):
    c = _cache(LLAMA3_8B, [90, 3], seed=3)
    q = _q(2, 32, 128, 3)
    got = oracle.reference_decode(q, c, sm_scale=sm_scale, out_dtype=torch.float32)
    assert (got.double() - c_oracle.decode(q, c, sm_scale=sm_scale)).abs().max().item() < 2e-5


# --------------------------------------------------------------------------
# closed forms
# --------------------------------------------------------------------------

def _dequant_dense(c):
    k, v = oracle.gather_contiguous(c)  # [B, Hkv, S, D] fp16
    return k.float(), v.float()


@pytest.mark.parametrize("kv_dtype", ["fp16", "fp8_e5m2", "int8"])
def test_single_token_returns_v_row(kv_dtype):
    c = _cache(LLAMA3_8B, [1, 1, 1], kv_dtype, seed=4)
    q = _q(3, 32, 128, 4)
    out = oracle.reference_decode(q, c, out_dtype=torch.float32)
    _, v = _dequant_dense(c)
    for h in range(32):
        assert torch.equal(out[:, h], v[:, h // 4, 0])
    assert torch.equal(c_oracle.decode(q, c).float(), out)


def test_zero_query_gives_mean_of_v():
    c = _cache(LLAMA3_8B, [37, 300], seed=5)
    q = torch.zeros((2, 32, 128), dtype=torch.float16)
    out = oracle.reference_decode(q, c, out_dtype=torch.float32)
    _, v = _dequant_dense(c)
    for bi, t in enumerate([37, 300]):
        mean = v[bi, :, :t].double().mean(dim=1)  # [Hkv, D]
        for h in range(32):
            assert (out[bi, h].double() - mean[h // 4]).abs().max().item() < 1e-6
    assert (c_oracle.decode(q, c) - out.double()).abs().max().item() < 1e-6


def test_constant_v_and_dominant_logit():
    g = torch.Generator().manual_seed(6)
    b, t, h, d = 2, 50, 2, 64
    shape = ModelShape(8, 2, 64, "t")
    k = torch.randn((b, t, h, d), generator=g).half()
    v = torch.full((b, t, h, d), 0.75, dtype=torch.float16)
    c = _dense_cache(shape, k, v, seed=6)
    q = _q(b, 8, d, 6)
    out = oracle.reference_decode(q, c, out_dtype=torch.float32)
    assert (out - 0.75).abs().max().item() < 1e-6
    # one token whose key is a large multiple of q wins the softmax
    v = torch.randn((b, t, h, d), generator=g).half()
    q = torch.zeros((b, 8, d), dtype=torch.float16)
    q[:, :, 0] = 1.0
    k = torch.zeros((b, t, h, d), dtype=torch.float16)
    k[:, 17, :, 0] = 400.0  # logit 50 vs 0 elsewhere
    c = _dense_cache(shape, k, v, seed=7)
    out = oracle.reference_decode(q, c, out_dtype=torch.float32)
    for hq in range(8):
        assert (out[:, hq] - v[:, 17, hq // 4].float()).abs().max().item() < 1e-12 + 1e-18
    assert (c_oracle.decode(q, c).float() - out).abs().max().item() < 1e-6


def test_query_head_reads_kv_head_h_div_group():
    # kv head j holds the constant j: output of q head h must be h // group
    b, t, hkv, d, g = 1, 40, 4, 32, 3
    shape = ModelShape(hkv * g, hkv, d, "map")
    k = torch.randn((b, t, hkv, d), generator=torch.Generator().manual_seed(8)).half()
    v = torch.arange(hkv, dtype=torch.float16).view(1, 1, hkv, 1).expand(b, t, hkv, d).contiguous()
    c = _dense_cache(shape, k, v, seed=8)
    out = oracle.reference_decode(_q(b, hkv * g, d, 8), c, out_dtype=torch.float32)
    for h in range(hkv * g):
        assert torch.allclose(out[0, h], torch.full((d,), float(h // g)), atol=1e-6)


# --------------------------------------------------------------------------
# library routine, invariants, splits
# --------------------------------------------------------------------------

def test_sdpa_math_crosscheck():
    c = _cache(LLAMA3_8B, [512, 100], seed=9)
    q = _q(2, 32, 128, 9)
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    assert (oracle.sdpa_math_decode(q, c) - ref).abs().max().item() < 1e-5


def test_block_permutation_invariance():
    lens = [300, 45]
    a = _cache(LLAMA3_8B, lens, seed=10, shuffle=False, slack=7)
    q = _q(2, 32, 128, 10)
    base = oracle.reference_decode(q, a, out_dtype=torch.float32)
    perm = torch.randperm(a.k_cache.shape[0], generator=torch.Generator().manual_seed(2))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    moved = PagedKVCache(a.shape, a.block_size, a.kv_dtype, a.k_cache[perm], a.v_cache[perm],
                         None, None, inv[a.block_table.long()].to(torch.int32), a.seq_lens)
    assert torch.equal(oracle.reference_decode(q, moved, out_dtype=torch.float32), base)


def test_page_size_invariance():
    # the same logical K/V laid out in pages of 16, 32 and 64 tokens
    g = torch.Generator().manual_seed(11)
    k = torch.randn((2, 200, 8, 128), generator=g).half()
    v = torch.randn((2, 200, 8, 128), generator=g).half()
    q = _q(2, 32, 128, 11)
    outs = [oracle.reference_decode(q, _dense_cache(LLAMA3_8B, k, v, bs, seed=bs),
                                    out_dtype=torch.float32) for bs in (16, 32, 64)]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


def test_padding_positions_read_clamped_page():
    # gather_contiguous pads shorter rows with the last block-table column
    # (cache.py:200-205); masked positions must not change the result
    c = _cache(LLAMA3_8B, [20, 70], seed=12)
    k, _ = oracle.gather_contiguous(c)
    assert k.shape == (2, 8, 70, 128)
    bt = c.block_table
    last = bt[0, bt.shape[1] - 1]
    assert torch.equal(k[0, :, 64:70], c.k_cache[last, 0:6].permute(1, 0, 2))


@pytest.mark.parametrize("num_splits", [1, 2, 3, 7, 40])
@pytest.mark.parametrize("balanced", [False, True])
def test_split_partials_merge_to_reference(num_splits, balanced):
    lens = [1, 33, 500, 96]
    c = _cache(LLAMA3_8B, lens, seed=13)
    q = _q(4, 32, 128, 13)
    msl = max(lens) if balanced else 0
    part, lse = oracle.split_partials(q, c, num_splits, align=32, max_seq_len=msl)
    cpart, clse = c_oracle.split(q, c, num_splits, align=32, max_seq_len=msl)
    fin = torch.isfinite(clse)
    assert torch.equal(torch.isfinite(lse), fin)
    assert (lse.double()[fin] - clse[fin]).abs().max().item() < 1e-4
    assert (part.double() - cpart).abs().max().item() < 2e-5
    merged = oracle.split_merge(part, lse)
    ref = c_oracle.decode(q, c)
    assert (merged.double() - ref).abs().max().item() < 2e-5
    # empty splits are exactly those that start at or past the sequence end
    for bi, t in enumerate(lens):
        ranges = oracle.split_ranges(t, num_splits, 32, msl)
        for s, (lo, hi) in enumerate(ranges):
            assert bool(fin[bi, 0, s]) == (lo < hi)


def test_split_ranges_closed_form():
    # chunk = ceil(ceil(T/align)/S) * align (triton_decode.py:78-85)
    assert oracle.split_ranges(100, 4, 32) == [(0, 32), (32, 64), (64, 96), (96, 100)]
    assert oracle.split_ranges(100, 3, 32) == [(0, 64), (64, 100), (100, 100)]
    # balanced mode: the chunk of the longest sequence (never below its own)
    assert oracle.split_ranges(100, 4, 32, max_seq_len=1000) == [(0, 100), (100, 100), (100, 100), (100, 100)]
    assert oracle.split_ranges(1000, 4, 32, max_seq_len=1000) == oracle.split_ranges(1000, 4, 32)
    assert oracle.split_ranges(2000, 4, 32, max_seq_len=1000) == oracle.split_ranges(2000, 4, 32)
    assert oracle.split_ranges(4096, 8, 64) == [(512 * i, 512 * i + 512) for i in range(8)]


def test_flat_segments_known_answer():
    # tiles [4, 0, 2] (align 32), total 6, per = ceil(6 / 2) = 3
    segs, per = oracle.flat_segments([100, 0, 33], 2)
    assert per == 3
    assert segs == [(0, 0, 0, 96), (1, 0, 96, 100), (1, 2, 0, 33)]
    # one range holds everything; more ranges than tiles leave ranges idle
    assert oracle.flat_segments([100, 0, 33], 1)[0] == [(0, 0, 0, 100), (0, 2, 0, 33)]
    segs, per = oracle.flat_segments([64, 1], 50)
    assert per == 1 and segs == [(0, 0, 0, 32), (1, 0, 32, 64), (2, 1, 0, 1)]
    assert oracle.flat_segments([0, 0], 4) == ([], 1)


def test_flat_segments_seq_cost_known_answer():
    # tiles [4, 2, 4]; cost 2: weights [6, 4, 6], W = 16, per = 8. Sequence 0's
    # tiles sit at weights 2..5 (range 0), sequence 1's at 8, 9 and sequence
    # 2's at 12..15 (range 1). Without the charge (per = 5) range 0 also takes
    # sequence 1's first tile.
    segs, per = oracle.flat_segments([100, 33, 100], 2, seq_cost=2)
    assert per == 8 and segs == [(0, 0, 0, 100), (1, 1, 0, 33), (1, 2, 0, 100)]
    assert oracle.flat_segments([100, 33, 100], 2)[0] == [
        (0, 0, 0, 100), (0, 1, 0, 32), (1, 1, 32, 33), (1, 2, 0, 100)]
    # ranges that cover charges only hold no tiles: weights [4, 4], per = 1
    assert oracle.flat_segments([32, 32], 8, seq_cost=3) == ([(3, 0, 0, 32), (7, 1, 0, 32)], 1)
    # an empty sequence carries no charge: weights [5, 0, 3], per = 4
    assert oracle.flat_segments([100, 0, 33], 2, seq_cost=1) == (
        [(0, 0, 0, 96), (1, 0, 96, 100), (1, 2, 0, 33)], 4)


def _flat_segments_brute(seq_lens, flat_splits, seq_cost, align=32):
    """The weighted flat split by expansion: each non-empty sequence becomes
    `seq_cost` charge units then one unit per tile, the units are cut into
    ranges of per = ceil(units / F), and each tile goes to its unit's range."""
    units = []  # (b, tile index) or None for a charge
    for b, t in enumerate(seq_lens):
        n = -(-max(0, t) // align)
        if n:
            units += [None] * seq_cost + [(b, k) for k in range(n)]
    per = max(1, -(-len(units) // flat_splits))
    pieces = {}
    for i, u in enumerate(units):
        if u is not None:
            pieces.setdefault((i // per, u[0]), []).append(u[1])
    segs = [(j, b, ks[0] * align, min((ks[-1] + 1) * align, seq_lens[b]))
            for (j, b), ks in sorted(pieces.items(), key=lambda kv: (kv[0][1], kv[0][0]))]
    return segs, per


@pytest.mark.parametrize("seq_cost", [1, 2, 5])
@pytest.mark.parametrize("flat_splits", [1, 2, 5, 13, 64, 500])
def test_flat_segments_seq_cost_against_brute_force(flat_splits, seq_cost):
    """The closed form (tile k of b at weight cw_b + cost + k) against the
    expansion into units, and the partition contract."""
    lens = _ragged_lens()
    segs, per = oracle.flat_segments(lens, flat_splits, seq_cost=seq_cost)
    assert (segs, per) == _flat_segments_brute(lens, flat_splits, seq_cost)
    assert _flat_partition_errors(lens, flat_splits, segs, per) == []


@pytest.mark.parametrize("mistake", ["charge_after_tiles", "charge_empty", "charge_per_tile"])
def test_planted_seq_cost_mistakes_are_caught(mistake):
    """Mutated weighted work lists disagree with the brute-force expansion."""
    lens = _ragged_lens()
    flat_splits, cost = 13, 2

    def mutated(seq_lens, f, c, align=32):
        tiles = [-(-max(0, t) // align) for t in seq_lens]
        if mistake == "charge_empty":
            weights = [n + c for n in tiles]
        elif mistake == "charge_per_tile":
            weights = [n * (1 + c) if n else 0 for n in tiles]
        else:
            weights = [n + c if n else 0 for n in tiles]
        per = max(1, -(-sum(weights) // f))
        segs, cw = [], 0
        for b, (t, n) in enumerate(zip(seq_lens, tiles)):
            first = cw if mistake == "charge_after_tiles" else cw + c
            step = 1 + c if mistake == "charge_per_tile" else 1
            pieces = {}
            for k in range(n):
                pieces.setdefault((first + k * step) // per, []).append(k)
            for j, ks in sorted(pieces.items()):
                segs.append((j, b, ks[0] * align, min((ks[-1] + 1) * align, t)))
            cw += weights[b]
        return segs, per

    assert mutated(lens, flat_splits, cost) != _flat_segments_brute(lens, flat_splits, cost), \
        f"{mistake} not caught"


def _flat_partition_errors(lens, flat_splits, segs, per):
    """Violations of the flat split's contract by a work list (empty if none)."""
    errs = []
    # every sequence is covered exactly once, in order, by tile-aligned pieces
    for b, t in enumerate(lens):
        pos = 0
        for _, bb, lo, hi in segs:
            if bb != b:
                continue
            if lo != pos or lo % 32 or hi <= lo:
                errs.append(f"sequence {b}: piece [{lo}, {hi}) after {pos}")
            pos = hi
        if pos != t:
            errs.append(f"sequence {b}: covered to {pos} of {t}")
    # a range holds at most `per` tiles, all ranges exist, they are in order,
    # and the slots b + j are unique
    tiles = {}
    for j, _, lo, hi in segs:
        tiles[j] = tiles.get(j, 0) + -(-(hi - lo) // 32)
    if tiles and (max(tiles.values()) > per or max(tiles) >= flat_splits):
        errs.append("a range is over-full or out of bounds")
    if [j for j, *_ in segs] != sorted(j for j, *_ in segs):
        errs.append("ranges out of order")
    slots = [b + j for j, b, _, _ in segs]
    if len(set(slots)) != len(slots):
        errs.append("slot collision")
    return errs


def _ragged_lens(seed=21, n=37):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(0, 3000, (n,), generator=g).tolist()
    lens[3] = 0
    lens[10] = 1
    return lens


@pytest.mark.parametrize("flat_splits", [1, 2, 5, 13, 64, 500])
def test_flat_segments_partition(flat_splits):
    lens = _ragged_lens()
    segs, per = oracle.flat_segments(lens, flat_splits)
    assert _flat_partition_errors(lens, flat_splits, segs, per) == []


@pytest.mark.parametrize("mistake", ["floor_per", "tile_end_past_length", "unaligned_start",
                                     "dropped_empty_skip"])
def test_planted_flat_mistakes_are_caught(mistake):
    """Mutated restatements of the flat work list fail the partition check."""
    lens = _ragged_lens()
    flat_splits = 13

    def mutated(seq_lens, f, align=32):
        tiles = [-(-max(0, t) // align) for t in seq_lens]
        total = sum(tiles)
        per = max(1, total // f) if mistake == "floor_per" else max(1, -(-total // f))
        segs, cu = [], 0
        for b, (t, n) in enumerate(zip(seq_lens, tiles)):
            if mistake == "dropped_empty_skip" and n == 0:
                segs.append((cu // per, b, 0, 0))
            fpos = cu
            while fpos < cu + n:
                j = fpos // per
                end = min(cu + n, (j + 1) * per)
                lo = (fpos - cu) * align + (1 if mistake == "unaligned_start" and fpos > cu else 0)
                hi = (end - cu) * align if mistake == "tile_end_past_length" else min((end - cu) * align, t)
                segs.append((j, b, lo, hi))
                fpos = end
            cu += n
        return segs, per

    segs, per = mutated(lens, flat_splits)
    assert _flat_partition_errors(lens, flat_splits, segs, per), f"{mistake} not caught"


@pytest.mark.parametrize("flat_splits,seq_cost", [(1, 0), (3, 0), (8, 0), (40, 0), (3, 1), (8, 2)])
def test_flat_partials_merge_to_reference(flat_splits, seq_cost):
    lens = [1, 33, 500, 0, 96, 260]
    c = _cache(LLAMA3_8B, lens, seed=15)
    q = _q(6, 32, 128, 15)
    part, lse, whole = oracle.flat_partials(q, c, flat_splits, seq_cost=seq_cost)
    ref = c_oracle.decode(q, c)
    segs, _ = oracle.flat_segments(lens, flat_splits, seq_cost=seq_cost)
    for b, t in enumerate(lens):
        js = [j for j, bb, _, _ in segs if bb == b]
        assert whole[b] == (len(js) == 1)
        if not js:
            continue
        merged = oracle.split_merge(part[[b + j for j in js]].permute(1, 0, 2).unsqueeze(0),
                                    lse[[b + j for j in js]].T.unsqueeze(0))[0]
        assert (merged.double() - ref[b]).abs().max().item() < 2e-5


def test_merge_of_all_empty_splits_is_nan():
    part = torch.zeros((1, 1, 3, 4))
    lse = torch.full((1, 1, 3), float("-inf"))
    assert torch.isnan(oracle.split_merge(part, lse)).all()


def test_empty_sequence_is_nan():
    c = _cache(LLAMA3_8B, [0, 5], seed=14)
    out = oracle.reference_decode(_q(2, 32, 128, 14), c, out_dtype=torch.float32)
    assert torch.isnan(out[0]).all() and torch.isfinite(out[1]).all()


# --------------------------------------------------------------------------
# quantisation semantics (cache.py:33-62)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
def test_int8_quant_roundtrip(scale_dtype):
    x = torch.randn((64, 16, 8, 128), generator=torch.Generator().manual_seed(15)).half()
    q, s = oracle.quantize_kv(x, "int8", scale_dtype)
    assert q.dtype == torch.int8 and s.dtype == scale_dtype and s.shape == x.shape[:-1]
    assert q.abs().max().item() <= 127
    amax = x.abs().amax(-1).float().clamp_min(1e-6)
    assert torch.equal(s, (amax / 127).to(scale_dtype))
    deq = oracle.dequantize_kv(q, s, "int8").float()
    half_step = s.float().unsqueeze(-1) / 2
    # rounding error <= half a step, plus the fp16 rounding of the product
    assert ((deq - x.float()).abs() <= half_step * 1.001 + deq.abs() * 2 ** -11 + 1e-7).all()


def test_int8_dequant_rounds_product_once_to_fp16():
    q = torch.tensor([[-127, -3, 0, 1, 77, 127]], dtype=torch.int8)
    s = torch.tensor([0.0123], dtype=torch.float16)
    got = oracle.dequantize_kv(q, s, "int8")
    want = torch.tensor([[c_oracle.round_half(int(v) * float(s[0])) for v in q[0]]]).half()
    assert torch.equal(got, want)


def test_e5m2_quant_error_bound():
    x = torch.randn(100000, generator=torch.Generator().manual_seed(16)).half()
    q, s = oracle.quantize_kv(x, "fp8_e5m2")
    assert s is None and q.dtype == torch.float8_e5m2
    deq = oracle.dequantize_kv(q, None, "fp8_e5m2").float()
    rel = ((deq - x.float()).abs() / x.float().abs().clamp_min(2 ** -14)).max().item()
    assert rel <= 0.125 + 1e-6  # half an ulp of a 2-bit mantissa


def test_oracle_quantize_matches_product():
    from pagedattn.cache import quantize_kv as product_quantize

    x = torch.randn((8, 16, 2, 64), generator=torch.Generator().manual_seed(17)).half()
    for kv, sd in (("fp16", torch.float16), ("fp8_e5m2", torch.float16),
                   ("int8", torch.float16), ("int8", torch.float32)):
        a, sa = oracle.quantize_kv(x, kv, sd)
        b, sb = product_quantize(x, kv, sd)
        assert torch.equal(a.view(torch.uint8) if a.element_size() == 1 else a,
                           b.view(torch.uint8) if b.element_size() == 1 else b)
        assert (sa is None and sb is None) or torch.equal(sa, sb)


def test_bytes_formula():
    c = _cache(LLAMA3_8B, [100, 3], "int8", seed=18, scale_dtype=torch.float32)
    assert oracle.bytes_read_per_decode_step(c) == 2 * 103 * 8 * 128 * 1 + 2 * 103 * 8 * 4
    assert c.bytes_read_per_decode_step() == oracle.bytes_read_per_decode_step(c)


# --------------------------------------------------------------------------
# golden fixtures (tests/golden/make_golden.py, written by the C oracle)
# --------------------------------------------------------------------------

def _golden_files():
    return sorted(GOLDEN.glob("*.npz"))


def test_golden_fixtures_present():
    assert len(_golden_files()) >= 4


@pytest.mark.parametrize("path", _golden_files(), ids=lambda p: p.stem)
def test_golden_fixture(path):
    q, c, sm, z = golden_case(path)
    want = torch.from_numpy(z["out"])
    got = oracle.reference_decode(q, c, sm_scale=sm, out_dtype=torch.float32)
    assert (got.double() - want).abs().max().item() < 2e-5
    assert (c_oracle.decode(q, c, sm_scale=sm) - want).abs().max().item() < 1e-12
    if "part" in z.files:
        ns = int(z["num_splits"])
        part, lse = oracle.split_partials(q, c, ns, align=32, sm_scale=sm)
        assert (part.double() - torch.from_numpy(z["part"])).abs().max().item() < 2e-5
        zl = torch.from_numpy(z["lse2"])
        fin = torch.isfinite(zl)
        assert torch.equal(torch.isfinite(lse), fin)
        assert (lse.double()[fin] - zl[fin]).abs().max().item() < 1e-4


# --------------------------------------------------------------------------
# planted mistakes: each mutated oracle must fail the C-oracle comparison
# --------------------------------------------------------------------------

def _mutant(kind):
    def decode(q, cache, sm_scale=None, out_dtype=None):
        qc = q.float()
        b, hq, d = qc.shape
        hkv = cache.shape.num_kv_heads
        group = hq // hkv
        k, v = oracle.gather_contiguous(cache)
        k, v = k.float(), v.float()
        lens = cache.seq_lens.long()
        s_max = k.shape[2]
        valid = torch.arange(s_max).unsqueeze(0) < lens.unsqueeze(1)
        if kind == "off_by_one_mask":
            valid = torch.arange(s_max).unsqueeze(0) <= lens.unsqueeze(1)
        scale = cache.shape.head_dim ** -0.5 if sm_scale is None else sm_scale
        if kind == "no_scale":
            scale = 1.0
        out = torch.empty((b, hq, d))
        for h in range(hq):
            kvh = h % hkv if kind == "wrong_head_map" else h // group
            logits = torch.einsum("bd,bsd->bs", qc[:, h], k[:, kvh]) * scale
            logits = logits.masked_fill(~valid, float("-inf"))
            p = torch.softmax(logits, dim=-1)
            vv = k[:, kvh] if kind == "k_for_v" else v[:, kvh]
            out[:, h] = torch.einsum("bs,bsd->bd", p, vv)
        return out
    return decode


@pytest.mark.parametrize("kind", ["wrong_head_map", "no_scale", "off_by_one_mask", "k_for_v"])
def test_planted_mistakes_are_caught(kind):
    c = _cache(ModelShape(8, 4, 64, "m"), [40, 200], seed=19, slack=4)
    q = _q(2, 8, 64, 19)
    ref = c_oracle.decode(q, c)
    honest = _mutant("none")(q, c)
    assert (honest.double() - ref).abs().max().item() < 2e-5
    bad = _mutant(kind)(q, c)
    assert (bad.double() - ref).abs().max().item() > 1e-2


def test_planted_dequant_mistake_is_caught():
    # an int8 oracle that forgets the scale must fail against the C oracle
    c = _cache(ModelShape(8, 2, 64, "m"), [60], "int8", seed=20)
    q = _q(1, 8, 64, 20)
    bad = types.SimpleNamespace(**{**c.__dict__, "k_scale": torch.ones_like(c.k_scale),
                                   "v_scale": torch.ones_like(c.v_scale)})
    got_bad = oracle.reference_decode(q, bad, out_dtype=torch.float32)
    assert (got_bad.double() - c_oracle.decode(q, c)).abs().max().item() > 1e-1


# --------------------------------------------------------------------------
# the KV write (vllm_backend.py:117-122 with cache.py:33-48 quantisation)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("kv_dtype,scale_dtype", [("fp16", torch.float16), ("fp8_e5m2", torch.float16),
                                                  ("int8", torch.float16), ("int8", torch.float32)])
def test_write_kv_equals_quantize(kv_dtype, scale_dtype):
    """Writing rows one slot at a time stores exactly quantize_kv of the rows,
    skips negative and out-of-pool slots, and leaves other slots untouched."""
    c = _cache(LLAMA3_8B, [40], kv_dtype, seed=21, scale_dtype=scale_dtype, slack=2)
    before_k = c.k_cache.clone()
    g = torch.Generator().manual_seed(22)
    n = 6
    key = torch.randn((n, 8, 128), generator=g).half() * 3
    value = torch.randn((n, 8, 128), generator=g).half()
    nb = c.k_cache.shape[0]
    slots = torch.tensor([5, -1, 17, nb * 16 + 3, 0, 47], dtype=torch.int64)
    oracle.write_kv(key, value, c, slots)
    qk, sk = oracle.quantize_kv(key, kv_dtype, scale_dtype)
    qv, sv = oracle.quantize_kv(value, kv_dtype, scale_dtype)
    raw = lambda t: t.view(torch.uint8) if t.element_size() == 1 else t
    for t, slot in enumerate(slots.tolist()):
        if slot < 0 or slot >= nb * 16:
            continue
        blk, off = divmod(slot, 16)
        assert torch.equal(raw(c.k_cache[blk, off]), raw(qk[t]))
        assert torch.equal(raw(c.v_cache[blk, off]), raw(qv[t]))
        if sk is not None:
            assert torch.equal(c.k_scale[blk, off], sk[t]) and torch.equal(c.v_scale[blk, off], sv[t])
    untouched = [s for s in range(nb * 16) if s not in slots.tolist()]
    for slot in untouched[:50]:
        blk, off = divmod(slot, 16)
        assert torch.equal(raw(c.k_cache[blk, off]), raw(before_k[blk, off]))


def test_write_then_decode_reads_the_new_token():
    """A token written at position T of a sequence is attended by the next
    decode: the dominant-logit closed form on the written key."""
    c = _cache(ModelShape(8, 2, 64, "w"), [31], "fp16", seed=23, slack=1)
    bt = c.block_table
    T = 31
    slot = int(bt[0, T // 16]) * 16 + T % 16
    q = torch.zeros((1, 8, 64), dtype=torch.float16)
    q[:, :, 0] = 1.0
    key = torch.zeros((1, 2, 64), dtype=torch.float16)
    key[0, :, 0] = 400.0
    value = torch.randn((1, 2, 64), generator=torch.Generator().manual_seed(24)).half()
    oracle.write_kv(key, value, c, torch.tensor([slot]))
    c.seq_lens = torch.tensor([T + 1], dtype=torch.int32)
    out = oracle.reference_decode(q, c, out_dtype=torch.float32)
    for h in range(8):
        assert (out[0, h] - value[0, h // 4].float()).abs().max().item() < 1e-3


def test_bf16_rows_are_read_as_fp16():
    """A bf16 cache is attended through fp16 (the reference's bf16 path,
    triton_decode.py:30,151 and cache.py:55-56): values that bf16 holds but
    fp16 rounds come out rounded, and the C oracle agrees."""
    c = _cache(LLAMA3_8B, [1], "bf16", seed=25)
    vals = torch.tensor([1 + 2 ** -7, 1e-8, 70000.0, 1.0 + 2 ** -8 + 2 ** -9], dtype=torch.bfloat16)
    c.v_cache[int(c.block_table[0, 0]), 0, 0, :4] = vals
    q = _q(1, 32, 128, 25)
    out = oracle.reference_decode(q, c, out_dtype=torch.float32)
    # bf16 -> fp16 with torch's cast: exact, underflow to 0, overflow to inf, exact
    want = vals.to(torch.float16).float()
    assert want[1] == 0 and torch.isinf(want[2]) and want[0] == 1 + 2 ** -7
    assert torch.equal(out[0, 0, :4], want)
    got_c = c_oracle.decode(q, c).float()
    assert torch.equal(got_c[0, 0, :4], want)


def test_flat_needs_merge_agrees_with_the_oracle_work_list():
    """The host's merge-free test (pagedattn.flat_needs_merge) against the
    oracle's restatement of the flat work list: no merge exactly when every
    sequence is one segment of one range."""
    import random

    from pagedattn import flat_needs_merge

    def oracle_needs(lens, flat, max_tokens=None, seq_cost=0):
        if max_tokens is not None:
            lens = [min(t, max_tokens) for t in lens]
        segs, _ = oracle.flat_segments(lens, flat, seq_cost=seq_cost)
        count = [0] * len(lens)
        for _, b, _, _ in segs:
            count[b] += 1
        return any(c != 1 for c in count)

    # known answers
    assert not flat_needs_merge([2048] * 128, 128)      # one sequence per range
    assert not flat_needs_merge([2048] * 256, 128)      # two per range
    assert flat_needs_merge([2048] * 64, 128)           # two ranges per sequence
    assert not flat_needs_merge([100] * 16, 16)
    assert flat_needs_merge([100] * 15 + [0], 16)       # an empty sequence: merge writes zeros
    assert flat_needs_merge([], 4) and flat_needs_merge([0, 0], 4)
    assert not flat_needs_merge([4096, 5000], 2, max_tokens=4096)   # clamped to 128 tiles each
    assert flat_needs_merge([4096, 5000], 2)                       # 128 + 157 tiles: cut
    rng = random.Random(5)
    for _ in range(500):
        lens = [rng.choice([0, 1, 31, 32, 33, 64, 100, 4096]) if rng.random() < 0.3 else rng.randint(0, 700)
                for _ in range(rng.randint(1, 20))]
        flat = rng.randint(1, 40)
        assert flat_needs_merge(lens, flat) == oracle_needs(lens, flat), (lens, flat)
        cap = rng.choice([32, 64, 512])
        assert flat_needs_merge(lens, flat, cap) == oracle_needs(lens, flat, cap), (lens, flat, cap)
        cost = rng.randint(1, 4)
        assert flat_needs_merge(lens, flat, cap, cost) == oracle_needs(lens, flat, cap, cost), \
            (lens, flat, cap, cost)
