"""Host wrapper of the gfx950 paged decode kernels.

Same call surface as the reference's `paged_decode_triton`
(ParamThakkar123/paged-decode-attention, pagedattn/triton_decode.py:285-377)
and `pick_num_splits` (:248-263); the launch itself goes through the C ABI of
`libpagedattn_hip.so` (include/pagedattn.h). Nothing here computes attention:
if the library is missing or the tensors are not on a GPU, the call raises.

Knobs of the reference that only steer Triton code generation (`per_page_bt`,
`num_warps`, `num_stages`) are accepted and ignored: the HIP kernels always
read one block-table entry per 16-token sub-tile (one per page at page size
16) and size their workgroups themselves (4 waves; the flat kernel's are the
CU's four SIMDs, one wave each, or two each for int8 caches). `block_n`
keeps the reference's check that it is a multiple of the page size; split
ranges are aligned to the kernels' 32-token tile.
"""

from __future__ import annotations

import ctypes
import dataclasses
import threading
import weakref

import numpy as np
import torch

from . import _abi
from .cache import PagedKVCache

# Work geometry of the decode kernel (csrc/paged_decode.hip): 4 wave64s per
# workgroup, 32 tokens per wave iteration; a CU has 4 SIMDs.
WAVES_PER_WORKGROUP = 4
TILE_TOKENS = 32
SIMDS_PER_CU = 4

# The launch planner's thresholds. Lengths are counted in 32-token tiles (the
# unit every kernel streams and the flat split deals out), batch sizes in
# workgroups or waves per CU, and cache sizes in K/V bytes per CU, so the
# rules scale with the CU count of the device. The values were measured on a
# 256-CU MI355X (graph-timed whole calls); the measurements are quoted at
# each constant.

# The classic split serves the batches too small for the flat split, which
# are latency-bound: it is sized for one round of one workgroup per CU, with
# chunks of at least MIN_SPLIT_TILES. Graph-timed whole calls at the
# Llama-3-8B shape, this rule against the previous one (two rounds of two
# workgroups per CU, chunks of at least 512 tokens): B = 1, T = 2048 9.6 /
# 12.3 us; B = 1, T = 8192 13.1 / 14.5; B = 4, T = 512 8.7 / 9.5; B = 4,
# T = 2048 12.4 / 13.5.
MIN_SPLIT_TILES = 2
# Sequences this short are never split: the merge launch costs more than the
# split saves (C1, T <= 192: 4.5 us unsplit, 6.9 with 2-3 splits).
UNSPLIT_MAX_TILES = 8
# A ragged batch with a workgroup for every CU is split only when its longest
# sequence exceeds this (B = 32, T <= 512: 11.0 us unsplit, 14.9 with 2
# splits, 22.6 with 8).
RAGGED_SPLIT_MIN_TILES = 32

# Flat split: one round of waves, at most FLAT_WAVES_PER_SIMD per SIMD even
# where the registers allow more. One streaming wave per SIMD measured
# fastest on every benchmark config with a split (C2-C5): with two, each
# SIMD's older wave runs ahead and the younger ones form a tail (C2 158.5 us
# at 1, 159.6 at 2; C3 39.3 and 40.6; C5 312.7 and 316.5); three per SIMD or
# a second round is slower still, and so are two per SIMD whose pairs
# balance their progress as int8's do (C2 163.7 against 160.2). Used when
# each wave gets at least MIN_FLAT_TILES_PER_WAVE 32-token tiles; smaller
# batches are latency-bound and run faster unsplit.
FLAT_WAVES_PER_SIMD = 1
# int8 tiles carry a dequantisation per K and V element (the reference's
# fp16(x * s)), which keeps one wave per SIMD busy issuing VALU work: a
# second wave per SIMD hides it. Decode kernel alone, one against two flat
# waves per SIMD: Llama-3-70B shape B = 32, T = 16384 (C4) fp32 scales 192.4
# / 176.3 us, fp16 scales 189.6 / 178.9; Llama-3-8B B = 64, T = 4096 fp32
# 107.1 / 95.0, fp16 97.1 / 92.4; Qwen2.5 B = 256, T = 2048 41.7 / 38.0.
FLAT_WAVES_PER_SIMD_KV = {"int8": 2}
MIN_FLAT_TILES_PER_WAVE = 4
# Tiles of weight the flat split charges each sequence of a ragged batch
# (flat_seq_cost): a wave that starts a sequence loads a new q, stores a
# result and restarts its tile pipeline, a fixed time, so the charge in
# tiles grows as the tiles shrink: 1 for 2-byte KV, 2 for 1-byte KV
# (RAGGED_FLAT_SEQ_COST_KV). Whole calls at the Llama-3-8B shape on C3's
# lengths (B = 64, T log-uniform 128..8192, F = 128; int8 F = 256), charge
# 0 / 1 / 2 / 3 tiles: fp8 - / 40.5 / 40.1 / 40.2 us (3 repetitions each,
# 0: 41.4), int8 + fp32 scales 52.2 / 50.8 / 49.1 / 50.1, fp16 73.5 / 72.7 /
# 73.0 / 72.8. Nearly uniform batches keep 0: their ranges then fall on
# sequence boundaries or cut every sequence alike, and a charge would only
# unbalance them.
RAGGED_FLAT_SEQ_COST = 1
RAGGED_FLAT_SEQ_COST_KV = {"fp8_e5m2": 2, "int8": 2}
# A single sequence up to this many tiles takes the classic split: cut into
# one chunk per CU it merges 32 partials per head, the flat split 128 (graph-
# timed whole calls, classic against flat: T = 16384 17.9 / 21.0 us, 32768
# 27.6 / 30.6, 65536 47.2 / 49.6; at 131072 the flat split wins, 87.9 against
# 91.4 with 64 splits).
SINGLE_SEQ_SPLIT_MAX_TILES = 2048
# A nearly uniform batch that fills the CUs unsplit (one workgroup per CU or
# more) runs unsplit while its K/V is at most this many bytes per CU: the
# flat pass streams faster but adds its merge launch (about 4 us). Whole-call
# break-even measured at the Llama-3-8B shape (B = 64, g = 4, D = 128, 256
# CUs), unsplit against flat: 2-byte KV 44.4 / 46.9 us at 268 MB, 85.2 / 85.1
# at 537 MB, 166 / 162 at 1074 MB; fp8 26.6 / 29.0 at 134 MB, 49.5 / 47.2 at
# 268 MB; int8 18.2 / 19.5 at 67 MB, 24.5 / 24.6 at 101 MB, 31.4 / 29.6 at
# 134 MB. (At 256 CUs: 512 MB, 192 MB and 96 MB.)
UNSPLIT_MAX_KV_BYTES_PER_CU = {"fp16": 2 << 20, "bf16": 2 << 20, "fp8_e5m2": 768 << 10,
                               "int8": 384 << 10}
# Rows shorter than UNSPLIT_MIN_ROW_BYTES (head_dim x element size: 1-byte
# KV at head_dim 64) stream slowly through the unsplit kernel, so there the
# limit is UNSPLIT_MAX_SHORT_ROW_BYTES_PER_CU. Whole calls at the
# Qwen2.5-0.5B shape (14 q / 2 kv heads, D = 64, 256 CUs), unsplit against
# flat (F = 512; int8 F = 1024): fp8 B = 128, T = 1024 (34 MB) 13.6 / 15.1
# us, B = 128, T = 2048 (67 MB) 23.8 / 20.1, B = 256, T = 1024 23.8 / 20.9,
# B = 256, T = 2048 (134 MB) 44.3 / 31.8; int8 B = 128, T = 1024 15.4 /
# 17.1, B = 256, T = 1024 26.2 / 24.1; fp16 (128-byte rows) B = 256,
# T = 2048 45.0 / 48.5.
UNSPLIT_MIN_ROW_BYTES = 128
UNSPLIT_MAX_SHORT_ROW_BYTES_PER_CU = 192 << 10
# Batches of short sequences that fill the CUs run unsplit, whatever their
# size and merge or not: the flat split loses there, because its waves
# switch sequences every few tiles. Per KV type, the longest sequence of a
# nearly uniform batch (UNSPLIT_SHORT_MAX_TILES), or of a ragged batch with
# at least RAGGED_UNSPLIT_MIN_WGS_PER_CU unsplit workgroups per CU
# (UNSPLIT_RAGGED_MAX_TILES). Graph-timed whole calls at the Llama-3-8B
# shape (g = 4, D = 128, 256 CUs), flat against unsplit, in us:
#   fp16 uniform: B = 128, T = 256 29.0 / 26.1, T = 1024 90.1 / 87.6, T = 2048
#     170.8 / 170.8; B = 1024, T = 256 208.9 / 189.2, T = 1024 700.4 / 689.9,
#     T = 2048 1355 / 1363 (bf16 the same);
#   fp16 ragged, T ~ U[32, hi]: B = 256, hi = 512 61.0 / 56.2, hi = 1024 102.3
#     / 101.1, hi = 2048 190.5 / 198.5; B = 1024, hi = 512 233.8 / 211.8,
#     hi = 1024 389.7 / 371.8, hi = 2048 711.0 / 707.2; B = 128 (4 workgroups
#     per CU), hi = 1024: 0.93 x the unsplit time;
#   fp8 uniform: B = 128, T = 256 19.2 / 16.4, T = 512 30.1 / 29.3, T = 1024
#     50.5 / 52.0; B = 512, T = 256 59.5 / 58.2, T = 512 0.96 x;
#   fp8 ragged: B = 256, hi = 512 39.4 / 35.2; B = 1024, hi = 256 97.4 / 80.3,
#     hi = 512 141.5 / 128.9;
#   int8 keeps the flat split (uniform B = 512, T = 256 64.3 / 73.4).
# With WIDE_GROUP_MIN or more q heads per kv head both limits double: at the
# Llama-3-70B shape (g = 8) and the Qwen2.5-0.5B shape (g = 7, D = 64) the
# unsplit kernel still wins at twice them (ragged, flat against unsplit:
# 70B B = 256 fp16 hi = 2048 191.2 / 185.2, fp8 hi = 1024 68.5 / 64.8;
# 70B B = 1024 fp16 hi = 2048 777.9 / 747.2, fp8 hi = 1024 262.7 / 243.8;
# Qwen B = 1024 fp16 hi = 2048 110.3 / 98.0, fp8 hi = 1024 52.8 / 51.5),
# while at g = 4 the flat split wins at fp16 hi = 2048.
UNSPLIT_SHORT_MAX_TILES = {"fp16": 32, "bf16": 32, "fp8_e5m2": 8}
UNSPLIT_RAGGED_MAX_TILES = {"fp16": 32, "bf16": 32, "fp8_e5m2": 16}
RAGGED_UNSPLIT_MIN_WGS_PER_CU = 8
WIDE_GROUP_MIN = 7
# Every flat wave and every merge wave scans seq_lens (512 lengths per round
# trip), so the merge grows with the batch: above this batch the classic
# kernel runs unsplit instead. Whole calls on ragged batches (T ~ U[256,
# 2048]), flat against unsplit: B = 512 fp16 406 / 415 us, int8 224 / 264;
# B = 1024 fp16 790 / 794, int8 434 / 490, fp8 425 / 451; B = 2048 fp16
# 1596 / 1566 ...
# Even a flat split that needs no merge (every range holds whole sequences)
# loses to the unsplit kernel above it: graph-timed uniform batches, flat
# against unsplit, fp16 B = 2048, T = 256 443 / 378 us, B = 4096, T = 128
# 668 / 489, B = 3072, T = 1024 2200 / 2072; int8 B = 2048, T = 512
# 469 / 439 (int8 at T = 1024 is the one case within 4% the other way).
FLAT_MAX_BATCH = 1024

_KV_CODE = {"fp16": _abi.PA_KV_FP16, "fp8_e5m2": _abi.PA_KV_FP8_E5M2, "int8": _abi.PA_KV_INT8,
            "bf16": _abi.PA_KV_BF16}
_STORE_DTYPE = {"fp16": torch.float16, "fp8_e5m2": torch.float8_e5m2, "int8": torch.int8,
                "bf16": torch.bfloat16}
_IO_CODE = {torch.float16: _abi.PA_IO_FP16, torch.bfloat16: _abi.PA_IO_BF16}
_SCALE_CODE = {torch.float16: _abi.PA_SCALE_FP16, torch.float32: _abi.PA_SCALE_FP32}
_KV_ELEM_BYTES = {"fp16": 2, "bf16": 2, "fp8_e5m2": 1, "int8": 1}


def _tiles(tokens: int) -> int:
    return -(-max(0, int(tokens)) // TILE_TOKENS)


def _units(num_kv_heads: int, group: int) -> int:
    """Workgroups of the unsplit kernel per sequence ((kv head, head tile) pairs)."""
    return num_kv_heads * -(-group // _abi.PA_MAX_GROUP)


def pick_num_splits(
    batch: int, num_kv_heads: int, max_seq_len: int, sm_count: int, block_n: int = 64
) -> int:
    """Split count for the split-KV path, sized for the MI355X's 256 CUs.

    Same signature as the reference (triton_decode.py:248-263), MI355X policy
    from measurements:
      * batch*kv_heads >= CUs (every CU already has a workgroup) or the
        longest sequence has at most UNSPLIT_MAX_TILES tiles: no split;
      * otherwise enough splits for one workgroup per CU, but never chunks
        below MIN_SPLIT_TILES tiles; no power-of-two rounding and no cap
        of 64.
    `block_n` is accepted for signature compatibility.
    """
    del block_n
    base = max(1, batch * num_kv_heads)
    if base >= max(1, sm_count) or _tiles(max_seq_len) <= UNSPLIT_MAX_TILES:
        return 1
    want = -(-max(1, sm_count) // base)
    max_useful = max(1, max_seq_len // (MIN_SPLIT_TILES * TILE_TOKENS))
    return int(max(1, min(want, max_useful, _abi.PA_MAX_SPLITS)))


def _lens_array(seq_lens) -> np.ndarray:
    """Host lengths (ints, a CPU tensor or an array) as int64, negatives as 0.
    The planners work on whole arrays: a serving step plans batches of
    hundreds of sequences, and a Python loop per length cost ~0.4 ms at 256."""
    if isinstance(seq_lens, torch.Tensor):
        arr = seq_lens.detach().cpu().numpy()
    else:
        arr = np.asarray(seq_lens)
    return np.maximum(arr.astype(np.int64, copy=False).reshape(-1), 0)


def _tiles_array(lens: np.ndarray) -> np.ndarray:
    return (lens + (TILE_TOKENS - 1)) // TILE_TOKENS


def _nearly_uniform(lens) -> bool:
    """Longest length at most 1.25 x the mean (a non-empty batch)."""
    lens = _lens_array(lens)
    if lens.size == 0:
        return False
    tmax = int(lens.max())
    return tmax > 0 and tmax <= 1.25 * int(lens.sum()) / lens.size


def _fills_unsplit(lens, num_kv_heads: int, group: int, sm_count: int) -> bool:
    """A nearly uniform batch whose unsplit workgroups already give every CU one."""
    lens = _lens_array(lens)
    return _nearly_uniform(lens) and lens.size * _units(num_kv_heads, group) >= max(1, sm_count)


def short_batch_runs_unsplit(batch: int, max_seq_len: int, num_kv_heads: int, group: int,
                             sm_count: int, kv_dtype: str, uniform: bool = False) -> bool:
    """Whether a batch of short sequences runs faster unsplit than flat.

    With `uniform` (a nearly uniform batch whose unsplit workgroups give every
    CU one, `_fills_unsplit`) the longest sequence may have up to
    UNSPLIT_SHORT_MAX_TILES tiles; any batch with
    RAGGED_UNSPLIT_MIN_WGS_PER_CU unsplit workgroups per CU up to
    UNSPLIT_RAGGED_MAX_TILES. Needs only the batch size and the longest
    length, so a caller without the lengths applies the ragged rule. Groups
    of WIDE_GROUP_MIN or more q heads per kv head double both limits.
    """
    if max_seq_len <= 0:
        return False
    wide = 2 if group >= WIDE_GROUP_MIN else 1
    tiles = _tiles(max_seq_len)
    if uniform and tiles <= wide * UNSPLIT_SHORT_MAX_TILES.get(kv_dtype, 0):
        return True
    return (batch * _units(num_kv_heads, group) >= RAGGED_UNSPLIT_MIN_WGS_PER_CU * max(1, sm_count)
            and tiles <= wide * UNSPLIT_RAGGED_MAX_TILES.get(kv_dtype, 0))


def plan_num_splits(seq_lens, num_kv_heads: int, group: int, sm_count: int) -> tuple[int, int]:
    """(num_splits, max_seq_len) of the classic split for a batch whose lengths the host knows.

    `pick_num_splits` sees only the longest length, so it cannot tell a
    uniform batch (best unsplit when it already fills the CUs) from a ragged
    one (whose long sequences then run alone at the end). With the lengths:
      * nearly uniform (longest <= 1.25 x mean) with a workgroup for every
        CU, or no sequence longer than UNSPLIT_MAX_TILES tiles: no split;
      * batches with fewer workgroups than CUs: the balanced chunking (every
        sequence cut with the longest one's chunk) with one workgroup of
        work per CU, chunk ~ sum(T) * heads / CUs (twice that for a ragged
        batch), at least MIN_SPLIT_TILES tiles;
      * ragged batches with a workgroup for every CU: unsplit up to
        RAGGED_SPLIT_MIN_TILES tiles, else about four rounds of workgroups,
        chunk ~ sum(T) * heads / (4 CUs).
    """
    lens = _lens_array(seq_lens)
    if lens.size == 0 or int(lens.max()) == 0:
        return 1, 0
    tmax = int(lens.max())
    units = _units(num_kv_heads, group)
    if _fills_unsplit(lens, num_kv_heads, group, sm_count) or _tiles(tmax) <= UNSPLIT_MAX_TILES:
        return 1, tmax
    work, cus = int(lens.sum()) * units, max(1, sm_count)
    if lens.size * units >= cus:
        # every CU has a workgroup already (a ragged batch): split only long
        # sequences, into several rounds of workgroups
        if _tiles(tmax) <= RAGGED_SPLIT_MIN_TILES:
            return 1, tmax
        chunk = work // (4 * cus)
    else:
        # one workgroup of work per CU; a ragged batch's chunks twice as long
        # (its short sequences add partly filled ones)
        chunk = (1 if _nearly_uniform(lens) else 2) * work // cus
    chunk = max(MIN_SPLIT_TILES * TILE_TOKENS, chunk)
    splits = max(1, min(-(-tmax // chunk), _abi.PA_MAX_SPLITS))
    return int(splits), tmax


def flat_splits_for(num_kv_heads: int, group: int, sm_count: int, waves_per_simd: int,
                    kv_dtype: str | None = None) -> int:
    """One round of waves over the (kv head, head tile) units: as many as
    the CUs hold (4 SIMDs each, `waves_per_simd` waves per SIMD), capped at
    FLAT_WAVES_PER_SIMD per SIMD (FLAT_WAVES_PER_SIMD_KV for the KV types
    that differ)."""
    cap = FLAT_WAVES_PER_SIMD_KV.get(kv_dtype, FLAT_WAVES_PER_SIMD)
    per_simd = max(1, min(waves_per_simd, cap))
    waves = max(1, sm_count) * SIMDS_PER_CU * per_simd
    return int(max(1, min(waves // _units(num_kv_heads, group), _abi.PA_MAX_FLAT_SPLITS)))


@dataclasses.dataclass(frozen=True)
class LaunchPlan:
    """How one decode call is launched.

    flat_splits > 0: the flat split with that many ranges per unit; `merge`
    says whether its merge pass has work (False when every sequence lies
    inside one range, so the decode pass writes all of `out`).
    flat_splits == 0: the classic kernel with `num_splits` per-sequence
    splits (1 = unsplit), chunked from `max_seq_len`. `flat_seq_cost`: the
    tiles of weight the flat split charges each sequence (0 = equal tiles).
    """

    num_splits: int
    max_seq_len: int
    flat_splits: int
    merge: bool = True
    flat_seq_cost: int = 0

    def launch_kwargs(self) -> dict:
        """Keywords of `paged_decode_hip` that select this launch."""
        if self.flat_splits:
            return {"flat_splits": self.flat_splits, "flat_seq_cost": self.flat_seq_cost}
        return {"num_splits": self.num_splits, "max_seq_len": self.max_seq_len}


def plan_launch(batch: int, max_seq_len: int, num_kv_heads: int, group: int, sm_count: int,
                waves_per_simd: int = 1, kv_dtype: str | None = None,
                head_dim: int | None = None, seq_lens=None) -> LaunchPlan:
    """The launch planner: every caller (the decode wrapper with
    `num_splits=None`, the vLLM boundary, the benchmarks) plans here.

    `seq_lens` (host ints) when the caller knows the lengths, else None: then
    only `batch` and `max_seq_len` are known (a serving step's metadata,
    which holds the lengths on the device only), and the planner assumes
    a ragged batch whose every sequence may be that long. Rules, in order:
      * the flat split (one round of waves, `flat_splits_for`) when each of
        its waves gets at least MIN_FLAT_TILES_PER_WAVE tiles, the batch is
        at most FLAT_MAX_BATCH and is not a single sequence of up to
        SINGLE_SEQ_SPLIT_MAX_TILES tiles; with `kv_dtype` and `head_dim`
        given, two exceptions run unsplit instead:
          - a batch of short sequences that fills the CUs
            (`short_batch_runs_unsplit`; the nearly-uniform limit only with
            known lengths);
          - a nearly uniform batch (known lengths) that fills the CUs
            unsplit, with at most UNSPLIT_MAX_KV_BYTES_PER_CU x CUs of K/V
            (UNSPLIT_MAX_SHORT_ROW_BYTES_PER_CU for rows under
            UNSPLIT_MIN_ROW_BYTES), unless the flat split needs no merge
            either (`flat_needs_merge`);
      * otherwise the classic split (`plan_num_splits`), on the known
        lengths or on `batch` sequences of `max_seq_len` tokens.
    A flat plan charges each sequence RAGGED_FLAT_SEQ_COST tiles
    (RAGGED_FLAT_SEQ_COST_KV for 1-byte KV) when the
    lengths are known and not nearly uniform, else nothing.
    """
    cus = max(1, sm_count)
    known = seq_lens is not None
    lens = _lens_array(seq_lens) if known else None
    if known:
        batch = int(lens.size)
        tmax = int(lens.max()) if batch else 0
        tiles = int(_tiles_array(lens).sum())
    else:
        tmax = max(0, int(max_seq_len))
        tiles = batch * _tiles(tmax)  # an upper bound
    flat = flat_splits_for(num_kv_heads, group, cus, waves_per_simd, kv_dtype)
    flat_ok = (batch <= FLAT_MAX_BATCH and tiles >= MIN_FLAT_TILES_PER_WAVE * flat
               and not (batch == 1 and _tiles(tmax) <= SINGLE_SEQ_SPLIT_MAX_TILES))
    if flat_ok:
        fills = known and _fills_unsplit(lens, num_kv_heads, group, cus)
        cost = RAGGED_FLAT_SEQ_COST_KV.get(kv_dtype, RAGGED_FLAT_SEQ_COST) \
            if known and not _nearly_uniform(lens) else 0
        merge = flat_needs_merge(lens, flat, seq_cost=cost) if known else True
        if kv_dtype is not None and head_dim is not None:
            if short_batch_runs_unsplit(batch, tmax, num_kv_heads, group, cus, kv_dtype,
                                        uniform=fills):
                return LaunchPlan(1, tmax, 0)
            kv_bytes = int(lens.sum()) * num_kv_heads * head_dim * _KV_ELEM_BYTES.get(kv_dtype, 2) * 2 \
                if known else 0
            limit = UNSPLIT_MAX_KV_BYTES_PER_CU.get(kv_dtype, 0)
            if head_dim * _KV_ELEM_BYTES.get(kv_dtype, 2) < UNSPLIT_MIN_ROW_BYTES:
                limit = min(limit, UNSPLIT_MAX_SHORT_ROW_BYTES_PER_CU)
            limit *= cus
            if fills and kv_bytes <= limit and merge:
                return LaunchPlan(1, tmax, 0)
        return LaunchPlan(1, tmax, flat, merge, cost)
    # the classic split, planned on the lengths (unknown: every sequence as
    # long as the longest, which sizes the chunks for the worst case)
    splits, tmax = plan_num_splits(lens if known else np.full(batch, tmax, dtype=np.int64),
                                   num_kv_heads, group, cus)
    return LaunchPlan(splits, tmax, 0)


def plan_decode(seq_lens, num_kv_heads: int, group: int, sm_count: int,
                waves_per_simd: int = 1, kv_dtype: str | None = None,
                head_dim: int | None = None) -> tuple[int, int, int]:
    """(num_splits, max_seq_len, flat_splits) for a batch whose lengths the
    host knows: `plan_launch` with the lengths."""
    lens = _lens_array(seq_lens)
    p = plan_launch(int(lens.size), 0, num_kv_heads, group, sm_count, waves_per_simd, kv_dtype,
                    head_dim, seq_lens=lens)
    return p.num_splits, p.max_seq_len, p.flat_splits


def flat_needs_merge(seq_lens, flat_splits: int, max_tokens: int | None = None,
                     seq_cost: int = 0) -> bool:
    """Whether a flat decode over these lengths leaves work to its merge pass.

    It does when a range boundary cuts a sequence (its pieces are partials)
    or a sequence is empty (the merge writes its zeros). Otherwise every
    sequence lies inside one range and the decode pass writes all of `out`
    itself, as for a uniform batch whose length in tiles times the batch
    divides evenly among the ranges. Lengths are clamped to `max_tokens` (the
    block table's capacity), as the kernels clamp them. `seq_cost` is the
    launch's flat_seq_cost: a non-empty sequence weighs its tiles plus
    `seq_cost`, and the ranges take equal weight.
    """
    lens = _lens_array(seq_lens)
    if max_tokens is not None:
        lens = np.minimum(lens, max_tokens)
    tiles = _tiles_array(lens)
    weights = np.where(tiles > 0, tiles + seq_cost, 0)
    total = int(weights.sum())
    if total == 0 or flat_splits <= 0:
        return True
    if bool((tiles == 0).any()):
        return True  # the merge writes an empty sequence's zeros
    per = max(1, -(-total // flat_splits))
    first = np.cumsum(weights) - weights + seq_cost  # weight of each sequence's tile 0
    return bool(((first // per) != ((first + tiles - 1) // per)).any())


class _Workspace:
    """Split-KV scratch (fp32 partial outputs and log2-sum-exps), per device.

    Grows to the largest request seen and hands out views, so repeated calls
    allocate nothing (the role of the reference's `_WS`, triton_decode.py:266-282).
    A buffer that is outgrown is retired, never freed: a HIP graph captured
    while it was current keeps launching into it, so it must stay valid for
    the life of the process. Growth is at least 2x, so the retired buffers
    together hold less than the current one. `reserve` sizes the workspace
    before a capture.
    """

    def __init__(self) -> None:
        self._buf: dict[torch.device, tuple[torch.Tensor, torch.Tensor]] = {}
        self._retired: dict[torch.device, list[tuple[torch.Tensor, torch.Tensor]]] = {}
        self._lock = threading.Lock()

    def _ensure(self, n_out: int, n_lse: int, device) -> tuple[torch.Tensor, torch.Tensor]:
        with self._lock:
            cur = self._buf.get(device)
            if cur is None or cur[0].numel() < n_out or cur[1].numel() < n_lse:
                grow_out = max(n_out, 1, 2 * cur[0].numel() if cur is not None else 0)
                grow_lse = max(n_lse, 1, 2 * cur[1].numel() if cur is not None else 0)
                if cur is not None:
                    self._retired.setdefault(device, []).append(cur)
                cur = (torch.empty(grow_out, dtype=torch.float32, device=device),
                       torch.empty(grow_lse, dtype=torch.float32, device=device))
                self._buf[device] = cur
            return cur

    def get(self, b: int, hq: int, splits: int, d: int, device) -> tuple[torch.Tensor, torch.Tensor]:
        n_out = b * hq * splits * d
        n_lse = b * hq * splits
        cur = self._ensure(n_out, n_lse, device)
        return cur[0][:n_out].view(b, hq, splits, d), cur[1][:n_lse].view(b, hq, splits)

    def get_flat(self, slots: int, hq: int, d: int, device) -> tuple[torch.Tensor, torch.Tensor]:
        """Flat-split slots: part_out [slots, hq, d], part_lse [slots, hq]."""
        out, lse = self.get(slots, hq, 1, d, device)
        return out.view(slots, hq, d), lse.view(slots, hq)

    def reserve(self, n_out: int, n_lse: int, device) -> None:
        self._ensure(n_out, n_lse, device)

    def current(self, device) -> tuple[torch.Tensor, torch.Tensor] | None:
        return self._buf.get(device)


_WS = _Workspace()


def reserve_workspace(batch: int, num_q_heads: int, head_dim: int, device,
                      num_splits: int = 1, flat_splits: int = 0) -> None:
    """Size the split workspace for calls up to this size before capturing
    them in a HIP graph, so that no later call grows it (a grown workspace
    leaves the captured graph's buffers in place, so replays stay correct;
    reserving only avoids the extra memory). Flat splits need
    (batch + flat_splits) slots, the classic split batch * num_splits."""
    slots = batch + flat_splits if flat_splits else batch * max(1, num_splits)
    dev = torch.device(device)
    if dev.index is None:
        dev = torch.device(dev.type, torch.cuda.current_device())
    _WS.reserve(slots * num_q_heads * head_dim, slots * num_q_heads, dev)


def _check_partials(device: torch.device, part_out: torch.Tensor, part_lse: torch.Tensor,
                    b: int, hq: int, d: int, num_splits: int, flat_splits: int) -> None:
    """Caller-supplied split workspace, checked before its pointers reach a
    kernel: float32, on `device`, head_dim contiguous, and the exact classic
    shapes [B, Hq, S, D] / [B, Hq, S] (split stride 1 in part_lse, which the
    kernels assume) or at least B + F flat slots [>= B+F, Hq, D] / [>= B+F, Hq]."""
    for name, t in (("part_out", part_out), ("part_lse", part_lse)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a tensor")
        if t.dtype != torch.float32:
            raise ValueError(f"{name} must be float32, got {t.dtype}")
        if t.device != device:
            raise ValueError(f"{name} is on {t.device}, q on {device}")
    if flat_splits > 0:
        slots = b + flat_splits
        if part_out.dim() != 3 or part_out.shape[0] < slots or tuple(part_out.shape[1:]) != (hq, d):
            raise ValueError(f"flat part_out {tuple(part_out.shape)} is not [>= {slots}, {hq}, {d}]")
        if part_lse.dim() != 2 or part_lse.shape[0] < slots or part_lse.shape[1] != hq:
            raise ValueError(f"flat part_lse {tuple(part_lse.shape)} is not [>= {slots}, {hq}]")
        if part_out.stride(2) != 1:
            raise ValueError("part_out must have a contiguous head dim")
    else:
        if tuple(part_out.shape) != (b, hq, num_splits, d):
            raise ValueError(f"part_out {tuple(part_out.shape)} is not {(b, hq, num_splits, d)}")
        if tuple(part_lse.shape) != (b, hq, num_splits):
            raise ValueError(f"part_lse {tuple(part_lse.shape)} is not {(b, hq, num_splits)}")
        if part_out.stride(3) != 1 or part_lse.stride(2) != 1:
            raise ValueError("part_out needs a contiguous head dim and part_lse a contiguous split dim")
_CU_COUNT: dict[int, int] = {}
_FLAT_WPS: dict[tuple, int] = {}


def flat_waves_per_simd(kv_dtype: str, head_dim: int, scale_dtype: torch.dtype | None = None) -> int:
    """Resident flat-kernel waves per SIMD, from the library's occupancy
    query on the current device (FLAT_WAVES_PER_SIMD without a GPU)."""
    sc = _abi.PA_SCALE_NONE if kv_dtype != "int8" else _SCALE_CODE.get(scale_dtype or torch.float16)
    key = (kv_dtype, head_dim, sc)
    n = _FLAT_WPS.get(key)
    if n is None:
        n = 0
        if torch.cuda.is_available() and kv_dtype in _KV_CODE:
            got = ctypes.c_int(0)
            if _abi.load().pa_flat_waves_per_simd(_KV_CODE[kv_dtype], sc, head_dim, ctypes.byref(got)) == 0:
                n = got.value
        if n <= 0:
            # every gfx950 instance holds at least the one wave per SIMD the
            # flat split launches (occupancy 2 to 5)
            n = FLAT_WAVES_PER_SIMD
        _FLAT_WPS[key] = n
    return n


def _cu_count(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    n = _CU_COUNT.get(idx)
    if n is None:
        n = torch.cuda.get_device_properties(idx).multi_processor_count
        _CU_COUNT[idx] = n
    return n


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# Validated argument structs, keyed by everything their validation read
# except the per-call pointers (q, out, workspace, host lengths). The cache's
# tensors enter the key by identity and data pointer and are held by weak
# references, so a key cannot match a new tensor that reuses a dead one's id;
# replacing a tensor or its storage validates again (the cache object's other
# fields enter by value). A tensor reshaped in place on the same memory
# (resize_, set_) is not noticed.
_ARG_TEMPLATES: dict[tuple, tuple] = {}
_ARG_TEMPLATES_MAX = 512


def _fill_args(
    q: torch.Tensor,
    cache: PagedKVCache,
    out: torch.Tensor,
    num_splits: int,
    sm_scale: float,
    part_out: torch.Tensor | None,
    part_lse: torch.Tensor | None,
    max_seq_len: int = 0,
    flat_splits: int = 0,
    flat_seq_cost: int = 0,
    seq_lens_host: torch.Tensor | None = None,
) -> _abi.PaDecodeArgs:
    """The pa_decode_args of one call: validated on the first call of its
    geometry (`_pack_args`), afterwards a copy of that struct with this
    call's pointers (the C side validates every call again)."""
    k, v, bt, sl = cache.k_cache, cache.v_cache, cache.block_table, cache.seq_lens
    ks, vs = cache.k_scale, cache.v_scale
    shape = cache.shape
    key = (id(k), k.data_ptr(), id(v), v.data_ptr(), id(bt), bt.data_ptr(), id(sl),
           sl.data_ptr(), id(ks), 0 if ks is None else ks.data_ptr(), id(vs), 0 if vs is None else vs.data_ptr(),
           cache.kv_dtype, cache.block_size, shape.num_q_heads, shape.num_kv_heads, shape.head_dim,
           q.shape, q.stride(), q.dtype, q.get_device(), out.shape, out.stride(), out.dtype,
           out.get_device(), num_splits, sm_scale, max_seq_len, flat_splits, flat_seq_cost,
           None if part_out is None else (part_out.shape, part_out.stride(), part_out.dtype,
                                          part_out.get_device(), part_lse.shape, part_lse.stride(),
                                          part_lse.dtype, part_lse.get_device()),
           seq_lens_host is None)
    hit = _ARG_TEMPLATES.get(key)
    if hit is not None:
        r = hit[0]
        hit = hit if (r[0]() is k and r[1]() is v and r[2]() is bt and r[3]() is sl
                      and (ks is None or r[4]() is ks) and (vs is None or r[5]() is vs)) else None
    if hit is not None:
        if seq_lens_host is not None and flat_splits > 0:
            _check_host_lens(seq_lens_host, q.shape[0])
        a = _abi.PaDecodeArgs.from_buffer_copy(hit[1])
        a.q = q.data_ptr()
        a.out = out.data_ptr()
        if part_out is not None:
            a.part_out = part_out.data_ptr()
            a.part_lse = part_lse.data_ptr()
        if seq_lens_host is not None and flat_splits > 0:
            a.seq_lens_host = seq_lens_host.data_ptr()
        return a
    tmpl = _pack_args(q, cache, out, num_splits, sm_scale, part_out, part_lse, max_seq_len,
                      flat_splits, flat_seq_cost, seq_lens_host)
    if len(_ARG_TEMPLATES) >= _ARG_TEMPLATES_MAX:
        _ARG_TEMPLATES.clear()
    refs = tuple(None if o is None else weakref.ref(o) for o in (k, v, bt, sl, ks, vs))
    _ARG_TEMPLATES[key] = (refs, tmpl)
    return _abi.PaDecodeArgs.from_buffer_copy(tmpl)


def _check_host_lens(seq_lens_host: torch.Tensor, b: int) -> None:
    if (seq_lens_host.device.type != "cpu" or seq_lens_host.dtype != torch.int32
            or tuple(seq_lens_host.shape) != (b,) or not seq_lens_host.is_contiguous()):
        raise ValueError(f"seq_lens_host must be a contiguous int32 CPU tensor of shape ({b},)")


def _pack_args(
    q: torch.Tensor,
    cache: PagedKVCache,
    out: torch.Tensor,
    num_splits: int,
    sm_scale: float,
    part_out: torch.Tensor | None,
    part_lse: torch.Tensor | None,
    max_seq_len: int = 0,
    flat_splits: int = 0,
    flat_seq_cost: int = 0,
    seq_lens_host: torch.Tensor | None = None,
) -> _abi.PaDecodeArgs:
    """Validate every tensor of a call and pack pa_decode_args."""
    b, hq, d = q.shape
    shape = cache.shape
    kv_dtype = cache.kv_dtype
    if kv_dtype not in _KV_CODE:
        raise NotImplementedError(f"kv_dtype {kv_dtype!r} is not supported by the HIP kernel")
    if q.dtype not in _IO_CODE or out.dtype != q.dtype:
        raise NotImplementedError(f"q/out dtype {q.dtype}/{out.dtype}: float16 or bfloat16, the same for both")
    if not q.is_cuda:
        raise ValueError(f"q is on {q.device}: the HIP decode kernel needs GPU tensors")
    k, v = cache.k_cache, cache.v_cache
    bt, sl = cache.block_table, cache.seq_lens
    dev = q.get_device()
    if (k.get_device() != dev or v.get_device() != dev or out.get_device() != dev
            or bt.get_device() != dev or sl.get_device() != dev):
        for name, t in (("k_cache", k), ("v_cache", v), ("out", out), ("block_table", bt), ("seq_lens", sl)):
            if t.get_device() != dev:
                raise ValueError(f"{name} is on {t.device}, q on {q.device}")
    if k.dtype != _STORE_DTYPE[kv_dtype] or v.dtype != k.dtype:
        raise ValueError(f"k/v cache dtype {k.dtype}/{v.dtype} does not match kv_dtype {kv_dtype}")
    kshape, kst = k.shape, k.stride()
    if len(kshape) != 4 or kshape[1] != cache.block_size or kshape[2] != shape.num_kv_heads or kshape[3] != d:
        raise ValueError(f"k_cache shape {tuple(kshape)} is not [NB, {cache.block_size}, "
                         f"{shape.num_kv_heads}, {d}]")
    if v.shape != kshape or v.stride() != kst:
        raise ValueError("v_cache must have k_cache's shape and strides")
    qst, ost = q.stride(), out.stride()
    if kst[3] != 1 or qst[2] != 1 or ost[2] != 1:
        raise ValueError("head_dim must be the contiguous (stride-1) dimension of q, out and the caches")
    if out.shape != (b, hq, d):
        raise ValueError(f"out shape {tuple(out.shape)} != {(b, hq, d)}")
    if bt.dtype != torch.int32 or sl.dtype != torch.int32:
        raise ValueError("block_table and seq_lens must be int32")
    btshape, btst = bt.shape, bt.stride()
    if len(btshape) != 2 or btshape[0] != b or sl.shape != (b,):
        raise ValueError(f"block_table {tuple(btshape)} / seq_lens {tuple(sl.shape)} do not match batch {b}")
    if btst[1] != 1 or sl.stride(0) != 1:
        raise ValueError("block_table rows and seq_lens must be contiguous")

    k_scale = v_scale = None
    sst = (0, 0)
    scale_code = _abi.PA_SCALE_NONE
    if kv_dtype == "int8":
        ks, vs = cache.k_scale, cache.v_scale
        if ks is None or vs is None:
            raise ValueError("int8 cache needs k_scale and v_scale")
        if ks.dtype not in _SCALE_CODE or vs.dtype != ks.dtype:
            raise ValueError(f"int8 scales must be float16 or float32, got {ks.dtype}/{vs.dtype}")
        sst = ks.stride()
        if tuple(ks.shape) != tuple(kshape[:3]) or vs.stride() != sst or sst[2] != 1:
            raise ValueError("k_scale/v_scale must be [NB, block_size, H_kv] with equal strides "
                             "and a contiguous head dimension")
        if ks.get_device() != dev or vs.get_device() != dev:
            raise ValueError("scales must live on q's device")
        k_scale, v_scale = ks.data_ptr(), vs.data_ptr()
        scale_code = _SCALE_CODE[ks.dtype]

    po = pl = None
    pst = (0, 0, 0)
    lst = (0, 0)
    if part_out is not None:
        po, pl = part_out.data_ptr(), part_lse.data_ptr()
        if flat_splits > 0:  # slots [B + F, Hq, D] / [B + F, Hq]
            if part_out.dim() != 3 or part_out.shape[0] < b + flat_splits or part_lse.shape[0] < b + flat_splits:
                raise ValueError(f"flat split workspace needs {b + flat_splits} slots")
            pst = (part_out.stride(0), part_out.stride(1), 0)
        else:
            pst = part_out.stride()[:3]
        lst = part_lse.stride()[:2]

    host_ptr = None
    if seq_lens_host is not None and flat_splits > 0:
        _check_host_lens(seq_lens_host, b)
        host_ptr = seq_lens_host.data_ptr()

    # one constructor call, fields in declaration order (include/pagedattn.h)
    return _abi.PaDecodeArgs(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), k_scale, v_scale, out.data_ptr(), po, pl,
        bt.data_ptr(), sl.data_ptr(),
        b, hq, shape.num_kv_heads, d, cache.block_size, kshape[0], btshape[1], num_splits,
        int(max_seq_len),
        qst[0], qst[1], kst[0], kst[1], kst[2], sst[0], sst[1], ost[0], ost[1],
        pst[0], pst[1], pst[2], lst[0], lst[1], btst[0],
        _KV_CODE[kv_dtype], scale_code, _IO_CODE[q.dtype], sm_scale, int(flat_splits),
        int(flat_seq_cost), host_ptr)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    """Handle of torch's current stream on `device` (the raw handle when torch
    exposes it: a Stream object per call costs more than the launch)."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


_get_device = getattr(torch._C, "_cuda_getDevice", None)


def _launch(t: torch.Tensor, fn, args) -> int:
    """fn(&args, stream) with t's device current, on that device's current
    torch stream (switching devices only when needed). The per-call path of
    every wrapper: a device index and the raw stream handle, no device or
    stream objects."""
    idx = t.get_device()
    cur = _get_device() if _get_device is not None else torch.cuda.current_device()
    if idx == cur:
        return fn(ctypes.byref(args), _raw_stream(idx) if _raw_stream is not None
                  else torch.cuda.current_stream(idx).cuda_stream)
    with torch.cuda.device(idx):
        return fn(ctypes.byref(args), _stream(torch.device("cuda", idx)))


def paged_decode_hip(
    q: torch.Tensor,
    cache: PagedKVCache,
    out: torch.Tensor | None = None,
    block_n: int = 64,
    num_splits: int | None = None,
    per_page_bt: bool = True,
    num_warps: int = 4,
    num_stages: int = 3,
    sm_scale: float | None = None,
    max_seq_len: int | None = None,
    flat_splits: int | None = None,
    flat_seq_cost: int | None = None,
    seq_lens_host: torch.Tensor | None = None,
) -> torch.Tensor:
    """Paged GQA decode attention. q: [B, Hq, D] fp16|bf16 -> [B, Hq, D] in q's dtype.

    Reference: pagedattn/triton_decode.py:285-377. `sm_scale` overrides the
    default 1/sqrt(head_dim) (a serving runtime may fold other factors in).
    With `num_splits=None` the split count comes from `plan_num_splits` on the
    lengths, read on the host in one device sync (the reference syncs there
    too, for `seq_lens.max()`); serving callers pass `num_splits` to avoid
    it. A sequence with seq_len == 0 produces zeros.

    `max_seq_len` (an addition; a host int such as vLLM's
    `attn_metadata.max_seq_len`) sizes every sequence's split chunk from the
    longest one, so a ragged batch gives its long sequences all the splits and
    its short ones few. Without it each sequence is cut into `num_splits`
    chunks of its own length (the reference's rule, triton_decode.py:78-85),
    except when `num_splits=None`, where the longest length is known anyway.
    Both rules compute the same attention.

    `flat_splits` (an addition) selects the flat, work-balanced split: per
    (kv head, head tile) the batch's 32-token tiles are concatenated and cut
    into `flat_splits` equal ranges, one wave each, so ragged lengths cost no
    tail; `num_splits` and `max_seq_len` are then unused. It needs no
    host-side lengths, so a serving loop can pass a fixed value
    (`flat_splits_for`). `flat_seq_cost` (0 when not given with
    `flat_splits`) charges each sequence that many tiles of weight when the
    ranges are cut, which balances ranges that start several sequences
    (`plan_launch` sets RAGGED_FLAT_SEQ_COST(_KV) for ragged batches).

    `seq_lens_host` (an addition): the lengths as a contiguous int32 CPU
    tensor equal to `cache.seq_lens`, when the caller has them (a serving
    step's metadata usually does). A flat launch then takes its ranges and
    its merge list from the host (no seq_lens scan on the GPU, no merge
    launch when no sequence is cut or empty). With `num_splits=None` the
    lengths come to the host anyway and are used so.
    """
    del per_page_bt, num_warps, num_stages
    b, hq, d = q.shape
    shape = cache.shape
    assert d == shape.head_dim
    assert block_n % cache.block_size == 0, "BLOCK_N must be a multiple of the page size"
    if hq != shape.num_q_heads:
        raise ValueError(f"q has {hq} heads, cache shape expects {shape.num_q_heads}")

    if out is None:
        out = torch.empty((b, hq, d), dtype=q.dtype, device=q.device)
    if b == 0:
        return out
    merge = True  # a flat decode runs its merge pass
    if flat_splits:
        num_splits = 1
        flat_seq_cost = int(flat_seq_cost or 0)
    elif num_splits is None:
        # the lengths come to the host in the one sync the reference also makes
        lens = cache.seq_lens.to("cpu")
        if seq_lens_host is None:
            seq_lens_host = lens.to(torch.int32).contiguous()
        wps = flat_waves_per_simd(cache.kv_dtype, d, None if cache.k_scale is None else cache.k_scale.dtype)
        plan = plan_launch(b, 0, shape.num_kv_heads, shape.gqa_group, _cu_count(q.device), wps,
                           kv_dtype=cache.kv_dtype, head_dim=d, seq_lens=lens)
        num_splits, flat_splits = plan.num_splits, plan.flat_splits
        if flat_seq_cost is None:
            flat_seq_cost = plan.flat_seq_cost
        if max_seq_len is None:
            max_seq_len = plan.max_seq_len
        if flat_splits:
            merge = flat_needs_merge(lens, flat_splits, cache.block_table.shape[1] * cache.block_size,
                                     int(flat_seq_cost))
    num_splits = int(num_splits)
    scale = d ** -0.5 if sm_scale is None else float(sm_scale)  # shape.softmax_scale

    part_out = part_lse = None
    flat = int(flat_splits or 0)
    if flat > 0:
        num_splits = 1
        part_out, part_lse = _WS.get_flat(b + flat, hq, d, q.device)
    elif num_splits > 1:
        part_out, part_lse = _WS.get(b, hq, num_splits, d, q.device)
    args = _fill_args(q, cache, out, num_splits, scale, part_out, part_lse, max_seq_len or 0, flat,
                      int(flat_seq_cost or 0) if flat else 0, seq_lens_host)
    lib = _abi.load()
    if flat > 0 and not merge:
        # every sequence inside one range: the decode pass writes all of out
        rc = _launch(q, lib.pa_decode_partials, args)
        _abi.check(rc, "pa_decode_partials")
        return out
    rc = _launch(q, lib.pa_decode, args)
    _abi.check(rc, "pa_decode")
    return out


# Import-path compatibility with the reference (pagedattn.triton_decode.
# paged_decode_triton): the same function, HIP underneath.
paged_decode_triton = paged_decode_hip


def decode_noalloc(
    q: torch.Tensor,
    cache: PagedKVCache,
    out: torch.Tensor,
    num_splits: int = 1,
    max_seq_len: int = 0,
    flat_splits: int = 0,
    sm_scale: float | None = None,
    flat_seq_cost: int = 0,
    seq_lens_host: torch.Tensor | None = None,
) -> torch.Tensor:
    """The decode through pa_decode_noalloc, which allocates nothing.

    The same launch and results as `paged_decode_hip(q, cache, out=out,
    num_splits=..., max_seq_len=..., flat_splits=..., flat_seq_cost=...)`, but the split
    partials live in the library's static per-GPU scratch
    (PA_NOALLOC_SCRATCH_BYTES) instead of a torch workspace, so the call
    makes no allocation and no host sync: for callers that cannot allocate
    (HIP graph capture, allocation-free serving loops). `out` must be given.
    Calls that overlap on one GPU share the scratch and race. A launch whose
    partials do not fit raises NotImplementedError before anything runs.
    """
    if out is None:
        raise ValueError("decode_noalloc writes into a caller-supplied out")
    scale = cache.shape.softmax_scale if sm_scale is None else float(sm_scale)
    flat = int(flat_splits or 0)
    args = _fill_args(q, cache, out, 1 if flat else int(num_splits), scale, None, None,
                      int(max_seq_len or 0), flat, int(flat_seq_cost or 0) if flat else 0, seq_lens_host)
    lib = _abi.load()
    rc = _launch(q, lib.pa_decode_noalloc, args)
    _abi.check(rc, "pa_decode_noalloc")
    return out


def decode_partials(
    q: torch.Tensor,
    cache: PagedKVCache,
    num_splits: int,
    sm_scale: float | None = None,
    part_out: torch.Tensor | None = None,
    part_lse: torch.Tensor | None = None,
    max_seq_len: int = 0,
    flat_splits: int = 0,
    out: torch.Tensor | None = None,
    flat_seq_cost: int = 0,
    seq_lens_host: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Run only the decode pass; returns (part_out [B,Hq,S,D], part_lse [B,Hq,S]).

    part_lse is log2(sum_j 2^(s_j)) of the split's scaled logits s = q.k *
    sm_scale * log2(e) and part_out the split's normalised output, the format
    of the reference's split epilogue (triton_decode.py:169-188).
    With `flat_splits` = F > 0 it is the flat decode pass: the partials are
    slots [B + F, Hq, D] / [B + F, Hq], and sequences that one wave range
    holds whole are written to `out`; `flat_seq_cost` and `seq_lens_host`
    as for `paged_decode_hip`.
    """
    b, hq, d = q.shape
    scale = cache.shape.softmax_scale if sm_scale is None else float(sm_scale)
    if flat_splits > 0:
        num_splits = 1
        if part_out is None:
            part_out = torch.empty((b + flat_splits, hq, d), dtype=torch.float32, device=q.device)
        if part_lse is None:
            part_lse = torch.empty((b + flat_splits, hq), dtype=torch.float32, device=q.device)
    if part_out is None:
        part_out = torch.empty((b, hq, num_splits, d), dtype=torch.float32, device=q.device)
    if part_lse is None:
        part_lse = torch.empty((b, hq, num_splits), dtype=torch.float32, device=q.device)
    if out is None:
        out = torch.empty((b, hq, d), dtype=q.dtype, device=q.device)
    _check_partials(q.device, part_out, part_lse, b, hq, d, num_splits, flat_splits)
    args = _fill_args(q, cache, out, num_splits, scale, part_out, part_lse, max_seq_len, flat_splits,
                      flat_seq_cost if flat_splits > 0 else 0, seq_lens_host)
    lib = _abi.load()
    rc = _launch(q, lib.pa_decode_partials, args)
    _abi.check(rc, "pa_decode_partials")
    return part_out, part_lse


def flat_merge(
    q: torch.Tensor,
    cache: PagedKVCache,
    flat_splits: int,
    part_out: torch.Tensor,
    part_lse: torch.Tensor,
    out: torch.Tensor,
    sm_scale: float | None = None,
    flat_seq_cost: int = 0,
    seq_lens_host: torch.Tensor | None = None,
) -> torch.Tensor:
    """The flat split's merge pass alone: after `decode_partials(...,
    flat_splits=F, out=out, flat_seq_cost=c)` with the same arguments, folds
    the slots into `out` (the pair equals `paged_decode_hip(...,
    flat_splits=F, flat_seq_cost=c)`)."""
    if flat_splits <= 0:
        raise ValueError("flat_merge needs flat_splits > 0")
    scale = cache.shape.softmax_scale if sm_scale is None else float(sm_scale)
    b, hq, d = q.shape
    _check_partials(q.device, part_out, part_lse, b, hq, d, 1, flat_splits)
    args = _fill_args(q, cache, out, 1, scale, part_out, part_lse, 0, flat_splits, flat_seq_cost,
                      seq_lens_host)
    lib = _abi.load()
    rc = _launch(q, lib.pa_flat_merge, args)
    _abi.check(rc, "pa_flat_merge")
    return out


def split_reduce(
    part_out: torch.Tensor, part_lse: torch.Tensor, out: torch.Tensor | None = None
) -> torch.Tensor:
    """Merge split partials into [B, H, D] fp16 or bf16 (triton_decode.py:198-240)."""
    if part_out.dim() != 4:
        raise ValueError(f"part_out {tuple(part_out.shape)} is not [B, H, S, D]")
    b, h, s, d = part_out.shape
    _check_partials(part_out.device, part_out, part_lse, b, h, d, s, 0)
    if out is None:
        out = torch.empty((b, h, d), dtype=torch.float16, device=part_out.device)
    if out.dtype not in _IO_CODE or out.stride(2) != 1:
        raise ValueError("out must be float16 or bfloat16 with a contiguous head dim")
    if tuple(out.shape) != (b, h, d) or out.device != part_out.device:
        raise ValueError(f"out {tuple(out.shape)} on {out.device} is not [{b}, {h}, {d}] on {part_out.device}")
    if not part_out.is_cuda:
        raise ValueError(f"part_out is on {part_out.device}: the merge kernel needs GPU tensors")
    r = _abi.PaReduceArgs()
    r.part_out = part_out.data_ptr()
    r.part_lse = part_lse.data_ptr()
    r.out = out.data_ptr()
    r.batch, r.num_heads, r.head_dim, r.num_splits = b, h, d, s
    r.stride_pb, r.stride_ph, r.stride_ps = part_out.stride(0), part_out.stride(1), part_out.stride(2)
    r.stride_lb, r.stride_lh = part_lse.stride(0), part_lse.stride(1)
    r.stride_ob, r.stride_oh = out.stride(0), out.stride(1)
    r.io_dtype = _IO_CODE[out.dtype]
    lib = _abi.load()
    rc = _launch(part_out, lib.pa_split_reduce, r)
    _abi.check(rc, "pa_split_reduce")
    return out


def split_count_for(cache: PagedKVCache, device: torch.device) -> int:
    """The classic split count `plan_num_splits` gives this batch."""
    return plan_num_splits(cache.seq_lens.to("cpu"), cache.shape.num_kv_heads, cache.shape.gqa_group,
                           _cu_count(device))[0]


__all__ = [
    "paged_decode_hip",
    "paged_decode_triton",
    "pick_num_splits",
    "decode_partials",
    "decode_noalloc",
    "split_reduce",
    "flat_merge",
    "split_count_for",
    "plan_num_splits",
    "plan_decode",
    "plan_launch",
    "LaunchPlan",
    "flat_needs_merge",
    "flat_splits_for",
    "flat_waves_per_simd",
    "reserve_workspace",
    "WAVES_PER_WORKGROUP",
    "TILE_TOKENS",
]
