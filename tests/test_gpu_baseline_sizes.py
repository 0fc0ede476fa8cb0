"""GPU checks at the full BASELINE.json sizes (C2-C5), where the CPU oracle
can only see a sample of the batch.

At these sizes the whole batch is checked through properties that do not
depend on size:
  * the three launch shapes (flat split at the planner's F, the reference's
    per-sequence split, unsplit) compute the same attention, so they agree
    on every row within the decode's bar;
  * two calls on the same inputs are bit-identical;
  * moving every page to another physical block and rewriting the block
    table leaves the output bit-identical (the reference's shuffle test,
    test_correctness.py:100-110, at pool scale);
and the CPU oracle (pagedattn/reference.py:28-49 restated) checks the first
and last sequences within max |HIP - oracle_fp32| < 2e-3.
"""

from __future__ import annotations

import dataclasses
import math

import pytest
import torch

from helpers import max_abs, seeded_q, subset_cache
from oracle import reference as oracle
from pagedattn import LLAMA3_8B, LLAMA3_70B, allocate, flat_splits_for, flat_waves_per_simd
from pagedattn.hip_decode import _cu_count, paged_decode_hip, pick_num_splits

pytestmark = pytest.mark.gpu

ABS_TOL = 2e-3


def _lens(cfg):
    if cfg == "c3":
        g = torch.Generator().manual_seed(2)
        u = torch.rand(64, generator=g, dtype=torch.float64)
        return torch.exp(math.log(128) + u * (math.log(8192) - math.log(128))).round().long().tolist()
    return {"c2": [4096] * 64, "c4": [16384] * 32, "c5": [131072] * 4}[cfg]


CONFIGS = {
    # name: (shape, kv dtype, scale dtype, pool blocks or None for an exact fit)
    "c2": (LLAMA3_8B, "fp16", torch.float16, None),
    "c3": (LLAMA3_8B, "fp8_e5m2", torch.float16, None),
    "c4": (LLAMA3_70B, "int8", torch.float32, None),
    "c5": (LLAMA3_8B, "fp16", torch.float16, 40_000),
}


def _build(cfg, seed):
    shape, kv, sdt, pool = CONFIGS[cfg]
    lens = _lens(cfg)
    used = sum(-(-t // 16) for t in lens)
    cache = allocate(shape, len(lens), lens, block_size=16, kv_dtype=kv, device="cuda", seed=seed,
                     slack_blocks=(pool - used) if pool else 0, scale_dtype=sdt, fill_device="cuda")
    q = seeded_q(len(lens), shape.num_q_heads, shape.head_dim, seed, device="cuda")
    return q, cache, lens


@pytest.mark.parametrize("cfg", ["c2", "c3", "c4", "c5"])
def test_launch_shapes_agree_at_full_size(cfg):
    q, c, lens = _build(cfg, seed=31)
    shape = c.shape
    dev = q.device
    wps = flat_waves_per_simd(c.kv_dtype, shape.head_dim, None if c.k_scale is None else c.k_scale.dtype)
    flat = flat_splits_for(shape.num_kv_heads, shape.gqa_group, _cu_count(dev), wps)
    # the reference's per-sequence split, at least two pieces per sequence
    splits = max(2, pick_num_splits(len(lens), shape.num_kv_heads, max(lens), _cu_count(dev)))
    print(f"{cfg}: flat={flat} classic splits={splits}", flush=True)

    a = paged_decode_hip(q, c, flat_splits=flat).clone()
    b = paged_decode_hip(q, c, flat_splits=flat)
    torch.cuda.synchronize()
    assert torch.equal(a, b), "flat split not bit-stable"
    classic = paged_decode_hip(q, c, num_splits=splits, max_seq_len=max(lens)).clone()
    unsplit = paged_decode_hip(q, c, num_splits=1).clone()
    torch.cuda.synchronize()
    d_classic = (a.float() - classic.float()).abs().max().item()
    d_unsplit = (a.float() - unsplit.float()).abs().max().item()
    print(f"{cfg}: max |flat - classic| = {d_classic:.2e}, |flat - unsplit| = {d_unsplit:.2e}", flush=True)
    assert d_classic < ABS_TOL and d_unsplit < ABS_TOL

    rows = [0, len(lens) - 1]
    want = oracle.reference_decode(q[rows].cpu(), subset_cache(c, rows), out_dtype=torch.float32)
    err = max_abs(a[rows], want)
    print(f"{cfg}: rows {rows} max_abs vs oracle = {err:.2e}", flush=True)
    assert err < ABS_TOL


def test_page_moves_leave_output_bit_identical_at_full_size():
    """C3 at full size: permute the physical blocks of the pool (data and
    block table together); the output must not change by a bit."""
    q, c, lens = _build("c3", seed=32)
    shape = c.shape
    flat = flat_splits_for(shape.num_kv_heads, shape.gqa_group, _cu_count(q.device),
                           flat_waves_per_simd(c.kv_dtype, shape.head_dim))
    before = paged_decode_hip(q, c, flat_splits=flat).clone()
    nb = c.k_cache.shape[0]
    g = torch.Generator().manual_seed(33)
    perm = torch.randperm(nb, generator=g).to(q.device)          # new block of old block i
    moved_k = torch.empty_like(c.k_cache)
    moved_v = torch.empty_like(c.v_cache)
    # byte views: the move is a copy of whole blocks whatever the element type
    moved_k.view(torch.uint8)[perm] = c.k_cache.view(torch.uint8)
    moved_v.view(torch.uint8)[perm] = c.v_cache.view(torch.uint8)
    bt = perm[c.block_table.long()].to(torch.int32)
    moved = dataclasses.replace(c, k_cache=moved_k, v_cache=moved_v, block_table=bt)
    after = paged_decode_hip(q, moved, flat_splits=flat)
    torch.cuda.synchronize()
    assert torch.equal(before, after)
