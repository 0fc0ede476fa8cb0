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
and the CPU oracle (pagedattn/reference.py:28-49 restated) checks the first,
middle and last sequences and five seeded others within max |HIP -
oracle_fp32| < 2e-3. The launch checked against the oracle is the one the
product makes (the planner's flat split with host launch tables: C3 with a
per-sequence charge of 2 tiles, C4 at two waves per SIMD), the launch the
reference's own full-batch tests exercise through `paged_decode_triton`
(tests/test_correctness.py:54-61, 100-110, 162-174).
"""

from __future__ import annotations

import dataclasses
import math

import pytest
import torch

from helpers import max_abs, seeded_q, subset_cache
from oracle import reference as oracle
from pagedattn import LLAMA3_8B, LLAMA3_70B, allocate, flat_splits_for, flat_waves_per_simd, plan_launch
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


def _product_plan(c, lens, dev):
    """The launch the product makes for this batch: `plan_launch` with the
    lengths, the KV dtype and head_dim (what paged_decode_hip(num_splits=None)
    and bench.py use)."""
    shape = c.shape
    wps = flat_waves_per_simd(c.kv_dtype, shape.head_dim, None if c.k_scale is None else c.k_scale.dtype)
    return plan_launch(len(lens), 0, shape.num_kv_heads, shape.gqa_group, _cu_count(dev), wps,
                       kv_dtype=c.kv_dtype, head_dim=shape.head_dim, seq_lens=lens)


# the launch each config takes on a 256-CU MI355X (checked when the GPU has 256 CUs)
EXPECTED_PLAN = {
    "c2": dict(flat_splits=128, flat_seq_cost=0),
    "c3": dict(flat_splits=128, flat_seq_cost=2),
    "c4": dict(flat_splits=256, flat_seq_cost=0),  # int8: two waves per SIMD
    "c5": dict(flat_splits=128, flat_seq_cost=0),
}


@pytest.mark.parametrize("cfg", ["c2", "c3", "c4", "c5"])
def test_launch_shapes_agree_at_full_size(cfg):
    q, c, lens = _build(cfg, seed=31)
    shape = c.shape
    dev = q.device
    plan = _product_plan(c, lens, dev)
    if _cu_count(dev) == 256:
        assert plan.launch_kwargs() == EXPECTED_PLAN[cfg], plan
    host = torch.tensor(lens, dtype=torch.int32)
    # the reference's per-sequence split, at least two pieces per sequence
    splits = max(2, pick_num_splits(len(lens), shape.num_kv_heads, max(lens), _cu_count(dev)))
    print(f"{cfg}: product launch {plan.launch_kwargs()} merge={plan.merge}, classic splits={splits}",
          flush=True)

    # the product's launch: planner's shape, host launch tables
    a = paged_decode_hip(q, c, seq_lens_host=host, **plan.launch_kwargs()).clone()
    b = paged_decode_hip(q, c, seq_lens_host=host, **plan.launch_kwargs())
    torch.cuda.synchronize()
    assert torch.equal(a, b), "product launch not bit-stable"
    # paged_decode_hip(num_splits=None) plans the same launch itself
    auto = paged_decode_hip(q, c)
    torch.cuda.synchronize()
    assert torch.equal(a, auto), "num_splits=None differs from the planner's launch"
    # the same ranges scanned on the GPU (a captured launch takes no host tables)
    scan = paged_decode_hip(q, c, **plan.launch_kwargs())
    torch.cuda.synchronize()
    assert torch.equal(a, scan), "host launch tables and the seq_lens scan differ"
    classic = paged_decode_hip(q, c, num_splits=splits, max_seq_len=max(lens)).clone()
    unsplit = paged_decode_hip(q, c, num_splits=1).clone()
    torch.cuda.synchronize()
    d_classic = (a.float() - classic.float()).abs().max().item()
    d_unsplit = (a.float() - unsplit.float()).abs().max().item()
    print(f"{cfg}: max |product - classic| = {d_classic:.2e}, |product - unsplit| = {d_unsplit:.2e}",
          flush=True)
    assert d_classic < ABS_TOL and d_unsplit < ABS_TOL

    # the oracle on the first, middle and last sequences and five seeded others
    n = len(lens)
    g = torch.Generator().manual_seed(1000 + n)
    extra = torch.randperm(n, generator=g).tolist()
    rows = sorted({0, n // 2, n - 1} | set([r for r in extra if r not in (0, n // 2, n - 1)][:5]))
    # C5's rows each hold 4 GiB of fp32 K/V in the oracle: two at a time
    for part in ([rows] if cfg != "c5" else [rows[i:i + 2] for i in range(0, len(rows), 2)]):
        want = oracle.reference_decode(q[part].cpu(), subset_cache(c, part), out_dtype=torch.float32)
        err = max_abs(a[part], want)
        rel = err / want.abs().max().item()
        print(f"{cfg}: rows {part} max_abs vs oracle = {err:.2e} rel {rel:.2e}", flush=True)
        assert err < ABS_TOL and rel < 1e-2


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


def test_c1_exact_workload_every_row():
    """BASELINE.json configs[0] exactly as bench.py builds it (Qwen2.5-0.5B
    shape 14q/2kv d64, B = 24, T ~ U[32, 192] with seed 0, a seeded
    permutation of a 512-block pool, fp16, scale 1/8, no split-KV). The
    oracle sees the whole batch here: all 24 rows within 2e-3 of the fp32
    oracle (and the reference's relative bar), for the planner's launch and
    an explicit num_splits=1, and two calls byte-equal. The reference's own
    Qwen-shape case is tests/test_correctness.py:162-174."""
    import bench
    from pagedattn import QWEN25_05B, plan_decode

    wl = bench.make_workload("c1")
    assert (wl.batch, wl.pool_blocks, wl.kv_dtype) == (24, 512, "fp16")
    assert min(wl.lens) >= 32 and max(wl.lens) <= 192
    used = sum(-(-t // 16) for t in wl.lens)
    c = allocate(QWEN25_05B, wl.batch, wl.lens, block_size=16, kv_dtype="fp16", device="cuda",
                 seed=wl.seed, slack_blocks=wl.pool_blocks - used)
    assert c.k_cache.shape[0] == 512
    bt = c.block_table.cpu()
    ids = torch.cat([bt[b, : -(-t // 16)] for b, t in enumerate(wl.lens)])
    assert ids.unique().numel() == used and int(ids.max()) < 512  # distinct pages of the pool
    g = torch.Generator().manual_seed(100 + wl.seed)
    q = torch.randn((24, 14, 64), dtype=torch.float16, generator=g).cuda()
    want = oracle.reference_decode(q.cpu(), c, out_dtype=torch.float32)
    assert plan_decode(wl.lens, 2, 7, _cu_count(q.device), 1, kv_dtype="fp16", head_dim=64)[:3:2] == (1, 0)
    for kw in ({}, {"num_splits": 1}):
        a = paged_decode_hip(q, c, **kw).clone()
        b = paged_decode_hip(q, c, **kw)
        torch.cuda.synchronize()
        err = max_abs(a, want)
        rel = err / want.abs().max().item()
        print(f"c1 {kw or 'planner'}: max_abs={err:.2e} rel={rel:.2e}", flush=True)
        assert torch.equal(a, b), "two calls differ"
        assert err < ABS_TOL and rel < 1e-2
