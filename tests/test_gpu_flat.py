"""GPU parity of the flat (work-balanced) split against the CPU oracle.

The flat split has no counterpart in the reference; its result is the same
attention (pagedattn/reference.py:28-49), so every case is held to the
decode's bar: max |HIP - oracle_fp32| < 2e-3, and the partial slots of the
decode pass to the oracle's restatement of the same ranges
(oracle.flat_partials). Cases cover ranges that cut sequences, sequences
inside one range, empty and 1-token sequences, more ranges than tiles, one
range for the whole batch, GQA groups above 16, every KV dtype and page
sizes above 16. The weighted ranges (flat_seq_cost > 0: each sequence
charged that many tiles of weight) are held to the same bar, including
ranges that cover charges only and batches above one wave.
"""

from __future__ import annotations

import pytest
import torch

from helpers import max_abs, seeded_q
from oracle import reference as oracle
from pagedattn import LLAMA3_8B, LLAMA3_70B, QWEN25_05B, ModelShape, allocate
from pagedattn.hip_decode import decode_partials, paged_decode_hip

pytestmark = pytest.mark.gpu

ABS_TOL = 2e-3

RAGGED = [300, 1, 4096, 0, 17, 33, 64, 1000]


def _case(shape, lens, kv_dtype="fp16", block_size=16, seed=0, scale_dtype=torch.float16):
    c = allocate(shape, len(lens), lens, block_size=block_size, kv_dtype=kv_dtype, seed=seed,
                 scale_dtype=scale_dtype, device="cuda")
    q = seeded_q(len(lens), shape.num_q_heads, shape.head_dim, seed, device="cuda")
    return q, c


def _check(q, c, flat, tol=ABS_TOL, seq_cost=0):
    # the reference's BLOCK_N rule: a multiple of the page size
    got = paged_decode_hip(q, c, flat_splits=flat, block_n=max(64, c.block_size), flat_seq_cost=seq_cost)
    torch.cuda.synchronize()
    want = oracle.reference_decode(q, c, out_dtype=torch.float32)
    lens = c.seq_lens.cpu().tolist()
    live = [b for b, t in enumerate(lens) if t > 0]
    dead = [b for b, t in enumerate(lens) if t == 0]
    err = max_abs(got[live], want[live]) if live else 0.0
    print(f"flat={flat} cost={seq_cost} lens={lens[:8]} max_abs={err:.2e}")
    assert err < tol
    if dead:
        assert torch.equal(got[dead].float().cpu(), torch.zeros_like(want[dead]))
    return got


@pytest.mark.parametrize("flat", [1, 2, 3, 7, 64, 1000])
def test_flat_ragged_fp16(flat):
    q, c = _case(LLAMA3_8B, RAGGED, seed=1)
    _check(q, c, flat)


@pytest.mark.parametrize("seq_cost", [1, 3])
@pytest.mark.parametrize("flat", [2, 7, 64, 1000])
def test_flat_seq_cost_ragged(flat, seq_cost):
    q, c = _case(LLAMA3_8B, RAGGED, seed=1)
    _check(q, c, flat, seq_cost=seq_cost)


@pytest.mark.parametrize("kv_dtype,scale_dtype", [("fp8_e5m2", torch.float16), ("int8", torch.float32)])
def test_flat_seq_cost_kv_dtypes(kv_dtype, scale_dtype):
    q, c = _case(LLAMA3_8B, RAGGED, kv_dtype=kv_dtype, seed=2, scale_dtype=scale_dtype)
    _check(q, c, 96, seq_cost=1)


def test_flat_seq_cost_ranges_of_charges_only():
    """Weights [4, 4] over 8 ranges of 1: six ranges cover charges only and
    hold no tiles; the two sequences are still written whole."""
    q, c = _case(ModelShape(8, 8, 64, "mha"), [32, 32], seed=20)
    _check(q, c, 8, seq_cost=3)
    q, c = _case(LLAMA3_8B, [0, 0, 0], seed=5)
    got = paged_decode_hip(q, c, flat_splits=8, flat_seq_cost=2)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), torch.zeros_like(got.cpu()))


@pytest.mark.parametrize("kv_dtype,scale_dtype", [("fp8_e5m2", torch.float16), ("int8", torch.float16),
                                                  ("int8", torch.float32), ("bf16", torch.float16)])
@pytest.mark.parametrize("flat", [5, 96])
def test_flat_kv_dtypes(kv_dtype, scale_dtype, flat):
    q, c = _case(LLAMA3_8B, RAGGED, kv_dtype=kv_dtype, seed=2, scale_dtype=scale_dtype)
    _check(q, c, flat)


@pytest.mark.parametrize("shape,lens,flat", [
    (QWEN25_05B, [32, 192, 77, 5, 0, 160], 9),              # group 7, head_dim 64
    (LLAMA3_70B, [513, 2, 1500], 11),                        # group 8
    (ModelShape(40, 2, 128, "g20"), [700, 31, 2049], 6),     # group 20: two head tiles
    (ModelShape(8, 8, 32, "d32"), [129, 64, 3], 4),          # head_dim 32
    (ModelShape(8, 4, 256, "d256"), [300, 1, 95], 5),        # head_dim 256
    (ModelShape(8, 8, 64, "mha"), [1, 1, 1, 1], 3),          # 1-token sequences
])
def test_flat_shapes(shape, lens, flat):
    q, c = _case(shape, lens, seed=3)
    _check(q, c, flat)


@pytest.mark.parametrize("block_size", [32, 64, 256])
def test_flat_page_sizes(block_size):
    q, c = _case(LLAMA3_8B, [700, 5, 1900, 33], block_size=block_size, seed=4)
    _check(q, c, 13)


def test_flat_all_empty():
    q, c = _case(LLAMA3_8B, [0, 0, 0], seed=5)
    got = paged_decode_hip(q, c, flat_splits=8)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), torch.zeros_like(got.cpu()))


def test_flat_bf16_io():
    q, c = _case(LLAMA3_8B, RAGGED, kv_dtype="bf16", seed=6)
    qb = q.to(torch.bfloat16)
    got = paged_decode_hip(qb, c, flat_splits=21)
    torch.cuda.synchronize()
    assert got.dtype == torch.bfloat16
    want = oracle.reference_decode(qb, c, out_dtype=torch.float32)
    live = [b for b, t in enumerate(RAGGED) if t > 0]
    err = (got[live].float().cpu() - want[live]).abs()
    assert bool((err <= ABS_TOL + 2.0 ** -8 * want[live].abs()).all())


def test_flat_bit_stable_and_matches_classic_split():
    q, c = _case(LLAMA3_8B, RAGGED, seed=7)
    a = paged_decode_hip(q, c, flat_splits=37).clone()
    b = paged_decode_hip(q, c, flat_splits=37)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    classic = paged_decode_hip(q, c, num_splits=6, max_seq_len=max(RAGGED))
    torch.cuda.synchronize()
    assert max_abs(a.float(), classic.float().cpu()) < ABS_TOL


@pytest.mark.parametrize("flat,seq_cost", [(3, 0), (16, 0), (3, 1), (16, 2)])
def test_flat_partial_slots_match_oracle(flat, seq_cost):
    """The decode pass alone: every slot a range writes equals the oracle's
    partial of the same token range, and sequences held by one range are
    already final in `out`."""
    lens = [300, 1, 900, 0, 64, 33]
    q, c = _case(LLAMA3_8B, lens, seed=8)
    b, hq, d = q.shape
    part = torch.full((b + flat, hq, d), float("nan"), device="cuda")
    lse = torch.full((b + flat, hq), float("nan"), device="cuda")
    out = torch.zeros_like(q)
    decode_partials(q, c, 1, part_out=part, part_lse=lse, flat_splits=flat, out=out,
                    flat_seq_cost=seq_cost)
    torch.cuda.synchronize()
    opart, olse, whole = oracle.flat_partials(q, c, flat, seq_cost=seq_cost)
    segs, _ = oracle.flat_segments(lens, flat, seq_cost=seq_cost)
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    written = set()
    for j, bb, _, _ in segs:
        if whole[bb]:
            continue
        written.add(bb + j)
    for slot in sorted(written):
        # P enters the PV product in fp16, as in the decode: the decode's bar
        assert max_abs(part[slot], opart[slot]) < ABS_TOL
        assert (lse[slot].cpu() - olse[slot]).abs().max().item() < 1e-3
    for bb, w in enumerate(whole):
        if w:
            assert max_abs(out[bb], ref[bb]) < ABS_TOL


@pytest.mark.parametrize("kv_dtype,scale_dtype", [("fp16", None), ("bf16", None), ("fp8_e5m2", None),
                                                  ("int8", torch.float16), ("int8", torch.float32)])
@pytest.mark.parametrize("d", [32, 64, 128, 256])
def test_flat_occupancy_query(kv_dtype, scale_dtype, d):
    """The library's occupancy answer sizes flat_splits; every instance holds
    the one wave per SIMD the flat split launches, so the size equals the
    one the planner uses without a GPU."""
    from pagedattn.hip_decode import FLAT_WAVES_PER_SIMD, flat_splits_for, flat_waves_per_simd

    n = flat_waves_per_simd(kv_dtype, d, scale_dtype)
    print(f"{kv_dtype} d={d}: {n} waves/SIMD")
    assert FLAT_WAVES_PER_SIMD <= n <= 8
    assert flat_splits_for(8, 4, 256, n) == flat_splits_for(8, 4, 256, FLAT_WAVES_PER_SIMD)


@pytest.mark.parametrize("seq_cost", [0, 2])
def test_flat_partials_then_merge_equals_decode(seq_cost):
    """pa_decode_partials + pa_flat_merge is pa_decode, bit for bit."""
    from pagedattn.hip_decode import flat_merge

    q, c = _case(LLAMA3_8B, RAGGED, seed=9)
    flat = 29
    b, hq, d = q.shape
    want = paged_decode_hip(q, c, flat_splits=flat, flat_seq_cost=seq_cost).clone()
    part = torch.empty((b + flat, hq, d), dtype=torch.float32, device="cuda")
    lse = torch.empty((b + flat, hq), dtype=torch.float32, device="cuda")
    out = torch.full_like(q, 3.0)
    decode_partials(q, c, 1, part_out=part, part_lse=lse, flat_splits=flat, out=out,
                    flat_seq_cost=seq_cost)
    flat_merge(q, c, flat, part, lse, out, flat_seq_cost=seq_cost)
    torch.cuda.synchronize()
    assert torch.equal(out, want)


@pytest.mark.parametrize("batch,flat,seq_cost", [(130, 37, 0), (300, 256, 0), (130, 37, 1), (300, 256, 2),
                                                 (700, 64, 1)])
def test_flat_batches_above_one_wave(batch, flat, seq_cost):
    """Batches above 64 sequences: the range locate and the merge scan
    seq_lens in several 64-lane chunks (and the locate takes its second pass)."""
    g = torch.Generator().manual_seed(batch)
    lens = torch.randint(0, 700, (batch,), generator=g).tolist()
    lens[5] = 0
    lens[64] = 1
    lens[-1] = 0
    shape = ModelShape(8, 2, 64, "b")
    q, c = _case(shape, lens, seed=10)
    _check(q, c, flat, seq_cost=seq_cost)


def test_flat_sm_scale_override():
    q, c = _case(LLAMA3_8B, [300, 7, 900], seed=11)
    got = paged_decode_hip(q, c, sm_scale=0.05, flat_splits=13)
    torch.cuda.synchronize()
    want = oracle.reference_decode(q, c, sm_scale=0.05, out_dtype=torch.float32)
    assert max_abs(got, want) < ABS_TOL


def test_flat_vllm_style_strided_views():
    """K/V as `kv_cache.unbind(0)` views, q/out as slices of larger buffers."""
    c = allocate(LLAMA3_8B, 3, [100, 1, 513], seed=12, device="cuda")
    kv = torch.stack([c.k_cache, c.v_cache])
    c.k_cache, c.v_cache = kv.unbind(0)
    qbuf = seeded_q(5, 32, 128, 12, device="cuda")
    outbuf = torch.zeros((5, 32, 128), dtype=torch.float16, device="cuda")
    paged_decode_hip(qbuf[:3], c, out=outbuf[:3], flat_splits=9)
    torch.cuda.synchronize()
    want = oracle.reference_decode(qbuf[:3], c, out_dtype=torch.float32)
    assert max_abs(outbuf[:3], want) < ABS_TOL
    assert torch.equal(outbuf[3:], torch.zeros_like(outbuf[3:])), "wrote outside out"


def test_flat_merge_of_many_slots():
    """A sequence cut into more slots than the merge holds in registers (32)
    and than it stages in LDS at once (256)."""
    lens = [40000, 3, 700]
    q, c = _case(LLAMA3_8B, lens, seed=13)
    _check(q, c, 1000)   # per = 2 tiles: the long sequence spans 625 slots
    _check(q, c, 40)     # per = 33 tiles: 38 slots


@pytest.mark.parametrize("kw", [{"flat_splits": 29}, {"num_splits": 5, "max_seq_len": 4096},
                                {"num_splits": 1}])
def test_decode_in_a_hip_graph(kw):
    """A fixed-shape decode captured in a HIP graph (no allocation, sync or
    memset inside a launch) replays correctly: three replays with new q
    values, eager work and synchronisations in between, each equal to the
    eager result bit for bit."""
    q, c = _case(LLAMA3_8B, RAGGED, seed=14)
    out = torch.empty_like(q)
    paged_decode_hip(q, c, out=out, **kw)  # workspace allocated outside the capture
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        paged_decode_hip(q, c, out=out, **kw)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged_decode_hip(q, c, out=out, **kw)
    for seed in (15, 16, 17):
        q.copy_(seeded_q(q.shape[0], 32, 128, seed, device="cuda"))
        eager = paged_decode_hip(q, c, **kw).clone()
        torch.cuda.synchronize()
        out.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay with q seed {seed} differs"


@pytest.mark.parametrize("kw", [{"flat_splits": 7}, {"num_splits": 3}])
def test_graph_replays_after_the_workspace_grows(kw, monkeypatch):
    """A decode captured in a HIP graph keeps the split workspace it was
    captured with: a later, larger eager call grows the workspace (the old
    buffers are retired, not freed), and every replay still equals the eager
    result of the captured call, bit for bit."""
    from pagedattn import hip_decode

    _WS = hip_decode._Workspace()  # a fresh workspace, sized by this test's calls only
    monkeypatch.setattr(hip_decode, "_WS", _WS)
    q, c = _case(LLAMA3_8B, RAGGED, seed=18)
    out = torch.empty_like(q)
    paged_decode_hip(q, c, out=out, **kw)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        paged_decode_hip(q, c, out=out, **kw)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged_decode_hip(q, c, out=out, **kw)
    want = paged_decode_hip(q, c, **kw).clone()
    before = _WS.current(q.device)[0].data_ptr()
    # a call with 8x the batch: the workspace grows
    big_lens = RAGGED * 8
    qb, cb = _case(LLAMA3_8B, big_lens, seed=19)
    big = {k: (v * 8 if k == "flat_splits" else v) for k, v in kw.items()}
    paged_decode_hip(qb, cb, **big)
    torch.cuda.synchronize()
    assert _WS.current(q.device)[0].data_ptr() != before, "the workspace did not grow"
    for rep in range(3):
        out.fill_(5.0)
        junk = torch.randn(1 << 20, device="cuda")  # allocator churn between replays
        graph.replay()
        torch.cuda.synchronize()
        del junk
        assert torch.equal(out, want), f"replay {rep} after the workspace grew differs"


@pytest.mark.parametrize("kw", [{"flat_splits": 7}, {"num_splits": 3}, {"num_splits": 1}])
def test_out_of_range_lengths_and_block_ids_are_clamped(kw):
    """The kernels' own bounds: a length past the block table reads the whole
    table, a negative length is empty, block ids outside the pool are clamped
    into it. Equal to the oracle on the clamped inputs."""
    import dataclasses

    c = allocate(LLAMA3_8B, 4, [70, 128, 40, 16], seed=15, device="cuda", slack_blocks=3)
    nb = c.k_cache.shape[0]
    bt = c.block_table.clone()
    assert bt.shape[1] == 8
    bt[2, 1] = nb + 5      # inside sequence 2 (40 tokens): clamped to nb - 1
    bt[3, 0] = -3          # inside sequence 3: clamped to 0
    lens = torch.tensor([70, 10**6, 40, -5], dtype=torch.int32, device="cuda")
    bad = dataclasses.replace(c, block_table=bt, seq_lens=lens)
    q = seeded_q(4, 32, 128, 15, device="cuda")
    got = paged_decode_hip(q, bad, **kw)
    torch.cuda.synchronize()
    good_bt = bt.clamp(0, nb - 1)
    good = dataclasses.replace(c, block_table=good_bt,
                               seq_lens=torch.tensor([70, 8 * 16, 40, 0], dtype=torch.int32, device="cuda"))
    want = oracle.reference_decode(q, good, out_dtype=torch.float32)
    assert max_abs(got[:3], want[:3]) < ABS_TOL
    assert torch.equal(got[3].cpu(), torch.zeros_like(got[3].cpu()))


def test_aligned_flat_batch_skips_the_merge():
    """A uniform batch whose ranges each hold whole sequences (B = 128 at
    T = 2048: one sequence per range at F = 128) runs the decode pass alone
    when the split is planned from the lengths; the result is bit-identical
    to the flat decode with its merge launched, and matches the oracle."""
    from helpers import subset_cache
    from pagedattn import flat_needs_merge, flat_splits_for, flat_waves_per_simd, plan_decode
    from pagedattn.hip_decode import _cu_count

    lens = [2048] * 128
    c = allocate(LLAMA3_8B, len(lens), lens, seed=41, device="cuda", fill_device="cuda")
    q = seeded_q(len(lens), 32, 128, 41, device="cuda")
    cus = _cu_count(q.device)
    flat = flat_splits_for(8, 4, cus, flat_waves_per_simd("fp16", 128))
    planned = plan_decode(lens, 8, 4, cus, 1, kv_dtype="fp16", head_dim=128)
    print(f"plan {planned}, needs merge {flat_needs_merge(lens, flat)}")
    if planned[2] == 0 or flat_needs_merge(lens, planned[2]):
        pytest.skip(f"{cus} CUs: the plan {planned} is not a merge-free flat split")
    auto = paged_decode_hip(q, c).clone()
    explicit = paged_decode_hip(q, c, flat_splits=planned[2])
    torch.cuda.synchronize()
    assert torch.equal(auto, explicit)
    rows = [0, 77, 127]
    want = oracle.reference_decode(q[rows].cpu(), subset_cache(c, rows), out_dtype=torch.float32)
    assert max_abs(auto[rows], want) < ABS_TOL


def test_large_uniform_batch_takes_the_merge_free_flat_split():
    """B = 1024 (FLAT_MAX_BATCH, the largest flat batch): each flat range holds 8 whole
    sequences, so the planner takes the flat split and the decode pass alone
    writes every output; it agrees with the unsplit kernel on every row and
    with the oracle on sampled rows."""
    from helpers import subset_cache
    from pagedattn import flat_needs_merge, plan_decode
    from pagedattn.hip_decode import _cu_count

    lens = [256] * 1024
    # int8: with 2-byte KV a batch of short sequences like this one runs unsplit
    c = allocate(LLAMA3_8B, len(lens), lens, seed=43, device="cuda", fill_device="cuda", kv_dtype="int8")
    q = seeded_q(len(lens), 32, 128, 43, device="cuda")
    planned = plan_decode(lens, 8, 4, _cu_count(q.device), 1, kv_dtype="int8", head_dim=128)
    print(f"plan {planned}")
    if planned[2] == 0 or flat_needs_merge(lens, planned[2]):
        pytest.skip(f"the plan {planned} is not a merge-free flat split on this GPU")
    auto = paged_decode_hip(q, c).clone()
    unsplit = paged_decode_hip(q, c, num_splits=1)
    torch.cuda.synchronize()
    assert (auto.float() - unsplit.float()).abs().max().item() < ABS_TOL
    rows = [0, 511, 1023]
    want = oracle.reference_decode(q[rows].cpu(), subset_cache(c, rows), out_dtype=torch.float32)
    assert max_abs(auto[rows], want) < ABS_TOL


def test_flat_ragged_batch_of_1000():
    """A ragged batch of 1,000 (two 512-length passes of every seq_lens scan,
    in the decode waves and in the merge) agrees with the unsplit kernel on
    every row and with the oracle on sampled rows."""
    import random

    from helpers import subset_cache

    rng = random.Random(44)
    lens = [rng.choice([0, 1, 17]) if rng.random() < 0.05 else rng.randint(2, 400) for _ in range(1000)]
    c = allocate(LLAMA3_8B, len(lens), lens, seed=44, device="cuda", fill_device="cuda")
    q = seeded_q(len(lens), 32, 128, 44, device="cuda")
    flat = paged_decode_hip(q, c, flat_splits=128).clone()
    unsplit = paged_decode_hip(q, c, num_splits=1)
    torch.cuda.synchronize()
    assert (flat.float() - unsplit.float()).abs().max().item() < ABS_TOL
    rows = [0, 1, 511, 512, 513, 998, 999]
    rows = [r for r in rows if lens[r] > 0]
    want = oracle.reference_decode(q[rows].cpu(), subset_cache(c, rows), out_dtype=torch.float32)
    assert max_abs(flat[rows], want) < ABS_TOL
    dead = [b for b, t in enumerate(lens) if t == 0]
    if dead:
        assert torch.equal(flat[dead].float().cpu(), torch.zeros((len(dead), 32, 128)))


@pytest.mark.parametrize("shape,batch,hi,kv", [
    (LLAMA3_8B, 256, 512, "fp16"), (LLAMA3_8B, 256, 512, "fp8_e5m2"),
    (QWEN25_05B, 1024, 1500, "fp16")], ids=["llama-fp16", "llama-fp8", "qwen-fp16-wide"])
def test_large_batch_of_short_sequences_runs_unsplit(shape, batch, hi, kv):
    """Ragged batches of short sequences with 8 unsplit workgroups per CU at
    256 CUs: the planner runs them unsplit (the Qwen shape's group of 7 q
    heads per kv head doubles the length limit, so its sequences reach 1,500
    tokens), the automatic launch is bit-identical to an explicit unsplit
    one, and sampled rows match the oracle."""
    from helpers import subset_cache
    from pagedattn import flat_waves_per_simd, plan_decode
    from pagedattn.hip_decode import _cu_count

    g = torch.Generator().manual_seed(47)
    lens = torch.randint(32, hi + 1, (batch,), generator=g).tolist()
    c = allocate(shape, len(lens), lens, seed=47, device="cuda", fill_device="cuda", kv_dtype=kv)
    q = seeded_q(len(lens), shape.num_q_heads, shape.head_dim, 47, device="cuda")
    planned = plan_decode(lens, shape.num_kv_heads, shape.gqa_group, _cu_count(q.device),
                          flat_waves_per_simd(kv, shape.head_dim), kv_dtype=kv, head_dim=shape.head_dim)
    print(f"{shape.name} kv={kv} plan {planned}", flush=True)
    if planned != (1, max(lens), 0):
        pytest.skip(f"the plan {planned} on this GPU is not unsplit")
    auto = paged_decode_hip(q, c).clone()
    unsplit = paged_decode_hip(q, c, num_splits=1)
    torch.cuda.synchronize()
    assert torch.equal(auto, unsplit)
    rows = [0, batch // 2, batch - 1]
    want = oracle.reference_decode(q[rows].cpu(), subset_cache(c, rows), out_dtype=torch.float32)
    assert max_abs(auto[rows], want) < ABS_TOL
