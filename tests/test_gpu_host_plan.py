"""GPU parity of the flat split with host-side lengths (seq_lens_host).

No counterpart in the reference. With the lengths on the host the library
passes the flat ranges and the merge's sequence list in the kernel
arguments instead of letting the kernels scan seq_lens. The ranges are the
same, so the result must equal the GPU-scan launch byte for byte, and the
CPU oracle (pagedattn/reference.py:28-49) within the decode's 2e-3 bar.
Covered: ragged batches with empty and cut sequences, every KV dtype, GQA
groups above 16, batches above 64, launches beyond the tables (the GPU scan
takes over), merge-free launches (no merge is launched; `out` starts as NaN
so every row must be written), the decode and merge passes alone, and HIP
graph replay.
"""

from __future__ import annotations

import pytest
import torch

from helpers import max_abs, seeded_q
from oracle import reference as oracle
from pagedattn import LLAMA3_8B, LLAMA3_70B, QWEN25_05B, ModelShape, allocate
from pagedattn.hip_decode import decode_partials, flat_merge, paged_decode_hip

pytestmark = pytest.mark.gpu

ABS_TOL = 2e-3
RAGGED = [300, 1, 4096, 0, 17, 33, 64, 1000]


def _case(shape, lens, kv_dtype="fp16", seed=0, scale_dtype=torch.float16, block_size=16):
    c = allocate(shape, len(lens), lens, block_size=block_size, kv_dtype=kv_dtype, seed=seed,
                 scale_dtype=scale_dtype, device="cuda")
    q = seeded_q(len(lens), shape.num_q_heads, shape.head_dim, seed, device="cuda")
    return q, c


def _host(c):
    return c.seq_lens.cpu().to(torch.int32).contiguous()


def _check(q, c, flat, cost=0):
    lens = c.seq_lens.cpu().tolist()
    kw = dict(flat_splits=flat, flat_seq_cost=cost, block_n=max(64, c.block_size))
    a = torch.full_like(q, float("nan"))
    paged_decode_hip(q, c, out=a, seq_lens_host=_host(c), **kw)
    b = torch.full_like(q, float("nan"))
    paged_decode_hip(q, c, out=b, **kw)
    torch.cuda.synchronize()
    want = oracle.reference_decode(q, c, out_dtype=torch.float32)
    live = [i for i, t in enumerate(lens) if t > 0]
    dead = [i for i, t in enumerate(lens) if t == 0]
    err = max_abs(a[live], want[live]) if live else 0.0
    print(f"flat={flat} cost={cost} B={len(lens)} max_abs={err:.2e}")
    assert torch.equal(a, b), "host tables and the GPU scan disagree"
    assert err < ABS_TOL
    if dead:
        assert torch.equal(a[dead], torch.zeros_like(a[dead]))


@pytest.mark.parametrize("flat", [1, 3, 7, 64, 256])
@pytest.mark.parametrize("cost", [0, 1])
def test_host_plan_ragged(flat, cost):
    q, c = _case(LLAMA3_8B, RAGGED, seed=1)
    _check(q, c, flat, cost)


@pytest.mark.parametrize("kv_dtype,scale_dtype", [("fp8_e5m2", torch.float16), ("int8", torch.float16),
                                                  ("int8", torch.float32), ("bf16", torch.float16)])
def test_host_plan_kv_dtypes(kv_dtype, scale_dtype):
    q, c = _case(LLAMA3_8B, RAGGED, kv_dtype=kv_dtype, seed=2, scale_dtype=scale_dtype)
    _check(q, c, 96, 1)


@pytest.mark.parametrize("shape,lens,flat", [
    (LLAMA3_70B, [2000, 50, 0, 777], 40),
    (QWEN25_05B, [500, 3, 1500, 64, 0], 33),
    (ModelShape(40, 2, 128, "g20"), [900, 17, 300], 21),   # head tiles of 16 and 4
    (ModelShape(16, 1, 256, "d256"), [700, 1, 1200], 19),
    (ModelShape(8, 8, 32, "d32"), [333, 2, 1000], 50),
])
def test_host_plan_shapes(shape, lens, flat):
    q, c = _case(shape, lens, seed=3)
    _check(q, c, flat)
    _check(q, c, flat, 2)


def test_host_plan_page_size_64():
    q, c = _case(LLAMA3_8B, RAGGED, seed=4, block_size=64)
    _check(q, c, 13, 1)


@pytest.mark.parametrize("batch,flat,cost", [(130, 37, 0), (300, 128, 1), (200, 256, 0)])
def test_host_plan_batches_above_one_wave(batch, flat, cost):
    g = torch.Generator().manual_seed(batch)
    lens = torch.randint(0, 600, (batch,), generator=g).tolist()
    lens[::9] = [0] * len(lens[::9])
    q, c = _case(LLAMA3_8B, lens, seed=5)
    _check(q, c, flat, cost)


def test_host_plan_beyond_the_tables():
    """300 ranges: more than the table holds, the kernels scan seq_lens."""
    q, c = _case(LLAMA3_8B, RAGGED * 4, seed=6)
    _check(q, c, 300, 1)


def test_host_plan_merge_free_launch():
    """64 x 4096 over 128 ranges: every boundary falls between sequences, so
    no merge is launched; every row of a NaN-filled out is written."""
    q, c = _case(LLAMA3_8B, [4096] * 64, seed=7)
    _check(q, c, 128)


def test_host_plan_passes_alone():
    """decode_partials and flat_merge with host tables equal the scan's."""
    q, c = _case(LLAMA3_8B, RAGGED, seed=8)
    flat, cost = 29, 1
    host = _host(c)
    outs = []
    for hl in (host, None):
        out = torch.full_like(q, float("nan"))
        po, pl = decode_partials(q, c, 1, flat_splits=flat, out=out, flat_seq_cost=cost, seq_lens_host=hl)
        flat_merge(q, c, flat, po, pl, out, flat_seq_cost=cost, seq_lens_host=hl)
        torch.cuda.synchronize()
        outs.append(out.clone())
    assert torch.equal(outs[0], outs[1])
    want = oracle.reference_decode(q, c, out_dtype=torch.float32)
    live = [i for i, t in enumerate(RAGGED) if t > 0]
    assert max_abs(outs[0][live], want[live]) < ABS_TOL


def test_host_plan_auto_launch():
    """num_splits=None reads the lengths to the host and uses them."""
    q, c = _case(LLAMA3_8B, RAGGED * 8, seed=9)
    got = paged_decode_hip(q, c)
    torch.cuda.synchronize()
    want = oracle.reference_decode(q, c, out_dtype=torch.float32)
    live = [i for i, t in enumerate(RAGGED * 8) if t > 0]
    assert max_abs(got[live], want[live]) < ABS_TOL


def test_host_plan_in_a_hip_graph():
    q, c = _case(LLAMA3_8B, RAGGED, seed=10)
    host = _host(c)
    out = torch.empty_like(q)
    kw = {"flat_splits": 29, "flat_seq_cost": 1, "seq_lens_host": host}
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
    for seed in (11, 12, 13):
        q.copy_(seeded_q(q.shape[0], 32, 128, seed, device="cuda"))
        eager = paged_decode_hip(q, c, flat_splits=29, flat_seq_cost=1).clone()
        torch.cuda.synchronize()
        out.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay with q seed {seed} differs"


def test_graph_captured_with_host_lengths_replays_new_lengths():
    """A serving loop captures a step once and replays it after updating
    seq_lens in place. The host lengths given at capture are ignored there
    (the captured kernels scan seq_lens), so every replay equals an eager
    decode at the lengths seq_lens holds at that replay."""
    import dataclasses

    lens0 = [300, 1, 1500, 17, 33, 64, 1000, 700]
    q, c = _case(LLAMA3_8B, lens0, seed=15)
    live = c.seq_lens
    host = _host(c)  # read before the capture: no sync may happen inside it
    out = torch.empty_like(q)
    kw = {"flat_splits": 29, "flat_seq_cost": 1}
    paged_decode_hip(q, c, out=out, seq_lens_host=host, **kw)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        paged_decode_hip(q, c, out=out, seq_lens_host=host, **kw)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged_decode_hip(q, c, out=out, seq_lens_host=host, **kw)
    # new lengths within the block table's capacity (each sequence keeps its pages)
    for lens in ([301, 2, 1501, 18, 34, 64, 1001, 701], [5, 1, 40, 17, 0, 64, 1000, 3],
                 [300, 1, 1500, 17, 33, 64, 1000, 700]):
        live.copy_(torch.tensor(lens, dtype=torch.int32))
        cap = [min(t, c.block_table.shape[1] * c.block_size) for t in lens]
        assert cap == lens
        eager = paged_decode_hip(q, dataclasses.replace(c, seq_lens=live.clone()), **kw).clone()
        torch.cuda.synchronize()
        out.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        print(f"replay at lengths {lens}", flush=True)
        assert torch.equal(out, eager), f"replay at lengths {lens} differs from the eager decode"


def test_host_plan_rejects_bad_host_lengths():
    q, c = _case(LLAMA3_8B, RAGGED, seed=14)
    for bad in (torch.tensor(RAGGED, dtype=torch.int64), torch.tensor(RAGGED[:3], dtype=torch.int32),
                torch.tensor(RAGGED, dtype=torch.int32, device="cuda")):
        with pytest.raises(ValueError):
            paged_decode_hip(q, c, flat_splits=7, seq_lens_host=bad)
