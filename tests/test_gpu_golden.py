"""The committed golden fixtures (tests/golden/*.npz, float64 outputs of the C
oracle) run through the HIP kernels, on every launch shape.

Each fixture holds a small seeded cache in the reference's NHD layout, fp16
q, the softmax scale and the float64 attention output; some also hold the
per-split partials of the reference's split epilogue
(pagedattn/triton_decode.py:78-85, 169-188: normalised output and log2-sum-
exp per split, -inf for an empty split). The kernels must reproduce `out`
within max |HIP - oracle| < 2e-3 (the reference's tolerance for its fp16
path against the fp32 oracle, tests/test_correctness.py:28,48-51, tightened
to an absolute bar) unsplit, split per sequence, split flat (with and without
host lengths and a per-sequence charge) and as planned; and the decode pass
alone must reproduce the stored partials.
"""

from __future__ import annotations

import dataclasses
import pathlib

import numpy as np
import pytest
import torch

from helpers import golden_case
from pagedattn.hip_decode import decode_partials, paged_decode_hip

pytestmark = pytest.mark.gpu

GOLDEN = sorted((pathlib.Path(__file__).resolve().parent / "golden").glob("*.npz"))
ABS_TOL = 2e-3


def _on_gpu(path):
    q, c, sm, z = golden_case(path)
    dev = torch.device("cuda")
    move = lambda t: None if t is None else t.to(dev)
    c = dataclasses.replace(c, k_cache=move(c.k_cache), v_cache=move(c.v_cache), k_scale=move(c.k_scale),
                            v_scale=move(c.v_scale), block_table=move(c.block_table),
                            seq_lens=move(c.seq_lens))
    return q.to(dev), c, sm, z


LAUNCHES = [
    ("unsplit", dict(num_splits=1)),
    ("split3", dict(num_splits=3)),
    ("split3_longest", dict(num_splits=3, max_seq_len=-1)),  # -1: the batch's longest length
    ("flat1", dict(flat_splits=1)),
    ("flat5", dict(flat_splits=5)),
    ("flat5_cost2_host", dict(flat_splits=5, flat_seq_cost=2, host=True)),
    ("flat64_host", dict(flat_splits=64, host=True)),
    ("planner", dict()),
]


def test_golden_fixtures_present():
    assert len(GOLDEN) >= 6


@pytest.mark.parametrize("launch,kw", LAUNCHES, ids=[x[0] for x in LAUNCHES])
@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: p.stem)
def test_golden_output(path, launch, kw):
    q, c, sm, z = _on_gpu(path)
    kw = dict(kw)
    print(f"[golden] {path.stem} {launch}", flush=True)
    if kw.pop("host", False):
        kw["seq_lens_host"] = c.seq_lens.cpu()
    if kw.get("max_seq_len") == -1:
        kw["max_seq_len"] = int(c.seq_lens.max())
    out = paged_decode_hip(q, c, sm_scale=sm, **kw)
    torch.cuda.synchronize()
    want = torch.from_numpy(z["out"])
    err = (out.double().cpu() - want).abs().max().item()
    rel = err / want.abs().max().item()
    assert err < ABS_TOL and rel < 1e-2, f"{path.stem} {launch}: max_abs {err:.3e} rel {rel:.2e}"


@pytest.mark.parametrize("path", [p for p in GOLDEN if "part" in np.load(p).files],
                         ids=lambda p: p.stem)
def test_golden_split_partials(path):
    """pa_decode_partials with the fixture's split count: every split's
    normalised output and log2-sum-exp, empty splits included."""
    q, c, sm, z = _on_gpu(path)
    ns = int(z["num_splits"])
    part, lse = decode_partials(q, c, ns, sm_scale=sm)
    torch.cuda.synchronize()
    want_p = torch.from_numpy(z["part"])
    want_l = torch.from_numpy(z["lse2"])
    fin = torch.isfinite(want_l)
    got_l = lse.double().cpu()
    assert torch.equal(torch.isfinite(got_l), fin), "empty splits differ"
    assert (got_l[fin] - want_l[fin]).abs().max().item() < 1e-3
    got_p = part.double().cpu()
    err = (got_p - want_p)[fin].abs().max().item()
    assert err < ABS_TOL, f"partials max_abs {err:.3e}"
