"""int8 caches: the QK product holds q per head in fixed point.

For an int8 cache the kernel multiplies the stored K bytes with Q in two int8
MFMAs. Q is first scaled per head by a power of two that puts max|q| in
[2^13, 2^14) and rounded to an integer (15 bits and a sign). These tests give the heads of one kv group q
magnitudes far apart: a zero head, 1e-3, 0.03, 1, 3 and a head with one
dominant element. Each head then gets its own exponent, checked against the
fp32 oracle (pagedattn/reference.py:28-49 restated) on every launch shape.

The bound is the decode's 2e-3 plus 2^-10 |oracle|. The larger q heads
concentrate the softmax, so outputs approach max|V| (about 4 here). There the
fp16 probabilities, which the reference also uses (triton_decode.py:165), and
the fp16 output each cost up to 2^-11 |out| whatever the q arithmetic. A CPU
emulation of these inputs with exact q gives the same worst errors as the
15-bit fixed point (1.5e-3 at D = 256). A zero head must return the plain
mean of V (softmax of equal logits) within 2e-3.
"""

from __future__ import annotations

import pytest
import torch

from helpers import seeded_q
from oracle import reference as oracle
from pagedattn import ModelShape, allocate
from pagedattn.hip_decode import paged_decode_hip

pytestmark = pytest.mark.gpu

ABS_TOL = 2e-3
LENS = [1, 37, 600, 2048, 5, 300]
HEAD_SCALES = [0.0, 1e-3, 0.03, 1.0, 3.0, 1.0, 0.5, 2.0]  # per query head of a group of 8
LAUNCHES = {"unsplit": {"num_splits": 1}, "split3": {"num_splits": 3}, "flat9": {"flat_splits": 9}}


def _q(batch, hq, d, seed):
    q = seeded_q(batch, hq, d, seed).float()
    scales = torch.tensor(HEAD_SCALES * (hq // len(HEAD_SCALES)))
    q = q * scales.view(1, hq, 1)
    q[:, 5, :] *= 0.01          # head 5 of each group: one element dominates
    q[:, 5, 3] = 2.5
    return q.to(torch.float16)


@pytest.mark.parametrize("launch", list(LAUNCHES))
@pytest.mark.parametrize("d", [32, 64, 128, 256])
@pytest.mark.parametrize("sdt", [torch.float16, torch.float32], ids=["s16", "s32"])
def test_int8_heads_with_distant_q_magnitudes(sdt, d, launch):
    hq, hkv = 16, 2
    seed = 5100 + d
    print(f"d={d} scales={sdt} launch={launch}", flush=True)
    c = allocate(ModelShape(hq, hkv, d, name="qrange"), len(LENS), LENS, block_size=16,
                 kv_dtype="int8", seed=seed, scale_dtype=sdt, device="cuda")
    q = _q(len(LENS), hq, d, seed).cuda()
    got = paged_decode_hip(q, c, **LAUNCHES[launch])
    torch.cuda.synchronize()
    want = oracle.reference_decode(q.cpu(), c, out_dtype=torch.float32)
    err = (got.float().cpu() - want).abs()
    excess = (err - (ABS_TOL + 2.0 ** -10 * want.abs())).max().item()
    print(f"  max_abs={err.max().item():.2e} excess over the bound={excess:.2e}", flush=True)
    assert excess < 0
    # zero-q heads: equal logits, so the output is the mean of the dequantised V rows
    _, v = oracle.gather_contiguous(c)  # [B, Hkv, S, D] fp16
    for b, t in enumerate(LENS):
        mean = v[b, :, :t].float().mean(dim=1)  # [Hkv, D]
        for h in range(0, hq, 8):
            assert (got[b, h].float().cpu() - mean[h // (hq // hkv)]).abs().max().item() < ABS_TOL
