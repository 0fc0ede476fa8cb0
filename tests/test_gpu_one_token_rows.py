"""One-token sequences return their dequantised V row exactly.

A sequence of one token attends to that token alone: its softmax weight is
exactly 1, so the output is the token's V row as the dequantised cache holds it
(cache.py:51-62, restated as oracle.reference.dequantize_kv: fp16, bf16 and
fp8_e5m2 widened to fp16, int8 as fp16(x * scale) with the product formed in
fp32), rounded to the output dtype. Every KV dtype and launch shape must give
it bit for bit. This pins the int8 V dequantisation: applying the scale
anywhere but per element (for instance folded into the fp16 probability)
returns x * fp16(scale) instead, up to 2^-11 relative away.
"""

from __future__ import annotations

import pytest
import torch

from helpers import seeded_q
from oracle import reference as oracle
from pagedattn import ModelShape, allocate
from pagedattn.hip_decode import paged_decode_hip

pytestmark = pytest.mark.gpu

KV_CASES = [
    ("fp16", None),
    ("bf16", None),
    ("fp8_e5m2", None),
    ("int8", torch.float16),
    ("int8", torch.float32),
]
SHAPES = [(32, 8, 128), (64, 8, 128), (14, 2, 64), (8, 8, 256), (16, 1, 32)]
# one-token sequences among longer ones, so flat ranges and splits cross them
LENS = [1, 700, 1, 33, 1, 2048, 0, 1, 95, 1]
LAUNCHES = {
    "unsplit": {"num_splits": 1},
    "split4": {"num_splits": 4},
    "flat7": {"flat_splits": 7},
    "flat64": {"flat_splits": 64},
    "auto": {},
}


@pytest.mark.parametrize("launch", list(LAUNCHES))
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}q{s[1]}kv_d{s[2]}")
@pytest.mark.parametrize("kv,sdt", KV_CASES, ids=lambda x: str(x).replace("torch.", ""))
def test_one_token_rows_are_the_dequantised_v_row(kv, sdt, shape, launch):
    hq, hkv, d = shape
    seed = 4000 + d + hq
    print(f"kv={kv} scales={sdt} shape={shape} launch={launch}", flush=True)
    c = allocate(ModelShape(hq, hkv, d, name="one"), len(LENS), LENS, block_size=16, kv_dtype=kv,
                 seed=seed, scale_dtype=sdt or torch.float16, device="cuda")
    for io in (torch.float16, torch.bfloat16):
        q = seeded_q(len(LENS), hq, d, seed, device="cuda").to(io)
        got = paged_decode_hip(q, c, **LAUNCHES[launch])
        torch.cuda.synchronize()
        bt = c.block_table.cpu().long()
        group = hq // hkv
        for b, t in enumerate(LENS):
            if t != 1:
                continue
            phys = int(bt[b, 0])
            scale = None if c.v_scale is None else c.v_scale[phys, 0].cpu()
            row = oracle.dequantize_kv(c.v_cache[phys, 0].cpu(), scale, kv)  # [hkv, d] fp16
            want = row.repeat_interleave(group, dim=0).to(io)                  # [hq, d]
            assert torch.equal(got[b].cpu(), want), (b, io)
