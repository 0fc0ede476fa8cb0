"""Pages more than 4 GiB past the pool base.

The kernels address K/V through one raw buffer per 16-token sub-tile, based at
that sub-tile's first row. The page offset, block id times page stride, is
formed in 64 bits, and only the offsets inside a page are 32-bit. Here a small
cache's pages are copied to the top of a pool over 4.5 GiB, and the block table
is shifted to match, so every page lies more than 4 GiB from the base. The
output must be bit-identical to the small cache's on every launch shape: the
same data and the same arithmetic, only the addresses differ (the reference's
shuffle test, test_correctness.py:100-110, at this offset).
"""

from __future__ import annotations

import dataclasses

import pytest
import torch

from helpers import seeded_q
from pagedattn import LLAMA3_8B, allocate
from pagedattn.hip_decode import paged_decode_hip

pytestmark = pytest.mark.gpu

LENS = [700, 1, 2048, 33, 0, 1500]
POOL_BYTES = int(4.5 * 2**30)
LAUNCHES = {"unsplit": {"num_splits": 1}, "split4": {"num_splits": 4}, "flat11": {"flat_splits": 11},
            "auto": {}}


def _lift(c):
    """The same cache with its pages moved to the top of a pool >= POOL_BYTES."""
    nb = c.k_cache.shape[0]
    page_bytes = c.k_cache[0].numel() * c.k_cache.element_size()
    total = max(nb, -(-POOL_BYTES // page_bytes)) + nb
    base = total - nb
    assert base * page_bytes >= 2**32, "the lifted pages must lie past 4 GiB"

    def lift(t):
        if t is None:
            return None
        big = torch.empty((total, *t.shape[1:]), dtype=t.dtype, device=t.device)
        big[base:] = t
        return big

    return dataclasses.replace(c, k_cache=lift(c.k_cache), v_cache=lift(c.v_cache),
                               k_scale=lift(c.k_scale), v_scale=lift(c.v_scale),
                               block_table=(c.block_table + base).to(torch.int32))


@pytest.mark.parametrize("kv,sdt", [("fp16", None), ("fp8_e5m2", None), ("int8", torch.float32)],
                         ids=["fp16", "fp8", "int8"])
def test_pages_past_4gib_give_identical_output(kv, sdt):
    print(f"kv={kv}", flush=True)
    c = allocate(LLAMA3_8B, len(LENS), LENS, block_size=16, kv_dtype=kv, seed=77,
                 scale_dtype=sdt or torch.float16, device="cuda")
    big = _lift(c)
    q = seeded_q(len(LENS), LLAMA3_8B.num_q_heads, LLAMA3_8B.head_dim, 77, device="cuda")
    try:
        for name, kw in LAUNCHES.items():
            a = paged_decode_hip(q, c, **kw).clone()
            b = paged_decode_hip(q, big, **kw)
            torch.cuda.synchronize()
            assert torch.equal(a, b), name
    finally:
        del big
        torch.cuda.empty_cache()
