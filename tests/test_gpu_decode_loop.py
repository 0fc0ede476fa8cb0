"""The serving loop: KV write then decode, with the lengths growing on the GPU.

integration/bench_decode_loop.py runs the attention part of decode steps: each
step adds one token to every sequence on the device, and per layer writes the
new token's K/V (pa_cache_write) and decodes with a fixed flat split
(pa_decode), with no host-side lengths. A short loop here must leave caches
whose last step's output, as the loop computed it, matches the fp32 oracle
(pagedattn/reference.py:28-49 restated) within 2e-3 for every KV dtype (the
writer itself is checked bit for bit in test_gpu_cache_write.py).
"""

from __future__ import annotations

import argparse
import pathlib
import sys

import pytest
import torch

from oracle import reference as oracle

sys.path.insert(0, str(pathlib.Path(__file__).resolve().parent.parent / "paged-decode-attention_amd" / "integration"))
import bench_decode_loop  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("graph", [False, True], ids=["eager", "graph"])
@pytest.mark.parametrize("kv", ["fp16", "bf16", "fp8_e5m2", "int8"])
def test_decode_loop_last_step_matches_the_oracle(kv, graph):
    """With `graph`, every step is one replay of a captured HIP graph. After
    each step (each replay) the loop synchronises and compares every layer's
    output with an eager decode of the same state, bit for bit."""
    args = argparse.Namespace(shape="qwen2.5-0.5b", layers=2, requests=5, prompt=77, output_tokens=6,
                              warmup=2, kv=kv, slo="1,10", seed=3, out=None, graph=graph, check_each=True)
    print(f"kv={kv} graph={graph}", flush=True)
    r, layers, flat = bench_decode_loop.run(args, keep_state=True)
    assert r.output_tokens == 5 * 6 and r.tpot_ms_p50 > 0
    for c, _, q, _, out in layers:
        assert c.seq_lens.tolist() == [77 + 2 + 6] * 5
        want = oracle.reference_decode(q.cpu(), c, out_dtype=torch.float32)
        err = (out.float().cpu() - want).abs()
        bound = 2e-3 + (2.0 ** -8 * want.abs() if q.dtype == torch.bfloat16 else 0.0)
        print(f"  max_abs={err.max().item():.2e} (F={flat})", flush=True)
        assert bool((err <= bound).all())
