"""GPU run of the vLLM boundary: PagedAttnTritonImpl.forward (built on
stand-in vLLM base classes) over a vLLM-shaped [2, NB, P, Hkv, D] cache with
padded query/output buffers, checked against the CPU oracle."""

from __future__ import annotations

import types

import pytest
import torch

from helpers import max_abs, seeded_q
from integration import vllm_backend as vb
from oracle import reference as oracle
from pagedattn import LLAMA3_8B, QWEN25_05B, allocate

pytestmark = pytest.mark.gpu


class _BaseImpl:
    def __init__(self, shape):
        self.num_heads = shape.num_q_heads
        self.num_kv_heads = shape.num_kv_heads
        self.head_size = shape.head_dim
        self.scale = shape.head_dim ** -0.5
        self.kv_cache_dtype = "auto"
        self.kv_sharing_target_layer_name = "shared"  # no KV write: the cache is pre-filled

    def forward(self, *a, **k):
        raise AssertionError("decode must not be delegated")


@pytest.mark.parametrize("shape,lens", [(LLAMA3_8B, [300, 1, 4096]), (QWEN25_05B, [32, 192, 77, 5])])
def test_impl_forward_matches_oracle(shape, lens):
    _, Impl = vb.build_backend_classes(object, _BaseImpl)
    n = len(lens)
    c = allocate(shape, n, lens, seed=31, device="cuda", slack_blocks=9)
    kv_cache = torch.stack([c.k_cache, c.v_cache])  # vLLM V1: [2, NB, P, Hkv, D]
    pad = 3  # vLLM pads the batch; rows past num_actual_tokens stay untouched
    bt = torch.zeros((n + pad, c.block_table.shape[1]), dtype=torch.int32, device="cuda")
    bt[:n] = c.block_table
    sl = torch.zeros(n + pad, dtype=torch.int32, device="cuda")
    sl[:n] = c.seq_lens
    meta = types.SimpleNamespace(max_query_len=1, num_actual_tokens=n, use_cascade=False,
                                 local_attn_metadata=None, max_seq_len=max(lens), block_table=bt,
                                 seq_lens=sl, slot_mapping=None)
    query = seeded_q(n + pad, shape.num_q_heads, shape.head_dim, 31, device="cuda")
    output = torch.full_like(query, 7.0)
    impl = Impl(shape)
    res = impl.forward(None, query, None, None, kv_cache, meta, output)
    torch.cuda.synchronize()
    assert res is output
    ref = oracle.reference_decode(query[:n], c, out_dtype=torch.float32)
    err = max_abs(output[:n], ref)
    print(f"vllm boundary max_abs={err:.2e}")
    assert err < 2e-3
    assert torch.equal(output[n:], torch.full_like(output[n:], 7.0))
    assert vb.STATS["decode_calls"] >= 1
