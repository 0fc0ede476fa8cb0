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


def test_impl_forward_writes_the_step_kv():
    """The full decode step through the boundary: this step's K/V are written
    (vLLM's op is absent here, so the HIP writer does it) and attended."""
    _, Impl = vb.build_backend_classes(object, _BaseImpl)
    shape = LLAMA3_8B
    lens = [16, 40, 1]  # lengths before this step
    n = len(lens)
    c = allocate(shape, n, lens, seed=32, device="cuda", slack_blocks=6)
    bt = c.block_table.clone()
    if bt.shape[1] < 4:
        bt = torch.cat([bt, torch.zeros((n, 4 - bt.shape[1]), dtype=torch.int32, device="cuda")], 1)
    used = {int(bt[b, j]) for b, t in enumerate(lens) for j in range(-(-t // 16))}
    free = [i for i in range(c.k_cache.shape[0]) if i not in used]
    slots = []
    for b, t in enumerate(lens):
        if t % 16 == 0:
            bt[b, t // 16] = free.pop()
        slots.append(int(bt[b, t // 16]) * 16 + t % 16)
    kv_cache = torch.stack([c.k_cache, c.v_cache])
    g = torch.Generator().manual_seed(33)
    key = torch.randn((n, shape.num_kv_heads, shape.head_dim), generator=g).half().cuda()
    value = torch.randn((n, shape.num_kv_heads, shape.head_dim), generator=g).half().cuda()
    new_lens = torch.tensor([t + 1 for t in lens], dtype=torch.int32, device="cuda")
    meta = types.SimpleNamespace(max_query_len=1, num_actual_tokens=n, use_cascade=False,
                                 local_attn_metadata=None, max_seq_len=max(lens) + 1,
                                 block_table=bt, seq_lens=new_lens,
                                 slot_mapping=torch.tensor(slots, dtype=torch.int64, device="cuda"))
    query = seeded_q(n, shape.num_q_heads, shape.head_dim, 33, device="cuda")
    output = torch.zeros_like(query)
    impl = Impl(shape)
    impl.kv_sharing_target_layer_name = None  # this layer writes its own K/V
    layer = types.SimpleNamespace(_k_scale=None, _v_scale=None)
    impl.forward(layer, query, key, value, kv_cache, meta, output)
    torch.cuda.synchronize()
    # oracle: the same cache with the new rows written on the CPU
    import dataclasses
    ref = dataclasses.replace(c, k_cache=c.k_cache.cpu().clone(), v_cache=c.v_cache.cpu().clone(),
                              block_table=bt.cpu(), seq_lens=new_lens.cpu())
    oracle.write_kv(key.cpu(), value.cpu(), ref, torch.tensor(slots))
    assert torch.equal(kv_cache[0].cpu(), ref.k_cache) and torch.equal(kv_cache[1].cpu(), ref.v_cache)
    want = oracle.reference_decode(query, ref, out_dtype=torch.float32)
    assert max_abs(output, want) < 2e-3


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


def test_impl_forward_bf16_cache():
    """bf16 models: the reference serves bf16 caches through its fp16 path
    (vllm_backend.py:132); so does this backend, with bf16 q/out."""
    _, Impl = vb.build_backend_classes(object, _BaseImpl)
    lens = [70, 5]
    c = allocate(LLAMA3_8B, 2, lens, kv_dtype="bf16", seed=34, device="cuda")
    kv_cache = torch.stack([c.k_cache, c.v_cache])
    meta = types.SimpleNamespace(max_query_len=1, num_actual_tokens=2, use_cascade=False,
                                 local_attn_metadata=None, max_seq_len=70, block_table=c.block_table,
                                 seq_lens=c.seq_lens, slot_mapping=None)
    query = seeded_q(2, 32, 128, 34, device="cuda").to(torch.bfloat16)
    output = torch.zeros_like(query)
    Impl(LLAMA3_8B).forward(None, query, None, None, kv_cache, meta, output)
    torch.cuda.synchronize()
    want = oracle.reference_decode(query, c, out_dtype=torch.float32)
    err = (output.float().cpu() - want).abs()
    assert bool((err <= 2e-3 + 2.0 ** -8 * want.abs()).all())


def test_impl_forward_large_step_takes_the_flat_split(monkeypatch):
    """A step big enough for the flat split (n * ceil(max_seq_len / 32) tiles
    reach the planner's threshold) through the boundary, vs the oracle."""
    _, Impl = vb.build_backend_classes(object, _BaseImpl)
    g = torch.Generator().manual_seed(35)
    lens = torch.randint(1, 2049, (16,), generator=g).tolist()
    lens[3] = 2048
    n = len(lens)
    c = allocate(LLAMA3_8B, n, lens, seed=35, device="cuda")
    kv_cache = torch.stack([c.k_cache, c.v_cache])
    meta = types.SimpleNamespace(max_query_len=1, num_actual_tokens=n, use_cascade=False,
                                 local_attn_metadata=None, max_seq_len=max(lens),
                                 block_table=c.block_table, seq_lens=c.seq_lens, slot_mapping=None)
    query = seeded_q(n, 32, 128, 35, device="cuda")
    output = torch.zeros_like(query)
    flat_calls = []
    real_forward, real_decode = vb.decode_forward, vb.paged_decode_triton

    def spy(*a, **kw):
        flat_calls.append(kw.get("flat_splits"))
        return real_decode(*a, **kw)

    monkeypatch.setattr(vb, "decode_forward", lambda *a, **kw: real_forward(*a, decode=spy, **kw))
    Impl(LLAMA3_8B).forward(None, query, None, None, kv_cache, meta, output)
    torch.cuda.synchronize()
    assert flat_calls and flat_calls[0]
    want = oracle.reference_decode(query, c, out_dtype=torch.float32)
    assert max_abs(output, want) < 2e-3


def test_impl_forward_with_host_lengths_passes_them_to_the_flat_split(monkeypatch):
    """Metadata that carries the lengths on the CPU (`seq_lens_cpu`): the
    boundary plans on them and hands them to the flat launch, whose ranges
    and merge list are then built on the host. The output matches the
    oracle and is byte-equal to the same launch without host lengths."""
    _, Impl = vb.build_backend_classes(object, _BaseImpl)
    g = torch.Generator().manual_seed(36)
    lens = torch.randint(1, 3000, (24,), generator=g).tolist()
    lens[5] = 2999
    n = len(lens)
    c = allocate(LLAMA3_8B, n, lens, seed=36, device="cuda")
    kv_cache = torch.stack([c.k_cache, c.v_cache])
    meta = types.SimpleNamespace(max_query_len=1, num_actual_tokens=n, use_cascade=False,
                                 local_attn_metadata=None, max_seq_len=max(lens),
                                 block_table=c.block_table, seq_lens=c.seq_lens, slot_mapping=None,
                                 seq_lens_cpu=torch.tensor(lens, dtype=torch.int32))
    query = seeded_q(n, 32, 128, 36, device="cuda")
    output = torch.zeros_like(query)
    calls = []
    real_forward, real_decode = vb.decode_forward, vb.paged_decode_triton

    def spy(*a, **kw):
        calls.append(dict(kw))
        return real_decode(*a, **kw)

    monkeypatch.setattr(vb, "decode_forward", lambda *a, **kw: real_forward(*a, decode=spy, **kw))
    Impl(LLAMA3_8B).forward(None, query, None, None, kv_cache, meta, output)
    torch.cuda.synchronize()
    kw = calls[-1]
    print(f"launch {({k: v for k, v in kw.items() if k not in ('seq_lens_host', 'out')})}", flush=True)
    assert kw.get("flat_splits") and kw["seq_lens_host"].tolist() == lens
    want = oracle.reference_decode(query, c, out_dtype=torch.float32)
    assert max_abs(output, want) < 2e-3
    scan = {k: v for k, v in kw.items() if k not in ("seq_lens_host", "out", "sm_scale")}
    again = real_decode(query, c, sm_scale=LLAMA3_8B.head_dim ** -0.5, **scan)
    torch.cuda.synchronize()
    assert torch.equal(again, output), "host-built tables and the seq_lens scan differ"
