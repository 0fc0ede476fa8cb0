"""The reference's package surface (pagedattn/__init__.py:3-13, cache.py) on CPU.

`gather_contiguous` and `dequantize_kv` are the product's own data-model code
(paged-decode-attention_amd/pagedattn/cache.py); the oracle keeps an
independent restatement of both (oracle/reference.py). They must agree bit for
bit for every KV dtype, including the page-table padding rows that the
reference's gather reads past a sequence's end (cache.py:200-205).
"""

from __future__ import annotations

import importlib

import pytest
import torch

from oracle import reference as oracle
from pagedattn import LLAMA3_8B, QWEN25_05B, ModelShape, allocate

CASES = [
    # (kv dtype, scale dtype, shape, lens, page)
    ("fp16", torch.float16, LLAMA3_8B, [1, 65, 300], 16),
    ("bf16", torch.float16, QWEN25_05B, [17, 3, 40], 16),
    ("fp8_e5m2", torch.float16, ModelShape(8, 2, 32, name="s"), [64, 7], 32),
    ("int8", torch.float16, LLAMA3_8B, [33, 100, 2], 16),
    ("int8", torch.float32, ModelShape(12, 4, 64, name="s"), [5, 129], 64),
]


@pytest.mark.parametrize("kv,sdt,shape,lens,page", CASES,
                         ids=[f"{c[0]}-{str(c[1])[6:]}-p{c[4]}" for c in CASES])
def test_gather_contiguous_matches_oracle(kv, sdt, shape, lens, page):
    from pagedattn import gather_contiguous

    c = allocate(shape, len(lens), lens, block_size=page, kv_dtype=kv, device="cpu", seed=3,
                 slack_blocks=5, scale_dtype=sdt)
    k, v = gather_contiguous(c)
    ok, ov = oracle.gather_contiguous(c)
    s_max = max(lens)
    assert k.shape == (len(lens), shape.num_kv_heads, s_max, shape.head_dim)
    assert k.dtype == torch.float16 and v.dtype == torch.float16
    # bit-identical everywhere, padding rows included
    assert torch.equal(k.view(torch.int16), ok.view(torch.int16))
    assert torch.equal(v.view(torch.int16), ov.view(torch.int16))


@pytest.mark.parametrize("kv,sdt", [("fp16", None), ("bf16", None), ("fp8_e5m2", None),
                                    ("int8", torch.float16), ("int8", torch.float32)])
def test_dequantize_kv_matches_oracle(kv, sdt):
    from pagedattn.cache import dequantize_kv, quantize_kv

    g = torch.Generator().manual_seed(9)
    x = (torch.randn((6, 16, 4, 64), generator=g) * 3).to(torch.float16)
    stored, scale = quantize_kv(x, kv, sdt or torch.float16)
    got = dequantize_kv(stored, scale, kv)
    want = oracle.dequantize_kv(stored, scale, kv)
    assert got.dtype == torch.float16
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_dequantize_int8_is_one_rounding_of_the_exact_product():
    """int8 -> fp16(x * s): with an fp16 scale the fp32 product is exact, so
    one rounding gives the same bits as the reference's fp16 multiply
    (cache.py:61); checked against a float64 product rounded once."""
    from pagedattn.cache import dequantize_kv

    x = torch.arange(-127, 128, dtype=torch.int8).repeat(40).view(40, 1, 1, 255)
    g = torch.Generator().manual_seed(4)
    s = (torch.rand(x.shape[:-1], generator=g) * 0.05 + 1e-4).to(torch.float16)
    got = dequantize_kv(x, s, "int8")
    want = (x.double() * s.double()[..., None]).to(torch.float16)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    fp16_mul = (x.to(torch.float16) * s[..., None]).to(torch.float16)
    assert torch.equal(got.view(torch.int16), fp16_mul.view(torch.int16))


def test_dequantize_int8_needs_scales():
    from pagedattn.cache import dequantize_kv

    with pytest.raises(ValueError):
        dequantize_kv(torch.zeros((2, 4), dtype=torch.int8), None, "int8")
    with pytest.raises(ValueError):
        dequantize_kv(torch.zeros((2, 4), dtype=torch.int8), None, "int4")


def test_gather_contiguous_empty_batch():
    from pagedattn import gather_contiguous

    c = allocate(LLAMA3_8B, 2, [0, 0], device="cpu", seed=1)
    k, v = gather_contiguous(c)
    assert k.shape == (2, 8, 0, 128) and v.shape == (2, 8, 0, 128)


def test_reference_import_lines_resolve():
    """The imports the reference's own files make from its package
    (tests/test_correctness.py:22-24, integration/vllm_backend.py:38-40,
    pagedattn/__init__.py:3-13), minus the oracle module `reference` and the
    NVIDIA-side VRAM planner, which are not part of the decode path."""
    pkg = importlib.import_module("pagedattn")
    for name in ("LLAMA3_8B", "LLAMA3_70B", "MHA_DEBUG", "ModelShape", "PagedKVCache", "allocate",
                 "gather_contiguous", "paged_decode_triton", "pick_num_splits"):
        assert hasattr(pkg, name), name
    cache = importlib.import_module("pagedattn.cache")
    for name in ("PagedKVCache", "allocate", "gather_contiguous", "quantize_kv", "dequantize_kv",
                 "FP8_E5M2_MAX", "INT8_MAX"):
        assert hasattr(cache, name), name
    td = importlib.import_module("pagedattn.triton_decode")
    assert td.paged_decode_triton is pkg.paged_decode_triton
    assert hasattr(td, "pick_num_splits")
    config = importlib.import_module("pagedattn.config")
    for name in ("ModelShape", "KVDType", "kv_bytes_per_token", "LLAMA3_8B", "LLAMA3_70B", "MHA_DEBUG"):
        assert hasattr(config, name), name
