"""Paged-KV GQA decode attention for MI355X (gfx950), HIP kernels behind a C ABI.

Public surface of the reference package (ParamThakkar123/paged-decode-attention,
pagedattn/__init__.py:3-13) restricted to the decode path: shapes, the paged
cache, the decode entry point and the split heuristic. The reference's fp32
oracle and dense SDPA baselines are test infrastructure here and live outside
the package (oracle/).
"""

from .config import LLAMA3_8B, LLAMA3_70B, MHA_DEBUG, QWEN25_05B, KVDType, ModelShape, kv_bytes_per_token
from .cache import PagedKVCache, allocate, dequantize_kv, gather_contiguous, quantize_kv
from .cache_ops import reshape_and_cache
from .hip_decode import (
    decode_partials,
    flat_needs_merge,
    flat_splits_for,
    flat_waves_per_simd,
    paged_decode_hip,
    paged_decode_triton,
    pick_num_splits,
    LaunchPlan,
    plan_decode,
    plan_launch,
    plan_num_splits,
    short_batch_runs_unsplit,
    split_reduce,
)

__all__ = [
    "LLAMA3_8B", "LLAMA3_70B", "MHA_DEBUG", "QWEN25_05B", "KVDType", "ModelShape",
    "kv_bytes_per_token",
    "PagedKVCache", "allocate", "gather_contiguous", "quantize_kv", "dequantize_kv", "reshape_and_cache",
    "paged_decode_hip", "paged_decode_triton", "pick_num_splits", "plan_num_splits",
    "plan_decode", "plan_launch", "LaunchPlan", "short_batch_runs_unsplit", "flat_needs_merge", "flat_splits_for", "flat_waves_per_simd",
    "decode_partials", "split_reduce",
]
