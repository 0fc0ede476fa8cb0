"""KV-cache write: this decode step's K/V rows into the paged cache (HIP).

`reshape_and_cache(key, value, cache, slot_mapping)` is the step before the
decode in the reference's serving path, where vLLM's `reshape_and_cache_flash`
writes the new K/V (ParamThakkar123/paged-decode-attention,
integration/vllm_backend.py:117-122). Here it writes into a `PagedKVCache` in
any of this library's formats, quantising with the reference's semantics
(pagedattn/cache.py:33-48): bit-identical to `quantize_kv` of the same rows.
The launch goes through `pa_cache_write` (include/pagedattn.h); there is no
CPU path.
"""

from __future__ import annotations

import weakref

import torch

from . import _abi
from .cache import PagedKVCache
from .hip_decode import _launch

_KV_CODE = {"fp16": _abi.PA_KV_FP16, "fp8_e5m2": _abi.PA_KV_FP8_E5M2, "int8": _abi.PA_KV_INT8,
            "bf16": _abi.PA_KV_BF16}
_STORE_DTYPE = {"fp16": torch.float16, "fp8_e5m2": torch.float8_e5m2, "int8": torch.int8,
                "bf16": torch.bfloat16}
_SCALE_CODE = {torch.float16: _abi.PA_SCALE_FP16, torch.float32: _abi.PA_SCALE_FP32}


# Validated argument structs, keyed by everything their validation read
# except the per-call pointers (key, value, slot_mapping). The cache's tensors
# enter the key by identity and data pointer and are held by weak references,
# so a key cannot match a new tensor that reuses a dead one's id. A decode
# step writes every layer with rows and slots of one geometry, so after the
# first step each call copies a struct and sets three pointers.
_WRITE_TEMPLATES: dict[tuple, tuple] = {}
_WRITE_TEMPLATES_MAX = 512


def reshape_and_cache(
    key: torch.Tensor, value: torch.Tensor, cache: PagedKVCache, slot_mapping: torch.Tensor
) -> None:
    """Write key/value [num_tokens, num_kv_heads, head_dim] (fp16) into the
    cache at slot_mapping [num_tokens] (int64, block * block_size + offset).

    Negative slots are skipped (vLLM pads batches with -1), and so are slots
    at or past num_blocks * block_size. For int8 caches the per-(token, head)
    scales are written too. Asynchronous on the current stream.
    """
    k, v, ks, vs = cache.k_cache, cache.v_cache, cache.k_scale, cache.v_scale
    tkey = (id(k), k.data_ptr(), id(v), v.data_ptr(), id(ks), 0 if ks is None else ks.data_ptr(), id(vs),
            0 if vs is None else vs.data_ptr(), cache.kv_dtype, cache.block_size, cache.shape.num_kv_heads,
            cache.shape.head_dim, key.shape, key.stride(), key.dtype, key.get_device(), value.shape,
            value.stride(), value.dtype, value.get_device(), slot_mapping.shape, slot_mapping.stride(),
            slot_mapping.dtype, slot_mapping.get_device())
    hit = _WRITE_TEMPLATES.get(tkey)
    if hit is not None:
        r = hit[0]
        if (r[0]() is k and r[1]() is v and (ks is None or r[2]() is ks)
                and (vs is None or r[3]() is vs)):
            a = _abi.PaCacheWriteArgs.from_buffer_copy(hit[1])
            a.key, a.value, a.slot_mapping = key.data_ptr(), value.data_ptr(), slot_mapping.data_ptr()
            _abi.check(_launch(key, _abi.load().pa_cache_write, a), "pa_cache_write")
            return
    a = _pack_write_args(key, value, cache, slot_mapping)
    if len(_WRITE_TEMPLATES) >= _WRITE_TEMPLATES_MAX:
        _WRITE_TEMPLATES.clear()
    _WRITE_TEMPLATES[tkey] = (tuple(None if o is None else weakref.ref(o) for o in (k, v, ks, vs)),
                              _abi.PaCacheWriteArgs.from_buffer_copy(a))
    _abi.check(_launch(key, _abi.load().pa_cache_write, a), "pa_cache_write")


def _pack_write_args(
    key: torch.Tensor, value: torch.Tensor, cache: PagedKVCache, slot_mapping: torch.Tensor
) -> _abi.PaCacheWriteArgs:
    """Validate every tensor of a write and pack pa_cache_write_args."""
    if cache.kv_dtype not in _KV_CODE:
        raise NotImplementedError(f"kv_dtype {cache.kv_dtype!r} is not supported by the HIP writer")
    k, v = cache.k_cache, cache.v_cache
    n, h, d = key.shape
    if key.device.type != "cuda":
        raise ValueError(f"key is on {key.device}: the HIP cache writer needs GPU tensors")
    row_dtype = torch.bfloat16 if cache.kv_dtype == "bf16" else torch.float16
    if key.dtype != row_dtype or value.dtype != row_dtype:
        raise NotImplementedError(f"key/value dtype {key.dtype}/{value.dtype}: a {cache.kv_dtype} cache "
                                  f"takes {row_dtype} rows")
    if tuple(value.shape) != (n, h, d) or h != cache.shape.num_kv_heads or d != cache.shape.head_dim:
        raise ValueError(f"key {tuple(key.shape)} / value {tuple(value.shape)} do not match the cache's "
                         f"[{cache.shape.num_kv_heads}, {cache.shape.head_dim}] rows")
    if key.stride(2) != 1 or value.stride(2) != 1 or k.stride(3) != 1:
        raise ValueError("head_dim must be the contiguous dimension of key, value and the caches")
    if k.dtype != _STORE_DTYPE[cache.kv_dtype] or v.dtype != k.dtype or v.stride() != k.stride():
        raise ValueError("k/v cache dtype or strides do not match kv_dtype")
    if tuple(k.shape[1:]) != (cache.block_size, h, d):
        raise ValueError(f"k_cache shape {tuple(k.shape)} is not [NB, {cache.block_size}, {h}, {d}]")
    if slot_mapping.dtype != torch.int64 or slot_mapping.dim() != 1 or slot_mapping.numel() != n:
        raise ValueError("slot_mapping must be int64 [num_tokens]")
    if slot_mapping.stride(0) != 1 and n > 1:
        raise ValueError("slot_mapping must be contiguous")
    for name, t in (("value", value), ("k_cache", k), ("v_cache", v), ("slot_mapping", slot_mapping)):
        if t.device != key.device:
            raise ValueError(f"{name} is on {t.device}, key on {key.device}")

    a = _abi.PaCacheWriteArgs()
    a.key, a.value = key.data_ptr(), value.data_ptr()
    a.k_cache, a.v_cache = k.data_ptr(), v.data_ptr()
    a.slot_mapping = slot_mapping.data_ptr()
    a.num_tokens, a.num_kv_heads, a.head_dim = n, h, d
    a.block_size, a.num_blocks = cache.block_size, k.shape[0]
    a.stride_kt, a.stride_kh = key.stride(0), key.stride(1)
    a.stride_vt, a.stride_vh = value.stride(0), value.stride(1)
    a.stride_cn, a.stride_ct, a.stride_ch = k.stride(0), k.stride(1), k.stride(2)
    a.kv_dtype = _KV_CODE[cache.kv_dtype]
    if cache.kv_dtype == "int8":
        ks, vs = cache.k_scale, cache.v_scale
        if ks is None or vs is None or ks.dtype not in _SCALE_CODE or vs.dtype != ks.dtype:
            raise ValueError("int8 cache needs float16 or float32 k_scale/v_scale")
        if tuple(ks.shape) != tuple(k.shape[:3]) or vs.stride() != ks.stride() or ks.stride(2) != 1:
            raise ValueError("k_scale/v_scale must be [NB, block_size, H_kv] with equal strides")
        if ks.device != key.device or vs.device != key.device:
            raise ValueError("scales must live on key's device")
        a.k_scale, a.v_scale = ks.data_ptr(), vs.data_ptr()
        a.stride_sn, a.stride_st = ks.stride(0), ks.stride(1)
        a.scale_dtype = _SCALE_CODE[ks.dtype]
    else:
        a.scale_dtype = _abi.PA_SCALE_NONE
    return a


# the vLLM op's name as an alias
write_kv = reshape_and_cache

__all__ = ["reshape_and_cache", "write_kv"]
