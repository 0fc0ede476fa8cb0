"""vLLM V1 attention backend whose pure-decode steps run the gfx950 HIP kernel.

Drop-in for the reference's `integration/vllm_backend.py`
(ParamThakkar123/paged-decode-attention): the same public names
(`install`, `maybe_install_from_env`, `PagedAttnTritonBackend`,
`PagedAttnTritonImpl`, `supports_shape`, `STATS`, `QUALNAME`) and the same
routing rule (`vllm_backend.py:67-149`):

    pure decode (max_query_len == 1), fp16, supported shape -> HIP kernel
    anything else                                          -> super().forward()

The backend subclasses vLLM's Triton backend, so vLLM keeps building the
metadata (slot mapping, block tables, seq_lens) and the
[2, num_blocks, block_size, num_kv_heads, head_size] cache; `kv_cache.unbind(0)`
gives the NHD views the kernel reads in place.

Differences from the reference:
  * bf16 caches are served as the reference serves them (vllm_backend.py:132):
    rows converted to fp16 in registers (round to nearest even), q/out bf16.
  * The classes are built by `build_backend_classes(base_backend, base_impl)`,
    so the routing is testable with stand-in base classes where vLLM is not
    installed; `install(platform_cls=...)` likewise accepts a stand-in platform.

vLLM is optional at import time: without it `HAVE_VLLM` is False and the two
classes are None.
"""

from __future__ import annotations

import os
import pathlib
import sys
from typing import Any, Callable

import torch

_PKG_ROOT = pathlib.Path(__file__).resolve().parent.parent
if str(_PKG_ROOT) not in sys.path:
    sys.path.insert(0, str(_PKG_ROOT))

from pagedattn.cache import PagedKVCache  # noqa: E402
from pagedattn.config import ModelShape  # noqa: E402
from pagedattn.hip_decode import (  # noqa: E402
    FLAT_MAX_BATCH,
    MIN_FLAT_TILES_PER_WAVE,
    SINGLE_SEQ_SPLIT_MAX_TOKENS,
    TILE_TOKENS,
    flat_splits_for,
    flat_waves_per_simd,
    short_batch_runs_unsplit,
)
from pagedattn.triton_decode import paged_decode_triton, pick_num_splits  # noqa: E402

QUALNAME = "integration.vllm_backend.PagedAttnTritonBackend"
BACKEND_NAME = "PAGEDATTN_HIP"
SUPPORTED_HEAD_DIMS = (32, 64, 128, 256)

# Proof that the kernel ran (vllm_backend.py:64): decode calls, decoded
# sequences, and calls handed back to vLLM's own attention.
STATS: dict[str, int] = {"decode_calls": 0, "decode_tokens": 0, "delegated_calls": 0}


def supports_shape(num_q_heads: int, num_kv_heads: int, head_dim: int) -> tuple[bool, str]:
    """(ok, reason) for an attention geometry (vllm_backend.py:54-60)."""
    if num_kv_heads <= 0 or num_q_heads % num_kv_heads:
        return False, f"num_q_heads {num_q_heads} not divisible by num_kv_heads {num_kv_heads}"
    if head_dim not in SUPPORTED_HEAD_DIMS:
        return False, f"head_dim {head_dim} not in {SUPPORTED_HEAD_DIMS}"
    return True, ""


def _reason_to_delegate(impl, attn_metadata, kv_cache, output, output_scale) -> str:
    """Why a forward call must go to vLLM's own attention ("" = ours).

    The reference's list (vllm_backend.py:67-90), in its order, plus one rule
    of this build: only fp16 and bf16 caches are served here.
    """
    checks = (
        (attn_metadata is None, "profiling run (no metadata)"),
        (output is None, "no output buffer"),
        (output_scale is not None, "fused output quantization"),
        (kv_cache is None or kv_cache.numel() == 0, "empty kv cache"),
        (str(getattr(impl, "kv_cache_dtype", "auto")).startswith("fp8"), "fp8 kv cache"),
        (getattr(impl, "alibi_slopes", None) is not None, "alibi slopes"),
        (bool(getattr(impl, "logits_soft_cap", 0)), "logits soft cap"),
        (tuple(getattr(impl, "sliding_window", (-1, -1)) or (-1, -1)) != (-1, -1), "sliding window"),
        (getattr(attn_metadata, "local_attn_metadata", None) is not None, "local (iRoPE) attention"),
        (bool(getattr(attn_metadata, "use_cascade", False)), "cascade attention"),
        (getattr(attn_metadata, "max_query_len", 2) != 1, "not a pure-decode batch"),
        (kv_cache is not None and kv_cache.dtype not in (torch.float16, torch.bfloat16),
         "cache dtype is not fp16 or bf16"),
    )
    for hit, why in checks:
        if hit:
            return why
    return ""


def _vllm_cache_op():
    """vLLM's `reshape_and_cache_flash`, or None where vLLM's ops are absent."""
    try:
        return torch.ops._C_cache_ops.reshape_and_cache_flash
    except (AttributeError, RuntimeError):
        return None


def _write_kv(layer, impl, key, value, key_cache, value_cache, slot_mapping) -> None:
    """This step's K/V into the paged cache (vllm_backend.py:117-122).

    vLLM's own op when it is loaded; otherwise this library's HIP writer,
    which stores the same bytes for the fp16 / bf16 caches this backend
    serves (`_reason_to_delegate` sends every other cache dtype to vLLM).
    """
    op = _vllm_cache_op()
    if op is not None:
        op(key, value, key_cache, value_cache, slot_mapping, impl.kv_cache_dtype,
           layer._k_scale, layer._v_scale)
        return
    from pagedattn.cache_ops import reshape_and_cache

    n = int(slot_mapping.shape[0])
    view = PagedKVCache(
        shape=ModelShape(impl.num_heads, impl.num_kv_heads, impl.head_size, name="vllm"),
        block_size=int(key_cache.shape[1]), kv_dtype=_kv_dtype_of(key_cache), k_cache=key_cache,
        v_cache=value_cache, k_scale=None, v_scale=None, block_table=None, seq_lens=None)
    reshape_and_cache(key[:n], value[:n], view, slot_mapping.to(torch.int64))


def _kv_dtype_of(cache: torch.Tensor) -> str:
    """The reference's mapping (vllm_backend.py:132): bf16 caches are served
    through the fp16 arithmetic, fp16 as is."""
    return "bf16" if cache.dtype == torch.bfloat16 else "fp16"


_CU_COUNT: dict[int, int] = {}


def _cu_count(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _CU_COUNT:
        _CU_COUNT[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _CU_COUNT[idx]


def decode_forward(impl, layer, query, key, value, kv_cache, attn_metadata, output,
                   write_kv: Callable = _write_kv, decode: Callable = paged_decode_triton):
    """The decode half of `forward` (vllm_backend.py:113-149): write K/V, view
    the cache as a PagedKVCache, launch the HIP kernel into `output`."""
    key_cache, value_cache = kv_cache.unbind(0)
    if getattr(impl, "kv_sharing_target_layer_name", None) is None:
        write_kv(layer, impl, key, value, key_cache, value_cache, attn_metadata.slot_mapping)
    n = int(attn_metadata.num_actual_tokens)
    cache = PagedKVCache(
        shape=ModelShape(impl.num_heads, impl.num_kv_heads, impl.head_size, name="vllm"),
        block_size=int(key_cache.shape[1]),
        kv_dtype=_kv_dtype_of(key_cache),
        k_cache=key_cache,
        v_cache=value_cache,
        k_scale=None,
        v_scale=None,
        block_table=attn_metadata.block_table[:n],
        seq_lens=attn_metadata.seq_lens[:n],
    )
    # Host-side only (no device sync): max_seq_len is a host int in the
    # metadata. The flat split needs no lengths; it is taken when the batch
    # can hold enough tiles for its waves (the upper bound
    # n * ceil(max_seq_len / 32) against plan_decode's threshold) and is not
    # a large batch of short sequences (plan_decode's ragged rule, which
    # needs only n and max_seq_len), otherwise the classic split, chunked
    # from the longest sequence.
    msl = int(attn_metadata.max_seq_len)
    group = impl.num_heads // impl.num_kv_heads
    cus = _cu_count(query.device)
    flat = flat_splits_for(impl.num_kv_heads, group, cus, flat_waves_per_simd(cache.kv_dtype, impl.head_size))
    single = n == 1 and msl <= SINGLE_SEQ_SPLIT_MAX_TOKENS  # plan_decode's single-sequence rule
    short = short_batch_runs_unsplit(n, msl, impl.num_kv_heads, group, cus, cache.kv_dtype)
    if (not single and not short and n <= FLAT_MAX_BATCH
            and n * -(-msl // TILE_TOKENS) >= MIN_FLAT_TILES_PER_WAVE * flat):
        decode(query[:n], cache, out=output[:n], sm_scale=impl.scale, flat_splits=flat)
    else:
        splits = pick_num_splits(n, impl.num_kv_heads, msl, cus)
        decode(query[:n], cache, out=output[:n], num_splits=splits, sm_scale=impl.scale,
               max_seq_len=msl)
    STATS["decode_calls"] += 1
    STATS["decode_tokens"] += n
    return output


def build_backend_classes(base_backend: type, base_impl: type) -> tuple[type, type]:
    """The (backend, impl) pair on top of vLLM's Triton backend classes."""

    class PagedAttnTritonImpl(base_impl):  # type: ignore[misc, valid-type]
        """Pure decode -> HIP kernel; everything else -> the base class."""

        def forward(self, layer, query, key, value, kv_cache, attn_metadata,
                    output=None, output_scale=None, *args: Any, **kwargs: Any):
            why = _reason_to_delegate(self, attn_metadata, kv_cache, output, output_scale)
            if not why:
                ok, why = supports_shape(self.num_heads, self.num_kv_heads, self.head_size)
                why = "" if ok else why
            if why:
                STATS["delegated_calls"] += 1
                return super().forward(layer, query, key, value, kv_cache, attn_metadata,
                                       output, output_scale, *args, **kwargs)
            return decode_forward(self, layer, query, key, value, kv_cache, attn_metadata, output)

    class PagedAttnTritonBackend(base_backend):  # type: ignore[misc, valid-type]
        """vLLM's Triton backend (metadata, cache layout) with our impl."""

        @staticmethod
        def get_name() -> str:
            return BACKEND_NAME

        @staticmethod
        def get_impl_cls():
            return PagedAttnTritonImpl

    return PagedAttnTritonBackend, PagedAttnTritonImpl


try:  # vLLM is optional: the module imports (and is testable) without it
    from vllm.v1.attention.backends.triton_attn import TritonAttentionBackend, TritonAttentionImpl

    HAVE_VLLM = True
except Exception:  # pragma: no cover - depends on the environment
    HAVE_VLLM = False

if HAVE_VLLM:  # pragma: no cover - needs vLLM
    PagedAttnTritonBackend, PagedAttnTritonImpl = build_backend_classes(
        TritonAttentionBackend, TritonAttentionImpl)
else:
    PagedAttnTritonBackend = None  # type: ignore[assignment]
    PagedAttnTritonImpl = None  # type: ignore[assignment]


def install(platform_cls: type | None = None) -> str:
    """Make vLLM pick this backend for plain (non-MLA) V1 attention.

    vLLM resolves the attention backend through the platform's
    `get_attn_backend_cls(...)`, which returns a qualname string; this wraps
    that classmethod once (idempotent) so the V1 non-MLA case returns
    QUALNAME (vllm_backend.py:180-205). Returns QUALNAME.
    """
    if platform_cls is None:
        from vllm.platforms import current_platform

        platform_cls = type(current_platform)
    if getattr(platform_cls, "_pagedattn_patched", False):
        return QUALNAME
    original = platform_cls.get_attn_backend_cls

    def get_attn_backend_cls(cls, selected_backend, head_size, dtype, kv_cache_dtype,
                             block_size, use_v1, use_mla, *args, **kwargs):
        if use_v1 and not use_mla:
            return QUALNAME
        return original(selected_backend, head_size, dtype, kv_cache_dtype, block_size,
                        use_v1, use_mla, *args, **kwargs)

    platform_cls.get_attn_backend_cls = classmethod(get_attn_backend_cls)
    platform_cls._pagedattn_patched = True
    return QUALNAME


def maybe_install_from_env(platform_cls: type | None = None) -> bool:
    """`install()` when PAGEDATTN_VLLM_BACKEND is 1/true: the hook for a
    `vllm.general_plugins` entry point in the worker (vllm_backend.py:208-214)."""
    if os.environ.get("PAGEDATTN_VLLM_BACKEND", "") not in ("1", "true", "True"):
        return False
    install(platform_cls)
    return True
