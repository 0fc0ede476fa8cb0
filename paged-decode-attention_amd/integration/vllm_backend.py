"""vLLM V1 attention backend whose pure-decode steps run the gfx950 HIP kernel.

Drop-in for the reference's `integration/vllm_backend.py`
(ParamThakkar123/paged-decode-attention): the same public names
(`install`, `maybe_install_from_env`, `PagedAttnTritonBackend`,
`PagedAttnTritonImpl`, `supports_shape`, `STATS`, `QUALNAME`) and the same
routing rule (`vllm_backend.py:67-149`):

    pure decode (max_query_len == 1), fp16, supported shape -> HIP kernel
    anything else                                          -> super().forward()

The backend subclasses vLLM's Triton backend (or, through
`install(prefill_backend=...)`, another vLLM backend with the same cache
layout, such as vLLM-ROCm's AITER flash-attention backend, which then serves
prefill and mixed batches), so vLLM keeps building the metadata (slot
mapping, block tables, seq_lens) and the
[2, num_blocks, block_size, num_kv_heads, head_size] cache; `kv_cache.unbind(0)`
gives the NHD views the kernel reads in place.

Differences from the reference:
  * bf16 caches are served as the reference serves them (vllm_backend.py:132):
    rows converted to fp16 in registers (round to nearest even), q/out bf16.
  * `install(prefill_backend=...)` / PAGEDATTN_PREFILL_BACKEND choose the base
    backend that serves prefill and mixed batches (`BASE_BACKENDS`).
  * The launch is planned by `pagedattn.plan_launch`, the planner the decode
    wrapper itself uses, from the step's size and longest length.
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
from pagedattn.hip_decode import flat_waves_per_simd, plan_launch  # noqa: E402
from pagedattn.triton_decode import paged_decode_triton, pick_num_splits  # noqa: E402

QUALNAME = "integration.vllm_backend.PagedAttnTritonBackend"
# The reference backend's registered name (vllm_backend.py:154-156), kept so
# that logs, configs and tooling keyed on it see the same backend; the
# kernels underneath are the HIP ones.
BACKEND_NAME = "PAGEDATTN_TRITON"
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


def _host_seq_lens(attn_metadata, n: int):
    """The step's lengths as a contiguous int32 CPU tensor when the metadata
    holds a CPU copy (`seq_lens_cpu`, as newer vLLM common metadata does),
    else None. The kernels trust it to equal `seq_lens` (a stale copy would
    attend over the wrong tokens); with PAGEDATTN_CHECK_HOST_LENS=1 every new
    step compares the two (one device sync) and raises if they differ."""
    t = getattr(attn_metadata, "seq_lens_cpu", None)
    if not (isinstance(t, torch.Tensor) and t.device.type == "cpu"):
        return None
    t = t[:n]
    if t.dtype != torch.int32 or not t.is_contiguous():
        t = t.to(torch.int32).contiguous()
    if os.environ.get("PAGEDATTN_CHECK_HOST_LENS") == "1":
        dev = attn_metadata.seq_lens[:n].to("cpu", torch.int32)
        if not torch.equal(dev, t):
            raise ValueError("attn_metadata.seq_lens_cpu differs from seq_lens: the host lengths "
                             "the decode would plan and launch from are stale")
    return t


# The plan of the current decode step. Every attention layer of a step gets
# the same metadata object, so the plan (and the host lengths view) is made
# once per step, not once per layer: planning a ragged batch of 256 cost
# ~0.1 ms, per layer. The key holds the metadata itself (one object, the last
# step's), the step's sizes and the layer geometry.
_STEP_PLAN: list = [None]


def _step_plan(attn_metadata, n: int, impl, kv_dtype: str, device: torch.device):
    msl = int(attn_metadata.max_seq_len)
    key = (id(attn_metadata.seq_lens), n, msl, impl.num_kv_heads, impl.num_heads, impl.head_size,
           kv_dtype, device)
    hit = _STEP_PLAN[0]
    if hit is not None and hit[0] is attn_metadata and hit[1] == key:
        return hit[2], hit[3]
    host = _host_seq_lens(attn_metadata, n)
    plan = plan_launch(n, msl, impl.num_kv_heads, impl.num_heads // impl.num_kv_heads, _cu_count(device),
                       flat_waves_per_simd(kv_dtype, impl.head_size), kv_dtype=kv_dtype,
                       head_dim=impl.head_size, seq_lens=host)
    _STEP_PLAN[0] = (attn_metadata, key, plan, host)
    return plan, host


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
    # Planned on the host with no device sync: the step's size and longest
    # length are host ints in the metadata. Metadata that also carries the
    # lengths on the host (`seq_lens_cpu`) gives the planner the whole batch,
    # the same input `paged_decode_hip(num_splits=None)` plans from;
    # otherwise it plans for a ragged batch of up to max_seq_len tokens.
    # A flat launch planned on host lengths also takes them (its ranges and
    # merge list are then built on the host).
    plan, host = _step_plan(attn_metadata, n, impl, cache.kv_dtype, query.device)
    kw = plan.launch_kwargs()
    if plan.flat_splits and host is not None:
        kw["seq_lens_host"] = host
    decode(query[:n], cache, out=output[:n], sm_scale=impl.scale, **kw)
    STATS["decode_calls"] += 1
    STATS["decode_tokens"] += n
    return output


def build_backend_classes(base_backend: type, base_impl: type) -> tuple[type, type]:
    """The (backend, impl) pair on top of a vLLM backend's classes (its
    metadata builder and cache layout, and its forward for everything this
    kernel does not serve)."""

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
        """The base backend (metadata, cache layout) with our impl."""

        @staticmethod
        def get_name() -> str:
            return BACKEND_NAME

        @staticmethod
        def get_impl_cls():
            return PagedAttnTritonImpl

    return PagedAttnTritonBackend, PagedAttnTritonImpl


# Base classes the backend can be built on. Prefill, mixed batches and every
# delegated case run the base class's `forward`, so the base decides their
# speed: the reference inherits vLLM's Triton backend and lost 1.9x on
# prefill that way (README.md:186; integration/vllm_backend.py:93-111).
# Each base must keep the NHD cache the decode reads in place,
# [2, num_blocks, block_size, num_kv_heads, head_size] (checked through its
# get_kv_cache_shape when the classes are built).
#   triton         vLLM's Triton backend: the reference's base, the default
#   rocm_aiter_fa  vLLM-ROCm's AITER flash-attention backend (CK kernels for
#                  prefill on MI300/MI355); needs the `aiter` package
#   flash_attn     vLLM's FlashAttention backend
#   auto           rocm_aiter_fa where it and `aiter` import, else triton
# A "module:BackendClass:ImplClass" string names any other base.
BASE_BACKENDS: dict[str, tuple[str, str, str]] = {
    "triton": ("vllm.v1.attention.backends.triton_attn", "TritonAttentionBackend",
               "TritonAttentionImpl"),
    "rocm_aiter_fa": ("vllm.v1.attention.backends.rocm_aiter_fa", "AiterFlashAttentionBackend",
                      "AiterFlashAttentionImpl"),
    "flash_attn": ("vllm.v1.attention.backends.flash_attn", "FlashAttentionBackend",
                   "FlashAttentionImpl"),
}
DEFAULT_BASE = "triton"
# The base the module-level classes are built on (None without vLLM).
BASE_NAME: str | None = None


def _import_base(spec: str) -> tuple[type, type]:
    """(backend class, impl class) of a BASE_BACKENDS key or a
    "module:BackendClass:ImplClass" string."""
    import importlib

    if spec in BASE_BACKENDS:
        mod_name, backend_name, impl_name = BASE_BACKENDS[spec]
    else:
        parts = spec.split(":")
        if len(parts) != 3:
            raise ValueError(f"unknown base backend {spec!r}: one of {sorted(BASE_BACKENDS)}, "
                             "'auto', or 'module:BackendClass:ImplClass'")
        mod_name, backend_name, impl_name = parts
    mod = importlib.import_module(mod_name)
    return getattr(mod, backend_name), getattr(mod, impl_name)


def resolve_base(spec: str | None = None) -> tuple[str, type, type]:
    """(name, backend class, impl class) of the base to build on. `auto`
    prefers rocm_aiter_fa when its module and the `aiter` package import."""
    spec = spec or DEFAULT_BASE
    if spec == "auto":
        import importlib

        try:
            importlib.import_module("aiter")
            backend, impl = _import_base("rocm_aiter_fa")
            return "rocm_aiter_fa", backend, impl
        except Exception:
            spec = "triton"
    backend, impl = _import_base(spec)
    return spec, backend, impl


def check_nhd_layout(base_backend: type) -> None:
    """Raise unless the base lays its cache out as [2, NB, P, H_kv, D]: the
    decode views `kv_cache.unbind(0)` as the NHD pages it reads."""
    get_shape = getattr(base_backend, "get_kv_cache_shape", None)
    if get_shape is None:
        raise ValueError(f"{base_backend.__name__} has no get_kv_cache_shape")
    got = tuple(get_shape(3, 16, 2, 64))
    if got != (2, 3, 16, 2, 64):
        raise ValueError(f"{base_backend.__name__} lays its KV cache out as {got} for "
                         "(num_blocks=3, block_size=16, num_kv_heads=2, head_size=64); the "
                         "decode kernel reads [2, num_blocks, block_size, num_kv_heads, head_size]")


def use_base(spec: str | None = None) -> str:
    """Rebuild the module's PagedAttnTritonBackend / PagedAttnTritonImpl on
    another base (`BASE_BACKENDS` key, `auto`, or a qualified pair), so that
    QUALNAME resolves to them. Returns the base's name."""
    global PagedAttnTritonBackend, PagedAttnTritonImpl, BASE_NAME
    name, backend, impl = resolve_base(spec)
    check_nhd_layout(backend)
    PagedAttnTritonBackend, PagedAttnTritonImpl = build_backend_classes(backend, impl)
    BASE_NAME = name
    return name


try:  # vLLM is optional: the module imports (and is testable) without it
    _import_base(DEFAULT_BASE)
    HAVE_VLLM = True
except Exception:  # pragma: no cover - depends on the environment
    HAVE_VLLM = False

PagedAttnTritonBackend = None  # type: ignore[assignment]
PagedAttnTritonImpl = None  # type: ignore[assignment]
if HAVE_VLLM:  # pragma: no cover - needs vLLM
    use_base(DEFAULT_BASE)


def install(platform_cls: type | None = None, prefill_backend: str | None = None) -> str:
    """Make vLLM pick this backend for plain (non-MLA) V1 attention.

    vLLM resolves the attention backend through the platform's
    `get_attn_backend_cls(...)`, which returns a qualname string; this wraps
    that classmethod once (idempotent) so the V1 non-MLA case returns
    QUALNAME (vllm_backend.py:180-205). Returns QUALNAME.

    `prefill_backend` (an addition) rebuilds the classes on another vLLM
    backend first (`use_base`): pure decode steps still run the HIP kernel,
    prefill and mixed batches run that backend's attention. None keeps the
    current base (vLLM's Triton backend unless changed).
    """
    if prefill_backend is not None:
        use_base(prefill_backend)
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
    `vllm.general_plugins` entry point in the worker (vllm_backend.py:208-214).
    PAGEDATTN_PREFILL_BACKEND, when set, is passed as `prefill_backend`."""
    if os.environ.get("PAGEDATTN_VLLM_BACKEND", "") not in ("1", "true", "True"):
        return False
    install(platform_cls, os.environ.get("PAGEDATTN_PREFILL_BACKEND") or None)
    return True
