"""Attention shapes and KV-cache dtype tables.

Mirrors the parts of the reference's `pagedattn/config.py` that the decode path
uses (ParamThakkar123/paged-decode-attention, pagedattn/config.py:16-71):
`KVDType`, per-element byte sizes, torch dtypes, `ModelShape` with its
`gqa_group` / `softmax_scale` properties, the Llama-3 presets and
`kv_bytes_per_token`. The reference's 4 GB VRAM planner and nvidia-smi probe
(config.py:74-133) are not part of the decode path and are not provided.
"""

from __future__ import annotations

import dataclasses
from typing import Literal

import torch

KVDType = Literal["fp16", "bf16", "fp8_e5m2", "int8"]

# Bytes per stored KV element (config.py:19-24).
_ELEM_BYTES: dict[str, float] = {
    "fp16": 2.0,
    "bf16": 2.0,
    "fp8_e5m2": 1.0,
    "int8": 1.0,
}

# Storage dtype per cache dtype (config.py:26-31). fp8 is the OCP e5m2 format.
_TORCH_DTYPE: dict[str, torch.dtype] = {
    "fp16": torch.float16,
    "bf16": torch.bfloat16,
    "fp8_e5m2": torch.float8_e5m2,
    "int8": torch.int8,
}


@dataclasses.dataclass(frozen=True)
class ModelShape:
    """Attention head geometry of one layer (config.py:34-53)."""

    num_q_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    name: str = "llama3-8b"

    @property
    def gqa_group(self) -> int:
        assert self.num_q_heads % self.num_kv_heads == 0, (
            f"num_q_heads={self.num_q_heads} not divisible by "
            f"num_kv_heads={self.num_kv_heads}"
        )
        return self.num_q_heads // self.num_kv_heads

    @property
    def softmax_scale(self) -> float:
        return self.head_dim**-0.5


# Presets (config.py:56-58) plus the Qwen2.5-0.5B shape the reference's vLLM
# run serves (README.md:36; 14 q heads / 2 kv heads / head_dim 64).
LLAMA3_8B = ModelShape(32, 8, 128, "llama3-8b")
LLAMA3_70B = ModelShape(64, 8, 128, "llama3-70b")
MHA_DEBUG = ModelShape(8, 8, 128, "mha-debug")
QWEN25_05B = ModelShape(14, 2, 64, "qwen2.5-0.5b")


def scale_bytes(scale_dtype: torch.dtype | None) -> int:
    """Bytes per int8 dequantisation scale (0 when the cache has none)."""
    if scale_dtype is None:
        return 0
    return torch.empty((), dtype=scale_dtype).element_size()


def kv_bytes_per_token(
    shape: ModelShape, kv_dtype: KVDType, scale_dtype: torch.dtype = torch.float16
) -> float:
    """Bytes of K+V cache for one token of one layer (config.py:61-67).

    The reference hard-codes 2-byte int8 scales; here the scale size follows
    `scale_dtype`, so fp32 scales are counted as 4 bytes.
    """
    per = 2 * shape.num_kv_heads * shape.head_dim * _ELEM_BYTES[kv_dtype]
    if kv_dtype == "int8":
        per += 2 * shape.num_kv_heads * scale_bytes(scale_dtype)
    return per


def torch_dtype(kv_dtype: KVDType) -> torch.dtype:
    return _TORCH_DTYPE[kv_dtype]
