"""Import-path compatibility with the reference's `pagedattn.triton_decode`.

Callers written against the reference (for example its vLLM backend,
integration/vllm_backend.py:40) import `paged_decode_triton` and
`pick_num_splits` from this module path. Both names resolve to the HIP
implementation in `hip_decode`; no Triton is involved.
"""

from .hip_decode import paged_decode_hip, paged_decode_triton, pick_num_splits

__all__ = ["paged_decode_hip", "paged_decode_triton", "pick_num_splits"]
