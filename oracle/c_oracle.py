"""ctypes binding of the float64 C oracle (pa_oracle.c) -- TEST INFRASTRUCTURE ONLY.

`decode` and `split` take a PagedKVCache-like object (fields shape,
block_size, kv_dtype, k_cache, v_cache, k_scale, v_scale, block_table,
seq_lens), copy everything to dense CPU buffers and return float64 tensors.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import torch

from . import C_LIBRARY, build_c_oracle

_KV = {"fp16": 0, "fp8_e5m2": 1, "int8": 2, "bf16": 3}
_SC = {None: 0, torch.float16: 1, torch.float32: 2}
_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        if not C_LIBRARY.exists():
            build_c_oracle(verbose=False)
        lib = ctypes.CDLL(str(C_LIBRARY))
        vp, i32, f64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_double
        common = [vp] * 7 + [i32] * 8 + [f64]
        lib.pa_oracle_decode.argtypes = common + [vp]
        lib.pa_oracle_decode.restype = i32
        lib.pa_oracle_split.argtypes = common + [i32, i32, i32, vp, vp]
        lib.pa_oracle_split.restype = i32
        lib.pa_oracle_half_to_double.argtypes = [ctypes.c_uint16]
        lib.pa_oracle_half_to_double.restype = f64
        lib.pa_oracle_e5m2_to_double.argtypes = [ctypes.c_uint8]
        lib.pa_oracle_e5m2_to_double.restype = f64
        lib.pa_oracle_round_half.argtypes = [f64]
        lib.pa_oracle_round_half.restype = f64
        _LIB = lib
    return _LIB


def _bytes(t: torch.Tensor | None) -> np.ndarray | None:
    if t is None:
        return None
    t = t.detach().cpu().contiguous()
    return t.view(torch.uint8).numpy() if t.element_size() == 1 else t.view(-1).view(torch.uint8).numpy()


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _args(q, cache, sm_scale):
    shape = cache.shape
    keep = []

    def hold(a):
        keep.append(a)
        return _ptr(a)

    qb = hold(_bytes(q.to(torch.float16)))
    kb = hold(_bytes(cache.k_cache))
    vb = hold(_bytes(cache.v_cache))
    sc_dtype = cache.k_scale.dtype if cache.kv_dtype == "int8" else None
    ksb = hold(_bytes(cache.k_scale)) if sc_dtype is not None else None
    vsb = hold(_bytes(cache.v_scale)) if sc_dtype is not None else None
    bt = cache.block_table.detach().cpu().to(torch.int32).contiguous().numpy()
    sl = cache.seq_lens.detach().cpu().to(torch.int32).contiguous().numpy()
    keep += [bt, sl]
    b, hq, d = q.shape
    scale = shape.head_dim ** -0.5 if sm_scale is None else float(sm_scale)
    args = [qb, kb, vb, ksb, vsb, _ptr(bt), _ptr(sl), b, hq, shape.num_kv_heads, d,
            cache.block_size, bt.shape[1], _KV[cache.kv_dtype], _SC[sc_dtype], scale]
    return args, keep


def decode(q: torch.Tensor, cache, sm_scale: float | None = None) -> torch.Tensor:
    """float64 [B, Hq, D] decode output (pagedattn/reference.py:28-49)."""
    args, keep = _args(q, cache, sm_scale)
    out = np.zeros(tuple(q.shape), dtype=np.float64)
    rc = _lib().pa_oracle_decode(*args, _ptr(out))
    assert rc == 0, "pa_oracle_decode rejected its arguments"
    del keep
    return torch.from_numpy(out)


def split(q: torch.Tensor, cache, num_splits: int, align: int = 32, sm_scale: float | None = None,
          max_seq_len: int = 0):
    """float64 per-split (normalised output [B,Hq,S,D], log2-sum-exp [B,Hq,S])."""
    args, keep = _args(q, cache, sm_scale)
    b, hq, d = q.shape
    part = np.zeros((b, hq, num_splits, d), dtype=np.float64)
    lse = np.zeros((b, hq, num_splits), dtype=np.float64)
    rc = _lib().pa_oracle_split(*args, num_splits, align, max_seq_len, _ptr(part), _ptr(lse))
    assert rc == 0, "pa_oracle_split rejected its arguments"
    del keep
    return torch.from_numpy(part), torch.from_numpy(lse)


def half_to_double(bits: int) -> float:
    return _lib().pa_oracle_half_to_double(bits)


def e5m2_to_double(byte: int) -> float:
    return _lib().pa_oracle_e5m2_to_double(byte)


def round_half(x: float) -> float:
    return _lib().pa_oracle_round_half(x)


LOG2E = math.log2(math.e)
