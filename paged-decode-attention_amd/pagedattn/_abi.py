"""ctypes binding of `libpagedattn_hip.so` (declared in include/pagedattn.h).

The structures below mirror `pa_decode_args` / `pa_reduce_args` field for
field. The library is looked up next to this file (where `build.py` writes
it) or at $PAGEDATTN_HIP_LIB. There is no fallback: a missing library raises.
"""

from __future__ import annotations

import ctypes
import os
import pathlib
import threading

PA_ABI_VERSION = 8

PA_OK = 0
PA_ERR_INVALID = -1
PA_ERR_UNSUPPORTED = -2
PA_ERR_HIP = -3

PA_KV_FP16 = 0
PA_KV_FP8_E5M2 = 1
PA_KV_INT8 = 2
PA_KV_BF16 = 3

PA_SCALE_NONE = 0
PA_SCALE_FP16 = 1
PA_SCALE_FP32 = 2

PA_IO_FP16 = 0
PA_IO_BF16 = 1

PA_MAX_SPLITS = 4096
PA_MAX_FLAT_SPLITS = 65536
PA_MAX_FLAT_SEQ_COST = 64
PA_NOALLOC_SCRATCH_BYTES = 32 << 20
PA_MAX_GROUP = 16
PA_HOST_TABLE_MAX = 256
PA_HOST_PLAN_RANGES = 1
PA_HOST_PLAN_MERGE = 2

LIB_NAME = "libpagedattn_hip.so"

# Every symbol include/pagedattn.h declares.
EXPORTED_SYMBOLS = (
    "pa_decode",
    "pa_decode_noalloc",
    "pa_decode_partials",
    "pa_split_reduce",
    "pa_cache_write",
    "pa_flat_merge",
    "pa_flat_waves_per_simd",
    "pa_flat_host_plan",
    "pa_last_error",
    "pa_abi_version",
)

_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


class PaDecodeArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp),
        ("k_cache", _vp),
        ("v_cache", _vp),
        ("k_scale", _vp),
        ("v_scale", _vp),
        ("out", _vp),
        ("part_out", _vp),
        ("part_lse", _vp),
        ("block_table", _vp),
        ("seq_lens", _vp),
        ("batch", _i32),
        ("num_q_heads", _i32),
        ("num_kv_heads", _i32),
        ("head_dim", _i32),
        ("block_size", _i32),
        ("num_blocks", _i32),
        ("max_blocks", _i32),
        ("num_splits", _i32),
        ("max_seq_len", _i32),
        ("stride_qb", _i64),
        ("stride_qh", _i64),
        ("stride_kn", _i64),
        ("stride_kt", _i64),
        ("stride_kh", _i64),
        ("stride_sn", _i64),
        ("stride_st", _i64),
        ("stride_ob", _i64),
        ("stride_oh", _i64),
        ("stride_pb", _i64),
        ("stride_ph", _i64),
        ("stride_ps", _i64),
        ("stride_lb", _i64),
        ("stride_lh", _i64),
        ("stride_btb", _i64),
        ("kv_dtype", _i32),
        ("scale_dtype", _i32),
        ("io_dtype", _i32),
        ("sm_scale", ctypes.c_float),
        ("flat_splits", _i32),
        ("flat_seq_cost", _i32),
        ("seq_lens_host", _vp),
    ]


class PaReduceArgs(ctypes.Structure):
    _fields_ = [
        ("part_out", _vp),
        ("part_lse", _vp),
        ("out", _vp),
        ("batch", _i32),
        ("num_heads", _i32),
        ("head_dim", _i32),
        ("num_splits", _i32),
        ("stride_pb", _i64),
        ("stride_ph", _i64),
        ("stride_ps", _i64),
        ("stride_lb", _i64),
        ("stride_lh", _i64),
        ("stride_ob", _i64),
        ("stride_oh", _i64),
        ("io_dtype", _i32),
    ]


class PaCacheWriteArgs(ctypes.Structure):
    _fields_ = [
        ("key", _vp),
        ("value", _vp),
        ("k_cache", _vp),
        ("v_cache", _vp),
        ("k_scale", _vp),
        ("v_scale", _vp),
        ("slot_mapping", _vp),
        ("num_tokens", _i32),
        ("num_kv_heads", _i32),
        ("head_dim", _i32),
        ("block_size", _i32),
        ("num_blocks", _i32),
        ("stride_kt", _i64),
        ("stride_kh", _i64),
        ("stride_vt", _i64),
        ("stride_vh", _i64),
        ("stride_cn", _i64),
        ("stride_ct", _i64),
        ("stride_ch", _i64),
        ("stride_sn", _i64),
        ("stride_st", _i64),
        ("kv_dtype", _i32),
        ("scale_dtype", _i32),
    ]


class HipLibraryMissing(ImportError):
    """The HIP library has not been built (run __graft_entry__.build())."""


def lib_path() -> pathlib.Path:
    env = os.environ.get("PAGEDATTN_HIP_LIB")
    if env:
        return pathlib.Path(env)
    return pathlib.Path(__file__).resolve().parent / LIB_NAME


_LIB: ctypes.CDLL | None = None
_LOCK = threading.Lock()


def load() -> ctypes.CDLL:
    """Load and type the library once; raises HipLibraryMissing if absent."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        path = lib_path()
        if not path.exists():
            raise HipLibraryMissing(
                f"{path} not found: the HIP decode library is not built "
                "(python -c 'import __graft_entry__ as g; g.build()')"
            )
        lib = ctypes.CDLL(str(path))
        lib.pa_decode.argtypes = [ctypes.POINTER(PaDecodeArgs), _vp]
        lib.pa_decode.restype = ctypes.c_int
        lib.pa_decode_noalloc.argtypes = [ctypes.POINTER(PaDecodeArgs), _vp]
        lib.pa_decode_noalloc.restype = ctypes.c_int
        lib.pa_decode_partials.argtypes = [ctypes.POINTER(PaDecodeArgs), _vp]
        lib.pa_decode_partials.restype = ctypes.c_int
        lib.pa_split_reduce.argtypes = [ctypes.POINTER(PaReduceArgs), _vp]
        lib.pa_split_reduce.restype = ctypes.c_int
        lib.pa_cache_write.argtypes = [ctypes.POINTER(PaCacheWriteArgs), _vp]
        lib.pa_cache_write.restype = ctypes.c_int
        lib.pa_flat_merge.argtypes = [ctypes.POINTER(PaDecodeArgs), _vp]
        lib.pa_flat_merge.restype = ctypes.c_int
        lib.pa_flat_waves_per_simd.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                  ctypes.POINTER(ctypes.c_int)]
        lib.pa_flat_waves_per_simd.restype = ctypes.c_int
        lib.pa_flat_host_plan.argtypes = [ctypes.POINTER(PaDecodeArgs), _vp, _vp, _vp, _vp]
        lib.pa_flat_host_plan.restype = ctypes.c_int
        lib.pa_last_error.argtypes = []
        lib.pa_last_error.restype = ctypes.c_char_p
        lib.pa_abi_version.argtypes = []
        lib.pa_abi_version.restype = ctypes.c_int
        ver = lib.pa_abi_version()
        if ver != PA_ABI_VERSION:
            raise HipLibraryMissing(f"{path} has ABI version {ver}, expected {PA_ABI_VERSION}")
        _LIB = lib
        return lib


def check(rc: int, what: str) -> None:
    """Raise the Python error matching a PA_ERR_* code."""
    if rc == PA_OK:
        return
    msg = load().pa_last_error().decode(errors="replace")
    if rc == PA_ERR_INVALID:
        raise ValueError(f"{what}: {msg}")
    if rc == PA_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (code {rc})")
