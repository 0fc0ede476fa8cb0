"""CPU tests of the host side: the C ABI surface, argument validation, the
Python mirror of the reference interface, split policy, cache generation and
byte accounting. Nothing here launches a kernel."""

from __future__ import annotations

import ctypes
import pathlib
import re
import subprocess
import types

import pytest
import torch

from pagedattn import (LLAMA3_8B, LLAMA3_70B, MHA_DEBUG, QWEN25_05B, ModelShape, allocate,
                       kv_bytes_per_token, pick_num_splits)
from pagedattn import _abi
from pagedattn.hip_decode import paged_decode_hip

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "pagedattn.h"


def _lib():
    if not _abi.lib_path().exists():
        import __graft_entry__

        __graft_entry__.build()
    return _abi.load()


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pa_\w+)\s*\(", text)))


def test_header_declares_the_bound_symbols():
    assert _declared_functions() == sorted(_abi.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = _lib()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_abi.lib_path())],
                        capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (pa_\w+)", nm))
    assert exported == set(_declared_functions())
    assert lib.pa_abi_version() == _abi.PA_ABI_VERSION


STRUCTS = (("pa_decode_args", _abi.PaDecodeArgs), ("pa_reduce_args", _abi.PaReduceArgs),
           ("pa_cache_write_args", _abi.PaCacheWriteArgs))


def test_struct_layout_matches_header(tmp_path):
    """ctypes mirrors of pa_decode_args / pa_reduce_args against gcc's layout."""
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "pagedattn.h"', 'int main(void){']
    for cname, cls in STRUCTS:
        lines.append(f'printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for f, _ in cls._fields_:
            lines.append(f'printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    got = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    table = {}
    for line in filter(None, got):
        s, f, v = line.split()
        table[(s, f)] = int(v)
    for cname, cls in STRUCTS:
        assert table[(cname, "sizeof")] == ctypes.sizeof(cls)
        for f, _ in cls._fields_:
            assert table[(cname, f)] == getattr(cls, f).offset, (cname, f)


def test_constants_match_header():
    text = HEADER.read_text()
    for name in ("PA_ABI_VERSION", "PA_OK", "PA_ERR_INVALID", "PA_ERR_UNSUPPORTED", "PA_ERR_HIP",
                 "PA_KV_FP16", "PA_KV_FP8_E5M2", "PA_KV_INT8", "PA_SCALE_NONE", "PA_SCALE_FP16",
                 "PA_SCALE_FP32", "PA_IO_FP16", "PA_MAX_SPLITS", "PA_MAX_GROUP", "PA_KV_BF16",
                 "PA_IO_BF16", "PA_MAX_FLAT_SPLITS", "PA_MAX_FLAT_SEQ_COST", "PA_HOST_TABLE_MAX",
                 "PA_HOST_PLAN_RANGES", "PA_HOST_PLAN_MERGE"):
        m = re.search(rf"#define {name} \(?(-?\d+)\)?", text)
        assert m, name
        assert int(m.group(1)) == getattr(_abi, name), name


# --------------------------------------------------------------------------
# argument validation through the C ABI: every case is rejected before any
# HIP call, so fake device addresses are never dereferenced. Skipped where a
# GPU is visible, so no such call can ever reach a device.
# --------------------------------------------------------------------------

cpu_only = pytest.mark.skipif(torch.cuda.is_available(), reason="fake-pointer validation runs on CPU hosts only")

FAKE = 0x10000  # 16-byte aligned, never dereferenced


def _valid_args(**over):
    a = _abi.PaDecodeArgs()
    a.q = a.k_cache = a.v_cache = a.out = a.block_table = a.seq_lens = FAKE
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim = 2, 32, 8, 128
    a.block_size, a.num_blocks, a.max_blocks, a.num_splits = 16, 64, 8, 1
    a.stride_qb, a.stride_qh = 32 * 128, 128
    a.stride_kn, a.stride_kt, a.stride_kh = 16 * 8 * 128, 8 * 128, 128
    a.stride_ob, a.stride_oh = 32 * 128, 128
    a.stride_btb = 8
    a.kv_dtype, a.scale_dtype, a.io_dtype = _abi.PA_KV_FP16, _abi.PA_SCALE_NONE, _abi.PA_IO_FP16
    a.sm_scale = 128 ** -0.5
    for k, v in over.items():
        setattr(a, k, v)
    return a


INVALID = [
    ("q", dict(q=None), _abi.PA_ERR_INVALID),
    ("batch", dict(batch=-1), _abi.PA_ERR_INVALID),
    ("heads", dict(num_q_heads=30), _abi.PA_ERR_INVALID),
    ("kv_heads", dict(num_kv_heads=0), _abi.PA_ERR_INVALID),
    ("head_dim", dict(head_dim=96), _abi.PA_ERR_UNSUPPORTED),
    ("page", dict(block_size=24), _abi.PA_ERR_UNSUPPORTED),
    ("page8", dict(block_size=8), _abi.PA_ERR_UNSUPPORTED),
    ("splits0", dict(num_splits=0), _abi.PA_ERR_INVALID),
    ("splits_big", dict(num_splits=_abi.PA_MAX_SPLITS + 1), _abi.PA_ERR_INVALID),
    ("seq_cost_neg", dict(flat_seq_cost=-1), _abi.PA_ERR_INVALID),
    ("seq_cost_big", dict(flat_seq_cost=_abi.PA_MAX_FLAT_SEQ_COST + 1), _abi.PA_ERR_INVALID),
    ("no_workspace", dict(num_splits=4), _abi.PA_ERR_INVALID),
    ("kv_dtype", dict(kv_dtype=7), _abi.PA_ERR_INVALID),
    ("io_dtype", dict(io_dtype=3), _abi.PA_ERR_UNSUPPORTED),
    ("bf16_scale", dict(kv_dtype=_abi.PA_KV_BF16, scale_dtype=_abi.PA_SCALE_FP16), _abi.PA_ERR_INVALID),
    ("int8_no_scale", dict(kv_dtype=_abi.PA_KV_INT8, scale_dtype=_abi.PA_SCALE_FP16), _abi.PA_ERR_INVALID),
    ("int8_scale_type", dict(kv_dtype=_abi.PA_KV_INT8, k_scale=FAKE, v_scale=FAKE), _abi.PA_ERR_INVALID),
    ("scale_on_fp16", dict(scale_dtype=_abi.PA_SCALE_FP32), _abi.PA_ERR_INVALID),
    ("misaligned_q", dict(q=FAKE + 2), _abi.PA_ERR_INVALID),
    ("misaligned_head_stride", dict(stride_kh=100), _abi.PA_ERR_INVALID),
    ("negative_stride", dict(stride_kt=-1024), _abi.PA_ERR_INVALID),
    ("no_blocks", dict(num_blocks=0), _abi.PA_ERR_INVALID),
    ("misaligned_workspace", dict(num_splits=2, part_out=FAKE + 4, part_lse=FAKE,
                                  stride_pb=1, stride_ph=1, stride_ps=128), _abi.PA_ERR_INVALID),
    ("flat_negative", dict(flat_splits=-1), _abi.PA_ERR_INVALID),
    ("flat_big", dict(flat_splits=_abi.PA_MAX_FLAT_SPLITS + 1), _abi.PA_ERR_INVALID),
    ("flat_no_workspace", dict(flat_splits=4), _abi.PA_ERR_INVALID),
    ("flat_misaligned_workspace", dict(flat_splits=4, part_out=FAKE + 4, part_lse=FAKE,
                                       stride_pb=32 * 128, stride_ph=128), _abi.PA_ERR_INVALID),
    # page offsets inside a page and page strides are 32-bit in the kernels
    ("page_2gib", dict(stride_kt=2**27, stride_kn=16 * 2**27), _abi.PA_ERR_UNSUPPORTED),
    ("page_stride_4gib", dict(stride_kn=2**31), _abi.PA_ERR_UNSUPPORTED),
    ("block_table_2pow31", dict(stride_btb=2**30), _abi.PA_ERR_UNSUPPORTED),
    ("scale_page_stride_4gib", dict(kv_dtype=_abi.PA_KV_INT8, scale_dtype=_abi.PA_SCALE_FP32, k_scale=FAKE,
                                    v_scale=FAKE, stride_sn=2**30, stride_st=8), _abi.PA_ERR_UNSUPPORTED),
    # the other strides are held in 32 bits by the kernels
    ("q_stride_2pow31", dict(stride_qb=2**31), _abi.PA_ERR_UNSUPPORTED),
    ("out_stride_2pow31", dict(stride_oh=2**31), _abi.PA_ERR_UNSUPPORTED),
    ("kv_head_stride_2gib", dict(stride_kh=2**30), _abi.PA_ERR_UNSUPPORTED),
    ("workspace_stride_2pow31", dict(num_splits=2, part_out=FAKE, part_lse=FAKE, stride_pb=2**31,
                                     stride_ph=256, stride_ps=128, stride_lb=64, stride_lh=2),
     _abi.PA_ERR_UNSUPPORTED),
]


@cpu_only
@pytest.mark.parametrize("name,over,code", INVALID, ids=[c[0] for c in INVALID])
def test_pa_decode_rejects(name, over, code):
    lib = _lib()
    a = _valid_args(**over)
    assert lib.pa_decode(ctypes.byref(a), None) == code
    msg = lib.pa_last_error().decode()
    assert msg, "no error message recorded"
    assert lib.pa_decode_partials(ctypes.byref(a), None) < 0


@cpu_only
def test_null_args_and_reduce_validation():
    lib = _lib()
    assert lib.pa_decode(None, None) == _abi.PA_ERR_INVALID
    assert lib.pa_split_reduce(None, None) == _abi.PA_ERR_INVALID
    r = _abi.PaReduceArgs()
    r.part_out = r.part_lse = r.out = FAKE
    r.batch, r.num_heads, r.head_dim, r.num_splits = 1, 4, 100, 2
    assert lib.pa_split_reduce(ctypes.byref(r), None) == _abi.PA_ERR_UNSUPPORTED
    r.head_dim, r.num_splits = 128, 0
    assert lib.pa_split_reduce(ctypes.byref(r), None) == _abi.PA_ERR_INVALID
    r.num_splits, r.stride_ob = 2, -1
    assert lib.pa_split_reduce(ctypes.byref(r), None) == _abi.PA_ERR_INVALID


def _write_args(**over):
    a = _abi.PaCacheWriteArgs()
    a.key = a.value = a.k_cache = a.v_cache = a.slot_mapping = FAKE
    a.num_tokens, a.num_kv_heads, a.head_dim, a.block_size, a.num_blocks = 4, 8, 128, 16, 32
    a.stride_kt, a.stride_kh, a.stride_vt, a.stride_vh = 1024, 128, 1024, 128
    a.stride_cn, a.stride_ct, a.stride_ch = 16 * 1024, 1024, 128
    a.kv_dtype, a.scale_dtype = _abi.PA_KV_FP16, _abi.PA_SCALE_NONE
    for k, v in over.items():
        setattr(a, k, v)
    return a


WRITE_INVALID = [
    ("key", dict(key=None), _abi.PA_ERR_INVALID),
    ("tokens", dict(num_tokens=-1), _abi.PA_ERR_INVALID),
    ("heads", dict(num_kv_heads=0), _abi.PA_ERR_INVALID),
    ("head_dim", dict(head_dim=80), _abi.PA_ERR_UNSUPPORTED),
    ("kv_dtype", dict(kv_dtype=5), _abi.PA_ERR_INVALID),
    ("int8_scales", dict(kv_dtype=_abi.PA_KV_INT8, scale_dtype=_abi.PA_SCALE_FP32), _abi.PA_ERR_INVALID),
    ("scale_on_fp16", dict(scale_dtype=_abi.PA_SCALE_FP16), _abi.PA_ERR_INVALID),
    ("misaligned_key", dict(key=FAKE + 8), _abi.PA_ERR_INVALID),
    ("misaligned_cache", dict(stride_ch=100), _abi.PA_ERR_INVALID),
    ("negative_stride", dict(stride_vt=-1), _abi.PA_ERR_INVALID),
]


@cpu_only
@pytest.mark.parametrize("name,over,code", WRITE_INVALID, ids=[c[0] for c in WRITE_INVALID])
def test_pa_cache_write_rejects(name, over, code):
    lib = _lib()
    a = _write_args(**over)
    assert lib.pa_cache_write(ctypes.byref(a), None) == code
    assert lib.pa_last_error().decode()


@cpu_only
def test_pa_cache_write_null_and_empty():
    lib = _lib()
    assert lib.pa_cache_write(None, None) == _abi.PA_ERR_INVALID
    # zero tokens is a no-op that returns before any HIP call
    assert lib.pa_cache_write(ctypes.byref(_write_args(num_tokens=0)), None) == _abi.PA_OK


def test_cache_writer_rejects_cpu_tensors():
    from pagedattn import reshape_and_cache

    c = allocate(LLAMA3_8B, 1, [16], device="cpu", seed=0)
    k = torch.zeros((2, 8, 128), dtype=torch.float16)
    with pytest.raises(ValueError, match="GPU"):
        reshape_and_cache(k, k, c, torch.zeros(2, dtype=torch.int64))


def test_python_errors_from_codes():
    with pytest.raises(ValueError):
        _abi.check(_abi.PA_ERR_INVALID, "x")
    with pytest.raises(NotImplementedError):
        _abi.check(_abi.PA_ERR_UNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _abi.check(_abi.PA_ERR_HIP, "x")
    _abi.check(_abi.PA_OK, "x")


# --------------------------------------------------------------------------
# the Python mirror of the reference interface
# --------------------------------------------------------------------------

def test_no_cpu_fallback():
    c = allocate(LLAMA3_8B, 2, [10, 20], device="cpu", seed=0)
    q = torch.randn((2, 32, 128), dtype=torch.float16)
    with pytest.raises(ValueError, match="GPU"):
        paged_decode_hip(q, c, num_splits=1)


def test_reference_names_resolve_to_hip():
    import pagedattn
    from pagedattn import triton_decode

    assert pagedattn.paged_decode_triton is paged_decode_hip
    assert triton_decode.paged_decode_triton is paged_decode_hip
    assert triton_decode.pick_num_splits is pick_num_splits


def test_model_shapes():
    assert LLAMA3_8B.gqa_group == 4 and LLAMA3_70B.gqa_group == 8
    assert MHA_DEBUG.gqa_group == 1 and QWEN25_05B.gqa_group == 7
    assert LLAMA3_8B.softmax_scale == 128 ** -0.5
    with pytest.raises(AssertionError):
        ModelShape(30, 8, 128).gqa_group


def test_kv_bytes_per_token():
    assert kv_bytes_per_token(LLAMA3_8B, "fp16") == 2 * 8 * 128 * 2
    assert kv_bytes_per_token(LLAMA3_8B, "fp8_e5m2") == 2 * 8 * 128
    assert kv_bytes_per_token(LLAMA3_8B, "int8") == 2 * 8 * 128 + 2 * 8 * 2
    assert kv_bytes_per_token(LLAMA3_8B, "int8", torch.float32) == 2 * 8 * 128 + 2 * 8 * 4


def test_pick_num_splits_policy():
    # enough work already: no split
    assert pick_num_splits(64, 8, 4096, 256) == 1
    assert pick_num_splits(24, 2, 192, 256) == 1  # C1: capped by the short context
    # long context, tiny batch: one workgroup per CU (B * Hkv * S >= CUs)
    assert pick_num_splits(4, 8, 131072, 256) == 8
    assert pick_num_splits(1, 8, 131072, 256) == 32
    assert pick_num_splits(1, 8, 512, 256) == 8      # chunks of at least 64 tokens
    assert pick_num_splits(32, 8, 4096, 256) == 1    # a workgroup per CU already
    for b, h, t in ((1, 1, 1), (1, 8, 5000), (32, 8, 16384), (4, 8, 131072), (3, 2, 0)):
        s = pick_num_splits(b, h, t, 256)
        assert 1 <= s <= _abi.PA_MAX_SPLITS


def test_allocate_is_deterministic_and_well_formed():
    a = allocate(LLAMA3_8B, 3, [5, 40, 17], device="cpu", seed=3, slack_blocks=4)
    b = allocate(LLAMA3_8B, 3, [5, 40, 17], device="cpu", seed=3, slack_blocks=4)
    assert torch.equal(a.k_cache, b.k_cache) and torch.equal(a.block_table, b.block_table)
    nb = [1, 3, 2]
    assert a.k_cache.shape == (sum(nb) + 4, 16, 8, 128)
    used = torch.cat([a.block_table[i, :n] for i, n in enumerate(nb)])
    assert used.unique().numel() == used.numel()  # each block used once
    assert a.block_table[0, 1:].eq(0).all() and a.block_table[2, 2:].eq(0).all()
    c = allocate(LLAMA3_8B, 1, [33], device="cpu", seed=4, shuffle=False)
    assert c.block_table[0].tolist() == [0, 1, 2]


def test_algorithmic_bytes_of_baseline_configs():
    """The published per-call byte counts of the benchmark configs, from the
    same formula bench.py uses."""
    import bench

    def fake(shape, lens, kv, scale_dt=None):
        meta = lambda dt: torch.empty(0, dtype=dt, device="meta")
        st = {"fp16": torch.float16, "fp8_e5m2": torch.float8_e5m2, "int8": torch.int8}[kv]
        return types.SimpleNamespace(shape=shape, block_size=16, kv_dtype=kv, k_cache=meta(st),
                                     k_scale=meta(scale_dt) if scale_dt else None,
                                     seq_lens=torch.tensor(lens))

    assert bench._algorithmic_bytes(fake(LLAMA3_8B, [4096] * 64, "fp16")) == 1_074_855_936
    assert bench._algorithmic_bytes(fake(LLAMA3_70B, [16384] * 32, "int8", torch.float32)) == 1_108_475_904
    assert bench._algorithmic_bytes(fake(LLAMA3_8B, [131072] * 4, "fp16")) == 2_147_680_256


def test_plan_num_splits():
    from pagedattn import plan_num_splits

    # uniform batches that fill the CUs stay unsplit (the headline shape)
    assert plan_num_splits([4096] * 64, 8, 4, 256) == (1, 4096)
    # a ragged batch of the same size splits its long sequences
    import math

    g = torch.Generator().manual_seed(2)
    u = torch.rand(64, generator=g, dtype=torch.float64)
    ragged = torch.exp(math.log(128) + u * (math.log(8192) - math.log(128))).round().long().tolist()
    s, m = plan_num_splits(ragged, 8, 4, 256)
    assert s >= 4 and m == max(ragged)
    # small batches of long sequences: one chunk of work per CU
    assert plan_num_splits([131072] * 4, 8, 4, 256) == (8, 131072)
    assert plan_num_splits([16384] * 32, 8, 8, 256) == (1, 16384)   # 256 units: one per CU
    assert plan_num_splits([2048], 8, 4, 256) == (32, 2048)           # 64-token chunks
    # a ragged batch takes chunks twice as long: 2 * 3584 * 8 / 256 = 224 tokens
    assert plan_num_splits([2048, 1024, 256, 256], 8, 4, 256) == (10, 2048)
    # a ragged batch with a workgroup per CU: unsplit while its sequences are
    # short, else about four rounds of workgroups (C3's lengths: 842-token chunks)
    assert plan_num_splits([500, 20] * 16, 8, 4, 256) == (1, 500)
    assert s == -(-max(ragged) // (sum(ragged) * 8 // 1024))
    # short sequences are never split (the merge would cost more)
    assert plan_num_splits([192, 40, 7], 2, 7, 256) == (1, 192)
    # edge cases
    assert plan_num_splits([], 8, 4, 256) == (1, 0)
    assert plan_num_splits([0, 0], 8, 4, 256) == (1, 0)
    assert plan_num_splits([1], 1, 1, 256)[0] == 1


def test_flat_splits_for_and_plan_decode():
    from pagedattn import flat_splits_for, plan_decode

    # one round of waves over the (kv head, head tile) units, one per SIMD
    # whatever the occupancy allows
    assert flat_splits_for(8, 4, 256, 2) == 128
    assert flat_splits_for(8, 4, 256, 3) == 128
    assert flat_splits_for(8, 4, 256, 1) == 128
    assert flat_splits_for(2, 20, 256, 2) == 256      # group 20: two head tiles
    assert flat_splits_for(64, 1, 4, 1) == 1
    # int8 caches take two waves per SIMD where the kernel's occupancy allows
    assert flat_splits_for(8, 8, 256, 2, "int8") == 256
    assert flat_splits_for(8, 8, 256, 1, "int8") == 128
    assert flat_splits_for(8, 8, 256, 4, "fp8_e5m2") == 128
    assert plan_decode([16384] * 32, 8, 8, 256, 2, kv_dtype="int8", head_dim=128) == (1, 16384, 256)
    # every benchmark config with a split (C2-C5) takes the flat split ...
    assert plan_decode([4096] * 64, 8, 4, 256, 2) == (1, 4096, 128)
    assert plan_decode([16384] * 32, 8, 8, 256, 3) == (1, 16384, 128)
    assert plan_decode([131072] * 4, 8, 4, 256, 2) == (1, 131072, 128)
    # ... and a latency-bound batch (too few tiles per wave) the classic path
    s, m, f = plan_decode([192] * 24, 2, 7, 256, 4)
    assert f == 0 and s >= 1 and m == 192
    assert plan_decode([], 8, 4, 256) == (1, 0, 0)
    # batches above FLAT_MAX_BATCH take the classic planner
    from pagedattn.hip_decode import FLAT_MAX_BATCH
    assert plan_decode([4096] * (FLAT_MAX_BATCH + 1), 8, 4, 256, 2)[2] == 0
    assert plan_decode([4096] * FLAT_MAX_BATCH, 8, 4, 256, 2)[2] == 128
    # ... even when the flat split would need no merge (whole sequences per
    # range): the unsplit kernel is faster there
    assert plan_decode([1024] * FLAT_MAX_BATCH, 8, 4, 256, 1)[2] == 128
    assert plan_decode([1024] * (FLAT_MAX_BATCH + 1), 8, 4, 256, 1) == (1, 1024, 0)
    assert plan_decode([128] * 4096, 8, 4, 256, 1) == (1, 128, 0)
    assert plan_decode([1024, 1056] * (FLAT_MAX_BATCH // 2 + 1), 8, 4, 256, 1)[2] == 0
    assert plan_decode([1024, 1056] * (FLAT_MAX_BATCH // 2), 8, 4, 256, 1)[2] == 128
    # with the KV type known, a nearly uniform batch that fills the CUs
    # unsplit stays unsplit while its K/V is small (no merge launch) ...
    assert plan_decode([1024] * 64, 8, 4, 256, 1, kv_dtype="fp16", head_dim=128) == (1, 1024, 0)
    assert plan_decode([1024] * 64, 8, 4, 256, 1, kv_dtype="bf16", head_dim=128) == (1, 1024, 0)
    assert plan_decode([1024] * 64, 8, 4, 256, 1, kv_dtype="fp8_e5m2", head_dim=128) == (1, 1024, 0)
    assert plan_decode([512] * 64, 8, 4, 256, 1, kv_dtype="int8", head_dim=128) == (1, 512, 0)
    # ... with a lower limit for short 1-byte rows (head_dim 64), which stream
    # faster flat (Qwen2.5-0.5B shape, 2 kv heads, group 7): 34 MB unsplit,
    # 67 MB flat
    assert plan_decode([1024] * 128, 2, 7, 256, 1, kv_dtype="fp8_e5m2", head_dim=64) == (1, 1024, 0)
    assert plan_decode([2048] * 128, 2, 7, 256, 1, kv_dtype="fp8_e5m2", head_dim=64)[2] == 512
    assert plan_decode([1024] * 128, 2, 7, 256, 2, kv_dtype="int8", head_dim=64) == (1, 1024, 0)
    assert plan_decode([1024] * 256, 2, 7, 256, 2, kv_dtype="int8", head_dim=64)[2] == 1024
    assert plan_decode([2048] * 128, 2, 7, 256, 1, kv_dtype="fp16", head_dim=64) == (1, 2048, 0)
    # ... and above the per-type byte limit takes the flat split
    assert plan_decode([4096] * 64, 8, 4, 256, 1, kv_dtype="fp16", head_dim=128)[2] == 128
    assert plan_decode([2048] * 64, 8, 4, 256, 1, kv_dtype="fp8_e5m2", head_dim=128)[2] == 128
    assert plan_decode([1024] * 64, 8, 4, 256, 1, kv_dtype="int8", head_dim=128)[2] == 128
    # ... and so does a batch the flat split covers with no merge (B = 128, F = 128:
    # one sequence per range) when its sequences are long or its KV 1-byte
    assert plan_decode([2048] * 128, 8, 4, 256, 1, kv_dtype="fp16", head_dim=128) == (1, 2048, 128)
    assert plan_decode([512] * 128, 8, 4, 256, 1, kv_dtype="int8", head_dim=128) == (1, 512, 128)
    # a batch of short sequences that fills the CUs runs unsplit at any size,
    # merge or not: nearly uniform up to UNSPLIT_SHORT_MAX_TOKENS ...
    from pagedattn.hip_decode import (RAGGED_UNSPLIT_MIN_WGS_PER_CU, TILE_TOKENS,
                                      UNSPLIT_RAGGED_MAX_TILES, UNSPLIT_SHORT_MAX_TILES)
    UNSPLIT_SHORT_MAX_TOKENS = {k: v * TILE_TOKENS for k, v in UNSPLIT_SHORT_MAX_TILES.items()}
    UNSPLIT_RAGGED_MAX_TOKENS = {k: v * TILE_TOKENS for k, v in UNSPLIT_RAGGED_MAX_TILES.items()}
    assert plan_decode([512] * 128, 8, 4, 256, 1, kv_dtype="fp16", head_dim=128) == (1, 512, 0)
    t16, t8 = UNSPLIT_SHORT_MAX_TOKENS["fp16"], UNSPLIT_SHORT_MAX_TOKENS["fp8_e5m2"]
    assert plan_decode([t16] * 1024, 8, 4, 256, 1, kv_dtype="bf16", head_dim=128) == (1, t16, 0)
    assert plan_decode([t16 + 32] * 1024, 8, 4, 256, 1, kv_dtype="fp16", head_dim=128)[2] == 128
    assert plan_decode([t8] * 512, 8, 4, 256, 1, kv_dtype="fp8_e5m2", head_dim=128) == (1, t8, 0)
    assert plan_decode([t8] * 128, 8, 4, 256, 1, kv_dtype="fp8_e5m2", head_dim=128) == (1, t8, 0)
    assert plan_decode([t8 + 256] * 128, 8, 4, 256, 1, kv_dtype="fp8_e5m2", head_dim=128)[2] == 128
    # ... int8 never ...
    assert plan_decode([256] * 512, 8, 4, 256, 1, kv_dtype="int8", head_dim=128)[2] == 128
    # ... and ragged, with RAGGED_UNSPLIT_MIN_WGS_PER_CU workgroups per CU, up to
    # UNSPLIT_RAGGED_MAX_TOKENS
    nb = RAGGED_UNSPLIT_MIN_WGS_PER_CU * 256 // 8
    r16, r8 = UNSPLIT_RAGGED_MAX_TOKENS["fp16"], UNSPLIT_RAGGED_MAX_TOKENS["fp8_e5m2"]
    ramp16 = [32 + (r16 - 32) * i // (nb - 1) for i in range(nb)]
    ramp8 = [32 + (r8 - 32) * i // (nb - 1) for i in range(nb)]
    assert max(ramp16) == r16 and max(ramp8) == r8
    assert plan_decode(ramp16, 8, 4, 256, 1, kv_dtype="fp16", head_dim=128) == (1, r16, 0)
    assert plan_decode(ramp8, 8, 4, 256, 1, kv_dtype="fp8_e5m2", head_dim=128) == (1, r8, 0)
    assert plan_decode(ramp16[:-1] + [r16 + 1], 8, 4, 256, 1, kv_dtype="fp16", head_dim=128)[2] == 128
    assert plan_decode(ramp16[: nb - 8], 8, 4, 256, 1, kv_dtype="fp16", head_dim=128)[2] == 128
    assert plan_decode(ramp8, 8, 4, 256, 1, kv_dtype="int8", head_dim=128)[2] == 128
    # a smaller ragged batch, or one that does not fill the CUs, keeps the flat split
    ragged = [256, 1792] * 32
    assert plan_decode(ragged, 8, 4, 256, 1, kv_dtype="fp16", head_dim=128)[2] == 128
    assert plan_decode([8192] * 8, 8, 4, 256, 1, kv_dtype="fp16", head_dim=128)[2] == 128
    # the threshold: MIN_FLAT_TILES_PER_WAVE tiles per wave
    from pagedattn.hip_decode import MIN_FLAT_TILES_PER_WAVE
    f = flat_splits_for(1, 1, 1, 1)
    assert f == 4
    half = 16 * MIN_FLAT_TILES_PER_WAVE * f
    assert plan_decode([half, half], 1, 1, 1, 1)[2] == f
    assert plan_decode([half, half - 32], 1, 1, 1, 1)[2] == 0
    # a single sequence takes the classic split up to SINGLE_SEQ_SPLIT_MAX_TILES
    from pagedattn.hip_decode import SINGLE_SEQ_SPLIT_MAX_TILES
    single = SINGLE_SEQ_SPLIT_MAX_TILES * TILE_TOKENS
    assert plan_decode([single], 8, 4, 256, 1)[2] == 0
    assert plan_decode([single + 32], 8, 4, 256, 1)[2] == 128


@cpu_only
def test_flat_occupancy_query_validates_before_hip():
    lib = _lib()
    out = ctypes.c_int(7)
    assert lib.pa_flat_waves_per_simd(_abi.PA_KV_FP16, _abi.PA_SCALE_NONE, 96, ctypes.byref(out)) \
        == _abi.PA_ERR_UNSUPPORTED
    assert out.value == 0
    assert lib.pa_flat_waves_per_simd(_abi.PA_KV_INT8, _abi.PA_SCALE_NONE, 128, ctypes.byref(out)) \
        == _abi.PA_ERR_INVALID
    assert lib.pa_flat_waves_per_simd(_abi.PA_KV_FP16, _abi.PA_SCALE_NONE, 128, None) \
        == _abi.PA_ERR_INVALID
    assert lib.pa_last_error().decode()


@cpu_only
def test_flat_merge_needs_flat_splits():
    lib = _lib()
    a = _valid_args(part_out=FAKE, part_lse=FAKE, stride_pb=32 * 128, stride_ph=128)
    assert lib.pa_flat_merge(ctypes.byref(a), None) == _abi.PA_ERR_INVALID
    assert "flat_splits" in lib.pa_last_error().decode()


def test_short_batch_runs_unsplit_thresholds():
    """The short-batch rule on its own: per-KV-type token limits, the
    workgroups-per-CU threshold scaling with the CU count, and head tiles
    (groups above PA_MAX_GROUP) counting as extra workgroups."""
    from pagedattn import short_batch_runs_unsplit as sbu
    from pagedattn.hip_decode import (RAGGED_UNSPLIT_MIN_WGS_PER_CU, TILE_TOKENS,
                                      UNSPLIT_RAGGED_MAX_TILES, UNSPLIT_SHORT_MAX_TILES, _abi)

    UNSPLIT_SHORT_MAX_TOKENS = {k: v * TILE_TOKENS for k, v in UNSPLIT_SHORT_MAX_TILES.items()}
    UNSPLIT_RAGGED_MAX_TOKENS = {k: v * TILE_TOKENS for k, v in UNSPLIT_RAGGED_MAX_TILES.items()}

    cus = 256
    nb = RAGGED_UNSPLIT_MIN_WGS_PER_CU * cus // 8  # 8 kv heads, group 4: one unit per kv head
    for kv, lim in UNSPLIT_RAGGED_MAX_TOKENS.items():
        assert sbu(nb, lim, 8, 4, cus, kv)
        assert not sbu(nb, lim + 1, 8, 4, cus, kv)
        assert not sbu(nb - 1, lim, 8, 4, cus, kv)
    for kv, lim in UNSPLIT_SHORT_MAX_TOKENS.items():
        # nearly uniform batches need only fill the CUs (the caller's check)
        assert sbu(1, lim, 8, 4, cus, kv, uniform=True)
        assert not sbu(1, lim + 1, 8, 4, cus, kv, uniform=True)  # a batch of 1 is not ragged-large
    # int8, unknown types and empty batches never
    assert not sbu(4 * nb, 64, 8, 4, cus, "int8")
    assert not sbu(4 * nb, 64, 8, 4, cus, "int8", uniform=True)
    assert not sbu(nb, 0, 8, 4, cus, "fp16")
    # twice the CUs need twice the batch
    assert not sbu(nb, 512, 8, 4, 2 * cus, "fp16")
    assert sbu(2 * nb, 512, 8, 4, 2 * cus, "fp16")
    # groups of WIDE_GROUP_MIN or more q heads per kv head double the limits
    from pagedattn.hip_decode import WIDE_GROUP_MIN as wg
    for kv, lim in UNSPLIT_RAGGED_MAX_TOKENS.items():
        assert sbu(nb, 2 * lim, 8, wg, cus, kv) and not sbu(nb, 2 * lim + 1, 8, wg, cus, kv)
        assert not sbu(nb, 2 * lim, 8, wg - 1, cus, kv)
    for kv, lim in UNSPLIT_SHORT_MAX_TOKENS.items():
        assert sbu(1, 2 * lim, 8, wg, cus, kv, uniform=True)
        assert not sbu(1, 2 * lim + 1, 8, wg, cus, kv, uniform=True)
    # a group above PA_MAX_GROUP takes two head tiles per kv head
    g2 = _abi.PA_MAX_GROUP + 1
    assert sbu(nb // 2, 512, 8, g2, cus, "fp16")
    assert not sbu(nb // 2, 512, 8, 4, cus, "fp16")


def test_public_partials_helpers_reject_bad_workspaces():
    """decode_partials / flat_merge / split_reduce check caller-supplied
    workspaces before any pointer reaches a kernel: dtype, device, exact
    classic shapes, enough flat slots, the split stride of part_lse, and the
    merge output's shape."""
    from pagedattn import LLAMA3_8B, allocate
    from pagedattn.hip_decode import decode_partials, flat_merge, split_reduce

    c = allocate(LLAMA3_8B, 2, [40, 70], device="cpu", seed=2)
    q = torch.zeros((2, 32, 128), dtype=torch.float16)
    f32 = dict(dtype=torch.float32)
    good_po, good_pl = torch.zeros((2, 32, 3, 128), **f32), torch.zeros((2, 32, 3), **f32)
    bad = [
        (torch.zeros((2, 32, 3, 128), dtype=torch.float16), good_pl, "float32"),
        (torch.zeros((2, 32, 2, 128), **f32), good_pl, "part_(out|lse)"),
        (good_po, torch.zeros((2, 32, 4), **f32), "part_lse"),
        (good_po, torch.zeros((2, 3, 32), **f32).transpose(1, 2), "contiguous split"),
    ]
    for po, pl, msg in bad:
        with pytest.raises(ValueError, match=msg):
            decode_partials(q, c, 3, part_out=po, part_lse=pl)
        with pytest.raises(ValueError, match=msg):
            split_reduce(po, pl)
    # the well-formed classic workspace passes the checks and stops at the
    # GPU-only launch
    with pytest.raises(ValueError, match="GPU"):
        decode_partials(q, c, 3, part_out=good_po, part_lse=good_pl)
    with pytest.raises(ValueError, match="GPU"):
        split_reduce(good_po, good_pl, torch.zeros((2, 32, 128), dtype=torch.float16))
    with pytest.raises(ValueError, match="out"):
        split_reduce(good_po, good_pl, torch.zeros((2, 32, 64), dtype=torch.float16))
    # flat slots: at least B + F of them
    F = 5
    few = (torch.zeros((2 + F - 1, 32, 128), **f32), torch.zeros((2 + F, 32), **f32))
    for po, pl in (few, (few[1].new_zeros((2 + F, 32, 128)), few[1][:-1])):
        with pytest.raises(ValueError, match="flat"):
            decode_partials(q, c, 1, part_out=po, part_lse=pl, flat_splits=F)
        with pytest.raises(ValueError, match="flat"):
            flat_merge(q, c, F, po, pl, torch.zeros_like(q))
    with pytest.raises(ValueError, match="float32"):
        flat_merge(q, c, F, torch.zeros((2 + F, 32, 128), dtype=torch.float16),
                   torch.zeros((2 + F, 32), **f32), torch.zeros_like(q))


def test_workspace_keeps_outgrown_buffers():
    """A grown workspace retires the old buffers instead of freeing them (a
    captured HIP graph may still launch into them), growing at least 2x."""
    from pagedattn.hip_decode import _Workspace

    ws = _Workspace()
    dev = torch.device("cpu")
    a, _ = ws.get(2, 4, 1, 8, dev)
    p0 = a.data_ptr()
    b, _ = ws.get(2, 4, 1, 8, dev)
    assert b.data_ptr() == p0                      # same size: no allocation
    c, _ = ws.get(3, 4, 1, 8, dev)                 # grows
    assert ws.current(dev)[0].numel() >= 2 * 64
    assert ws._retired[dev][0][0].data_ptr() == p0  # the old buffer is kept alive
    d, _ = ws.get(4, 4, 1, 8, dev)                 # within the 2x growth: no new buffer
    assert d.data_ptr() == c.data_ptr() and len(ws._retired[dev]) == 1


def test_plan_charges_ragged_sequences_by_kv_width():
    """A ragged batch with known lengths is charged RAGGED_FLAT_SEQ_COST tiles
    per sequence for 2-byte KV and RAGGED_FLAT_SEQ_COST_KV for 1-byte KV (a
    sequence start costs a fixed time, more tiles when tiles are half the
    bytes); nearly uniform batches and unknown lengths are charged nothing."""
    import math

    from pagedattn.hip_decode import (RAGGED_FLAT_SEQ_COST, RAGGED_FLAT_SEQ_COST_KV, plan_launch)

    g = torch.Generator().manual_seed(2)
    u = torch.rand(64, generator=g, dtype=torch.float64)
    ragged = torch.exp(math.log(128) + u * (math.log(8192) - math.log(128))).round().long().tolist()
    for kv, want in (("fp16", RAGGED_FLAT_SEQ_COST), ("bf16", RAGGED_FLAT_SEQ_COST),
                     ("fp8_e5m2", RAGGED_FLAT_SEQ_COST_KV["fp8_e5m2"]), ("int8", RAGGED_FLAT_SEQ_COST_KV["int8"])):
        p = plan_launch(64, 0, 8, 4, 256, 2, kv_dtype=kv, head_dim=128, seq_lens=ragged)
        assert p.flat_splits > 0 and p.flat_seq_cost == want, (kv, p)
    assert RAGGED_FLAT_SEQ_COST_KV["fp8_e5m2"] == 2 and RAGGED_FLAT_SEQ_COST == 1
    p = plan_launch(64, 0, 8, 4, 256, 1, kv_dtype="fp8_e5m2", head_dim=128, seq_lens=[4096] * 64)
    assert p.flat_seq_cost == 0
    p = plan_launch(64, 8192, 8, 4, 256, 1, kv_dtype="fp8_e5m2", head_dim=128)
    assert p.flat_seq_cost == 0
