"""pa_decode_noalloc: the decode that allocates nothing.

The entry point keeps the split partials in a static per-GPU device array
inside the library (PA_NOALLOC_SCRATCH_BYTES) instead of a caller workspace.
It has no counterpart in the reference; it serves callers that cannot
allocate. Its results must be pa_decode's, bit for bit (same kernels, same
launch), on consecutive calls that reuse the scratch, the second one
smaller, and under HIP graph capture; requests beyond the scratch are
refused before anything runs.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from helpers import max_abs, seeded_q
from oracle import reference as oracle
from pagedattn import LLAMA3_8B, LLAMA3_70B, QWEN25_05B, ModelShape, allocate
from pagedattn import _abi
from pagedattn.hip_decode import decode_noalloc, paged_decode_hip

ABS_TOL = 2e-3
LAUNCHES = {"flat": {"flat_splits": 23}, "split": {"num_splits": 5, "max_seq_len": 0},
            "unsplit": {"num_splits": 1}}


def _case(shape, lens, kv="fp16", seed=0, sdt=torch.float16):
    c = allocate(shape, len(lens), lens, kv_dtype=kv, seed=seed, scale_dtype=sdt, device="cuda")
    return seeded_q(len(lens), shape.num_q_heads, shape.head_dim, seed, device="cuda"), c


@pytest.mark.gpu
@pytest.mark.parametrize("launch", list(LAUNCHES))
@pytest.mark.parametrize("kv,sdt", [("fp16", torch.float16), ("int8", torch.float32),
                                    ("fp8_e5m2", torch.float16)], ids=["fp16", "int8", "fp8"])
def test_noalloc_equals_pa_decode_on_consecutive_calls(kv, sdt, launch):
    """Two calls in a row through pa_decode_noalloc, the second with a
    smaller batch and shorter sequences: each equals pa_decode's output bit
    for bit and the oracle within the decode's bar."""
    kw = LAUNCHES[launch]
    for shape, lens, seed in ((LLAMA3_70B, [700, 1, 2500, 0, 64, 1029, 333, 4096], 41),
                              (LLAMA3_8B, [90, 17, 400], 42)):
        print(f"{launch} {kv} {shape.name} lens={lens}", flush=True)
        q, c = _case(shape, lens, kv, seed, sdt)
        want = paged_decode_hip(q, c, **kw).clone()
        out = torch.full_like(q, 7.0)
        before = torch.cuda.memory_allocated()
        decode_noalloc(q, c, out, **kw)
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() == before
        assert torch.equal(out, want), "pa_decode_noalloc differs from pa_decode"
        ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
        assert max_abs(out[[i for i, t in enumerate(lens) if t > 0]],
                       ref[[i for i, t in enumerate(lens) if t > 0]]) < ABS_TOL


@pytest.mark.gpu
def test_noalloc_under_graph_capture():
    """Captured in a HIP graph (no allocation inside the capture at all),
    replayed with new q values between eager work: every replay equals
    pa_decode on the same inputs."""
    q, c = _case(QWEN25_05B, [300, 2000, 5, 1200], seed=43)
    out = torch.empty_like(q)
    decode_noalloc(q, c, out, flat_splits=40)  # the scratch address is looked up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        decode_noalloc(q, c, out, flat_splits=40)
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        decode_noalloc(q, c, out, flat_splits=40)
    for seed in (44, 45, 46):
        q.copy_(seeded_q(4, 14, 64, seed, device="cuda"))
        want = paged_decode_hip(q, c, flat_splits=40).clone()
        torch.cuda.synchronize()
        out.fill_(3.0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay with q seed {seed} differs"


@pytest.mark.gpu
def test_noalloc_refuses_partials_beyond_its_scratch():
    """A flat split whose slots exceed PA_NOALLOC_SCRATCH_BYTES is refused
    before anything is launched; `out` stays untouched."""
    shape = ModelShape(64, 1, 256, name="wide")
    q, c = _case(shape, [64] * 4, seed=47)
    out = torch.full_like(q, 5.0)
    rows_fit = _abi.PA_NOALLOC_SCRATCH_BYTES // (4 * 257 * 64)  # slots that fit
    with pytest.raises(NotImplementedError, match="scratch"):
        decode_noalloc(q, c, out, flat_splits=rows_fit)
    torch.cuda.synchronize()
    assert bool((out == 5.0).all())


# validation through the C ABI, before any HIP call (fake device addresses,
# never dereferenced): CPU hosts only
cpu_only = pytest.mark.skipif(torch.cuda.is_available(), reason="fake-pointer validation runs on CPU hosts only")
FAKE = 0x10000


def _args(**over):
    a = _abi.PaDecodeArgs()
    a.q = a.k_cache = a.v_cache = a.out = a.block_table = a.seq_lens = FAKE
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim = 4, 32, 8, 128
    a.block_size, a.num_blocks, a.max_blocks, a.num_splits = 16, 64, 16, 1
    a.stride_qb, a.stride_qh = 32 * 128, 128
    a.stride_kn, a.stride_kt, a.stride_kh = 16 * 8 * 128, 8 * 128, 128
    a.stride_ob, a.stride_oh = 32 * 128, 128
    a.stride_btb = 16
    a.kv_dtype, a.scale_dtype, a.io_dtype = _abi.PA_KV_FP16, _abi.PA_SCALE_NONE, _abi.PA_IO_FP16
    a.sm_scale = 0.088
    for k, v in over.items():
        setattr(a, k, v)
    return a


@cpu_only
def test_noalloc_validates_before_any_hip_call():
    lib = _abi.load()
    # caller workspace pointers and strides are ignored: no workspace needed
    assert lib.pa_decode_noalloc(None, None) == _abi.PA_ERR_INVALID
    assert lib.pa_decode_noalloc(ctypes.byref(_args(q=None, num_splits=4)), None) == _abi.PA_ERR_INVALID
    assert lib.pa_decode_noalloc(ctypes.byref(_args(head_dim=96, num_splits=4)), None) \
        == _abi.PA_ERR_UNSUPPORTED
    assert lib.pa_decode_noalloc(ctypes.byref(_args(num_splits=5000)), None) == _abi.PA_ERR_INVALID
    # partials beyond the static scratch: 2048 x 64 x (256 + 1) floats
    big = _args(batch=1024, num_q_heads=64, num_kv_heads=8, head_dim=256, flat_splits=1024,
                stride_qb=64 * 256, stride_qh=256, stride_kn=16 * 8 * 256, stride_kt=8 * 256,
                stride_kh=256, stride_ob=64 * 256, stride_oh=256)
    assert lib.pa_decode_noalloc(ctypes.byref(big), None) == _abi.PA_ERR_UNSUPPORTED
    assert "scratch" in lib.pa_last_error().decode()
    big.num_splits, big.flat_splits = 4096, 0
    assert lib.pa_decode_noalloc(ctypes.byref(big), None) == _abi.PA_ERR_UNSUPPORTED
