"""GPU parity of the HIP decode path against the CPU oracle.

Re-expresses the reference's 49-case matrix
(ParamThakkar123/paged-decode-attention, tests/test_correctness.py) plus the
cases the HIP build adds (fp32 int8 scales, head_dim 32/256, group > 16,
empty sequences, strided vLLM views, bit stability, split partials).

Every case calls the library through its C ABI (pagedattn.hip_decode ->
libpagedattn_hip.so). The bar: max |HIP - oracle_fp32| < 2e-3 (fp16 output
against the fp32 oracle; quantised caches against the oracle applied to the
same quantised cache) and the reference's own relative metric < 1e-2.
"""

from __future__ import annotations

import pytest
import torch

from helpers import max_abs, rel_err, seeded_q, subset_cache
from oracle import reference as oracle
from pagedattn import LLAMA3_8B, LLAMA3_70B, MHA_DEBUG, ModelShape, allocate
from pagedattn.hip_decode import decode_partials, paged_decode_hip, split_reduce

pytestmark = pytest.mark.gpu

ABS_TOL = 2e-3  # max-abs error bar, fp16 output vs fp32 oracle
REL_TOL = 1e-2  # the reference's relative bar (test_correctness.py:28)

# The reference's awkward sizes (test_correctness.py:30-36).
SHAPES = [(2, 64), (2, 65), (3, 300), (1, 1024), (4, 1023), (2, 4097)]


def _qkv(batch, seqlen, kv_dtype="fp16", block_size=16, shape=LLAMA3_8B, seed=0,
         scale_dtype=torch.float16, shuffle=True):
    c = allocate(shape, batch, seqlen, block_size=block_size, kv_dtype=kv_dtype,
                 seed=seed, scale_dtype=scale_dtype, shuffle=shuffle, device="cuda")
    q = seeded_q(batch, shape.num_q_heads, shape.head_dim, seed, device="cuda")
    return q, c


def _check(got, ref, abs_tol=ABS_TOL):
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all(), "non-finite output"
    ma, re = max_abs(got, ref), rel_err(got, ref)
    print(f"max_abs={ma:.2e} rel={re:.2e}", flush=True)
    assert ma < abs_tol, f"max abs error {ma:.3e} >= {abs_tol}"
    assert re < REL_TOL, f"relative error {re:.3e} >= {REL_TOL}"


@pytest.mark.parametrize("batch,seqlen", SHAPES)
@pytest.mark.parametrize("num_splits", [1, 4])
def test_matches_reference(batch, seqlen, num_splits):
    """test_correctness.py:54-61. The reference also sweeps per_page_bt, a
    Triton code-generation knob that this build accepts and ignores; one
    case below checks that it changes nothing."""
    q, c = _qkv(batch, seqlen)
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    got = paged_decode_hip(q, c, num_splits=num_splits)
    _check(got, ref)


def test_per_page_bt_is_ignored():
    """per_page_bt=False (the reference's per-token block-table reads) gives
    the same bytes as the default."""
    q, c = _qkv(4, 1023)
    for splits in (1, 4):
        a = paged_decode_hip(q, c, num_splits=splits, per_page_bt=True).clone()
        b = paged_decode_hip(q, c, num_splits=splits, per_page_bt=False, num_warps=8, num_stages=2)
        torch.cuda.synchronize()
        assert torch.equal(a, b)


@pytest.mark.parametrize("kv_dtype", ["fp16", "fp8_e5m2", "int8"])
@pytest.mark.parametrize("num_splits", [1, 8])
def test_quantized_kv(kv_dtype, num_splits):
    """test_correctness.py:64-70: oracle on the same quantised cache."""
    q, c = _qkv(2, 2048, kv_dtype=kv_dtype)
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    got = paged_decode_hip(q, c, num_splits=num_splits)
    _check(got, ref)


@pytest.mark.parametrize("num_splits", [1, 5])
def test_int8_fp32_scales(num_splits):
    """int8 with fp32 per-(token, head) scales (the C4 benchmark config)."""
    q, c = _qkv(2, 1500, kv_dtype="int8", scale_dtype=torch.float32, shape=LLAMA3_70B, seed=4)
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    got = paged_decode_hip(q, c, num_splits=num_splits)
    _check(got, ref)


@pytest.mark.parametrize("block_size", [16, 32, 64])
def test_page_sizes(block_size):
    """test_correctness.py:73-78."""
    q, c = _qkv(3, 1000, block_size=block_size)
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    got = paged_decode_hip(q, c, block_n=max(64, block_size))
    _check(got, ref)


@pytest.mark.parametrize("block_size", [128, 256])
def test_large_pages(block_size):
    q, c = _qkv(2, 700, block_size=block_size, seed=2)
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    for ns in (1, 3):
        _check(paged_decode_hip(q, c, block_n=block_size, num_splits=ns), ref)


def test_ragged_batch():
    """test_correctness.py:81-90, plus the balanced (max_seq_len) chunking."""
    lens = [7, 1, 4096, 513, 16, 2047, 64, 129]
    c = allocate(LLAMA3_8B, len(lens), lens, seed=3, device="cuda")
    q = seeded_q(len(lens), LLAMA3_8B.num_q_heads, LLAMA3_8B.head_dim, 3, device="cuda")
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    for ns in (1, 4):
        _check(paged_decode_hip(q, c, num_splits=ns), ref)
    for ns in (3, 16, 130):
        _check(paged_decode_hip(q, c, num_splits=ns, max_seq_len=max(lens)), ref)
    # a max_seq_len below the true longest must not drop tokens
    _check(paged_decode_hip(q, c, num_splits=8, max_seq_len=100), ref)


def test_mha_group_one():
    """test_correctness.py:93-97."""
    q, c = _qkv(2, 512, shape=MHA_DEBUG)
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    _check(paged_decode_hip(q, c), ref)


def test_fragmented_vs_sequential_blocks_agree():
    """test_correctness.py:100-110: the block table changes speed, not results."""
    q = seeded_q(2, LLAMA3_8B.num_q_heads, LLAMA3_8B.head_dim, 5, device="cuda")
    for shuffle in (False, True):
        c = allocate(LLAMA3_8B, 2, 1024, shuffle=shuffle, seed=5, device="cuda")
        got = paged_decode_hip(q, c)
        _check(got, oracle.reference_decode(q, c, out_dtype=torch.float32))
    # The same logical cache stored under a permuted pool must give the same bits.
    c = allocate(LLAMA3_8B, 2, 1024, shuffle=False, seed=5, device="cuda", slack_blocks=37)
    base = paged_decode_hip(q, c).clone()
    perm = torch.randperm(c.k_cache.shape[0], generator=torch.Generator().manual_seed(1)).cuda()
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel(), device="cuda")
    c.k_cache = c.k_cache[perm].contiguous()
    c.v_cache = c.v_cache[perm].contiguous()
    c.block_table = inv[c.block_table.long()].to(torch.int32)
    moved = paged_decode_hip(q, c)
    torch.cuda.synchronize()
    assert torch.equal(base, moved), "same logical cache, different block order, different bits"


def test_sdpa_math_crosscheck():
    """test_correctness.py:118-122: the oracle against torch SDPA (math)."""
    q, c = _qkv(2, 512)
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    sdpa = oracle.sdpa_math_decode(q, c)
    assert max_abs(sdpa, ref) < 1e-5
    _check(paged_decode_hip(q, c), sdpa)


@pytest.mark.parametrize("kv_dtype", ["fp8_e5m2", "int8"])
def test_quantization_accuracy(kv_dtype):
    """test_correctness.py:125-145: quantised KV vs the fp16 cache it came from.
    Ceilings int8 0.02, e5m2 0.15 (relative)."""
    q, c16 = _qkv(2, 2048, kv_dtype="fp16", seed=11)
    _, cq = _qkv(2, 2048, kv_dtype=kv_dtype, seed=11)
    ref = oracle.reference_decode(q, c16, out_dtype=torch.float32)
    got = paged_decode_hip(q, cq)
    torch.cuda.synchronize()
    rel = rel_err(got, ref)
    ceiling = {"int8": 0.02, "fp8_e5m2": 0.15}[kv_dtype]
    print(f"{kv_dtype}: max relative output error vs fp16 cache = {rel:.4f}")
    assert rel < ceiling


# (num_q_heads, num_kv_heads, head_dim) of real models (test_correctness.py:156-162)
OTHER_SHAPES = [(32, 8, 128), (64, 8, 128), (32, 8, 64), (14, 2, 64), (16, 2, 64)]


@pytest.mark.parametrize("hq,hkv,d", OTHER_SHAPES)
@pytest.mark.parametrize("num_splits", [1, 4])
def test_other_model_shapes(hq, hkv, d, num_splits):
    """test_correctness.py:165-174."""
    shape = ModelShape(hq, hkv, d, name=f"{hq}x{hkv}x{d}")
    q, c = _qkv(3, 777, shape=shape, seed=7)
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    _check(paged_decode_hip(q, c, num_splits=num_splits), ref)


@pytest.mark.parametrize("hq,hkv,d", [(8, 2, 32), (16, 4, 256), (40, 2, 128), (24, 1, 64)])
@pytest.mark.parametrize("kv_dtype", ["fp16", "fp8_e5m2", "int8"])
def test_head_dims_and_wide_groups(hq, hkv, d, kv_dtype):
    """head_dim 32 / 256 and groups above 16 (two head tiles)."""
    shape = ModelShape(hq, hkv, d, name=f"{hq}x{hkv}x{d}")
    q, c = _qkv(2, 333, shape=shape, seed=8, kv_dtype=kv_dtype)
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    for ns in (1, 3):
        _check(paged_decode_hip(q, c, num_splits=ns), ref)


def test_sm_scale_override():
    q, c = _qkv(2, 300, seed=9)
    ref = oracle.reference_decode(q, c, sm_scale=0.05, out_dtype=torch.float32)
    _check(paged_decode_hip(q, c, sm_scale=0.05), ref)
    _check(paged_decode_hip(q, c, sm_scale=0.05, num_splits=3), ref)


def test_empty_sequences_give_zeros():
    lens = [0, 5, 0, 40]
    c = allocate(LLAMA3_8B, 4, lens, seed=12, device="cuda")
    q = seeded_q(4, 32, 128, 12, device="cuda")
    for ns in (1, 4):
        got = paged_decode_hip(q, c, num_splits=ns)
        torch.cuda.synchronize()
        assert torch.equal(got[0], torch.zeros_like(got[0]))
        assert torch.equal(got[2], torch.zeros_like(got[2]))
        ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
        _check(got[[1, 3]], ref[[1, 3]])


def test_vllm_style_strided_views():
    """K/V as `kv_cache.unbind(0)` views of a [2, NB, P, Hkv, D] tensor, q/out
    as slices of larger buffers (integration/vllm_backend.py:113,124-126)."""
    c = allocate(LLAMA3_8B, 3, [100, 1, 513], seed=13, device="cuda")
    kv = torch.stack([c.k_cache, c.v_cache])  # [2, NB, P, H, D]
    k_view, v_view = kv.unbind(0)
    c.k_cache, c.v_cache = k_view, v_view
    qbuf = seeded_q(5, 32, 128, 13, device="cuda")
    q = qbuf[:3]
    outbuf = torch.zeros((5, 32, 128), dtype=torch.float16, device="cuda")
    out = outbuf[:3]
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    paged_decode_hip(q, c, out=out, num_splits=2)
    _check(out, ref)
    torch.cuda.synchronize()
    assert torch.equal(outbuf[3:], torch.zeros_like(outbuf[3:])), "wrote outside out"


def test_reduce_many_splits():
    """The reduce kernel over more splits than it stages at once (256)."""
    lens = [40000, 3]
    c = allocate(LLAMA3_8B, 2, lens, seed=17, device="cuda")
    q = seeded_q(2, 32, 128, 17, device="cuda")
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    _check(paged_decode_hip(q, c, num_splits=600, max_seq_len=max(lens)), ref)
    _check(paged_decode_hip(q, c, num_splits=300), ref)


@pytest.mark.parametrize("kv_dtype", ["fp16", "fp8_e5m2", "int8"])
def test_bit_stable(kv_dtype):
    q, c = _qkv(4, 3000, seed=14, kv_dtype=kv_dtype)
    for ns in (1, 7):
        a = paged_decode_hip(q, c, num_splits=ns).clone()
        b = paged_decode_hip(q, c, num_splits=ns).clone()
        torch.cuda.synchronize()
        assert torch.equal(a, b)


@pytest.mark.parametrize("num_splits", [1, 3, 16])
@pytest.mark.parametrize("balanced", [False, True])
def test_split_partials_match_oracle(num_splits, balanced):
    """The decode pass alone against the oracle's per-split restatement
    (triton_decode.py:169-188), and the reduce kernel against split_merge."""
    lens = [1, 100, 700]
    c = allocate(LLAMA3_8B, 3, lens, seed=15, device="cuda")
    q = seeded_q(3, 32, 128, 15, device="cuda")
    msl = max(lens) if balanced else 0
    po, pl = decode_partials(q, c, num_splits, max_seq_len=msl)
    torch.cuda.synchronize()
    ref_po, ref_pl = oracle.split_partials(q, c, num_splits, align=32, max_seq_len=msl)
    fin = torch.isfinite(ref_pl)
    assert torch.equal(torch.isfinite(pl.cpu()), fin), "empty-split pattern differs"
    assert (pl.cpu()[fin] - ref_pl[fin]).abs().max().item() < 1e-3
    assert (po.cpu() - ref_po).abs().max().item() < 2e-3
    out = split_reduce(po, pl)
    ref = oracle.split_merge(ref_po, ref_pl)
    _check(out, ref)
    _check(out, oracle.reference_decode(q, c, out_dtype=torch.float32))


def test_auto_split_count():
    q, c = _qkv(1, 5000, seed=16)
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    _check(paged_decode_hip(q, c), ref)


# bf16 output is rounded to bf16 (8-bit significand): half an ulp of |ref| on
# top of the kernel's own 2e-3 bar
def _check_bf16(got, ref):
    torch.cuda.synchronize()
    assert got.dtype == torch.bfloat16
    err = (got.float().cpu() - ref.float().cpu()).abs()
    bound = ABS_TOL + 2.0 ** -8 * ref.float().cpu().abs()
    print(f"bf16 max_abs={err.max().item():.2e} worst margin={(err - bound).max().item():.2e}")
    assert bool((err <= bound).all()), f"bf16 error above bound by {(err - bound).max().item():.3e}"


@pytest.mark.parametrize("kv_dtype", ["bf16", "fp16", "fp8_e5m2", "int8"])
@pytest.mark.parametrize("num_splits", [1, 5])
def test_bf16_q_and_out(kv_dtype, num_splits):
    """bf16 q/out (converted in registers; the reference maps bf16 onto its
    fp16 path, triton_decode.py:30,151-153) with every KV dtype."""
    lens = [1, 300, 2049]
    c = allocate(LLAMA3_8B, 3, lens, kv_dtype=kv_dtype, seed=19, device="cuda")
    q = seeded_q(3, 32, 128, 19, device="cuda").to(torch.bfloat16)
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    got = paged_decode_hip(q, c, num_splits=num_splits)
    _check_bf16(got, ref)


@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (8, 2, 32), (16, 4, 256)])
def test_bf16_cache_fp16_q(hq, hkv, d):
    shape = ModelShape(hq, hkv, d, name=f"{hq}x{hkv}x{d}")
    q, c = _qkv(2, 333, shape=shape, seed=20, kv_dtype="bf16")
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    for ns in (1, 3):
        _check(paged_decode_hip(q, c, num_splits=ns), ref)


def test_bf16_split_reduce_output():
    lens = [700, 40]
    c = allocate(LLAMA3_8B, 2, lens, kv_dtype="bf16", seed=21, device="cuda")
    q = seeded_q(2, 32, 128, 21, device="cuda").to(torch.bfloat16)
    po, pl = decode_partials(q, c, 4)
    out = split_reduce(po, pl, torch.empty((2, 32, 128), dtype=torch.bfloat16, device="cuda"))
    _check_bf16(out, oracle.reference_decode(q, c, out_dtype=torch.float32))


@pytest.mark.parametrize("block_size", [128, 256])
@pytest.mark.parametrize("kv_dtype,scale_dtype", [("fp16", torch.float16), ("bf16", torch.float16),
                                                  ("fp8_e5m2", torch.float16), ("int8", torch.float16),
                                                  ("int8", torch.float32)])
@pytest.mark.parametrize("shape", [LLAMA3_8B, ModelShape(12, 2, 64, "g6-d64")], ids=["llama3-8b", "g6-d64"])
def test_large_pages_every_kv_dtype_and_launch(block_size, kv_dtype, scale_dtype, shape):
    """Pages of 128 and 256 tokens (several 32-token tiles per page, so a
    tile's two 16-row sub-tiles share one block-table entry) for every KV
    type, through the unsplit, classic split and flat launches (with and
    without host lengths). At 2 kv heads a flat workgroup spans several
    ranges (4 per workgroup for int8, 2 otherwise)."""
    lens = [700, 1, 0, 2 * block_size + 5, 257]
    c = allocate(shape, len(lens), lens, block_size=block_size, kv_dtype=kv_dtype, seed=11,
                 scale_dtype=scale_dtype, device="cuda")
    q = seeded_q(len(lens), shape.num_q_heads, shape.head_dim, 11, device="cuda")
    ref = oracle.reference_decode(q, c, out_dtype=torch.float32)
    host = torch.tensor(lens, dtype=torch.int32)
    live = [i for i, t in enumerate(lens) if t > 0]

    def check(got):
        # the oracle's empty row is 0/0; the kernels write zeros there
        _check(got[live], ref[live])
        assert torch.equal(got[2].float().cpu(), torch.zeros(shape.num_q_heads, shape.head_dim))

    bn = block_size  # the reference's BLOCK_N check: a multiple of the page size
    check(paged_decode_hip(q, c, block_n=bn, num_splits=1))
    check(paged_decode_hip(q, c, block_n=bn, num_splits=3, max_seq_len=max(lens)))
    for f in (1, 7, 64):
        check(paged_decode_hip(q, c, block_n=bn, flat_splits=f))
        check(paged_decode_hip(q, c, block_n=bn, flat_splits=f, flat_seq_cost=2, seq_lens_host=host))
