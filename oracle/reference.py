"""CPU oracle for paged GQA decode attention -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker. The product
(paged-decode-attention_amd/) never imports it and has no CPU path.

A from-scratch restatement, in torch on the CPU, of the reference's algorithm
(ParamThakkar123/paged-decode-attention):

  quantize_kv        pagedattn/cache.py:33-48
  dequantize_kv      pagedattn/cache.py:51-62
  gather_contiguous  pagedattn/cache.py:187-215
  reference_decode   pagedattn/reference.py:28-49
  split_partials     pagedattn/triton_decode.py:78-85 (per-split KV range) and
                     :169-188 (normalised partial + log2-sum-exp, empty = -inf)
  split_merge        pagedattn/triton_decode.py:198-240
  sdpa_math_decode   pagedattn/reference.py:57-72 (SDPA math backend, GQA)
  write_kv           the KV write before the decode (integration/vllm_backend.py:
                     117-122, vLLM's reshape_and_cache_flash) with the
                     quantisation of pagedattn/cache.py:33-48

Deviations, each deliberate: `reference_decode` takes `sm_scale` (the
reference always uses head_dim**-0.5, reference.py:45) and can return the
fp32 result before the final cast (`out_dtype=torch.float32`); the reference
casts to q.dtype (reference.py:49). Everything works on any object carrying
the PagedKVCache field names (shape, block_size, kv_dtype, k_cache, v_cache,
k_scale, v_scale, block_table, seq_lens), so this module does not import the
product package.

How each function is pinned (tests/test_oracle.py): an independent float64
C implementation that walks the pages directly (oracle/pa_oracle.c), closed
forms (T=1, q=0, constant V, a dominant logit), torch SDPA's math backend on
the gathered cache, block-table permutation invariance, e5m2 bit identities
and int8 round-trip bounds, and the golden fixtures under tests/golden/.
"""

from __future__ import annotations

import math

import torch

INT8_MAX = 127.0


def quantize_kv(x: torch.Tensor, kv_dtype: str, scale_dtype: torch.dtype = torch.float16):
    """fp16 [..., H, D] -> (stored, scale or None). cache.py:33-48."""
    if kv_dtype == "fp16":
        return x.to(torch.float16), None
    if kv_dtype == "bf16":
        return x.to(torch.bfloat16), None
    if kv_dtype == "fp8_e5m2":
        return x.to(torch.float8_e5m2), None
    if kv_dtype == "int8":
        amax = x.abs().amax(dim=-1, keepdim=True).float().clamp_min(1e-6)
        scale = (amax / INT8_MAX).to(scale_dtype)
        q = torch.round(x.float() / scale.float()).clamp(-INT8_MAX, INT8_MAX).to(torch.int8)
        return q, scale.squeeze(-1)
    raise ValueError(f"unknown kv_dtype {kv_dtype}")


def dequantize_kv(q: torch.Tensor, scale: torch.Tensor | None, kv_dtype: str) -> torch.Tensor:
    """Stored KV -> fp16. cache.py:51-62.

    int8: the product int8 * scale is formed in fp32 and rounded once to fp16.
    With an fp16 scale this equals the reference's fp16 multiply (the product
    of an 8-bit integer and an 11-bit significand is exact in fp32).
    """
    if kv_dtype in ("fp16", "bf16", "fp8_e5m2"):
        return q.to(torch.float16)
    if kv_dtype == "int8":
        assert scale is not None
        return (q.float() * scale.float().unsqueeze(-1)).to(torch.float16)
    raise ValueError(f"unknown kv_dtype {kv_dtype}")


def gather_contiguous(cache) -> tuple[torch.Tensor, torch.Tensor]:
    """Dense [B, H_kv, S_max, D] fp16 K and V. cache.py:187-215.

    Positions past a sequence's last page read the page-table entry clamped to
    the last column (padding rows); the caller masks them.
    """
    bt = cache.block_table.cpu().long()
    lens = cache.seq_lens.cpu().long()
    b = bt.shape[0]
    s_max = int(lens.max().item()) if b else 0
    bs = cache.block_size
    pos = torch.arange(s_max)
    blk = (pos // bs).clamp(max=bt.shape[1] - 1)
    off = pos % bs
    phys = bt[:, blk]  # [B, S]
    offs = off.unsqueeze(0).expand(b, -1)
    out = []
    for cache_t, scale_t in ((cache.k_cache, cache.k_scale), (cache.v_cache, cache.v_scale)):
        c = cache_t.cpu()
        flat = c[phys, offs]  # [B, S, H, D]
        s = scale_t.cpu()[phys, offs] if scale_t is not None else None
        flat = dequantize_kv(flat, s, cache.kv_dtype)
        out.append(flat.permute(0, 2, 1, 3).contiguous())
    return out[0], out[1]


def _softmax_scale(cache, sm_scale: float | None) -> float:
    return cache.shape.head_dim ** -0.5 if sm_scale is None else float(sm_scale)


def reference_decode(
    q: torch.Tensor,
    cache,
    sm_scale: float | None = None,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """fp32 paged GQA decode attention on the CPU. reference.py:28-49.

    q: [B, H_q, D] -> [B, H_q, D] in `out_dtype` (default q.dtype). Query head
    h reads kv head h // group. A sequence of length 0 gives NaN, as in the
    reference (softmax over an all -inf row).
    """
    qc = q.cpu()
    b, hq, d = qc.shape
    hkv = cache.shape.num_kv_heads
    group = hq // hkv
    k, v = gather_contiguous(cache)
    k = k.float()
    v = v.float()
    qf = qc.float()
    s_max = k.shape[2]
    lens = cache.seq_lens.cpu().long()
    valid = torch.arange(s_max).unsqueeze(0) < lens.unsqueeze(1)  # [B, S]
    scale = _softmax_scale(cache, sm_scale)
    out = torch.empty((b, hq, d), dtype=torch.float32)
    for h in range(hq):
        kvh = h // group
        logits = torch.einsum("bd,bsd->bs", qf[:, h], k[:, kvh]) * scale
        logits = logits.masked_fill(~valid, float("-inf"))
        p = torch.softmax(logits, dim=-1)
        out[:, h] = torch.einsum("bs,bsd->bd", p, v[:, kvh])
    return out.to(q.dtype if out_dtype is None else out_dtype)


def split_ranges(seq_len: int, num_splits: int, align: int, max_seq_len: int = 0) -> list[tuple[int, int]]:
    """[lo, hi) of each split: chunk = ceil(ceil(T/align)/S)*align.
    triton_decode.py:78-85 with the alignment unit as a parameter.

    With max_seq_len > 0 the chunk is sized from max_seq_len instead (but
    never below the sequence's own chunk): the HIP build's balanced mode for
    ragged batches. Ranges are clamped to [T, T) once past the end."""
    def chunk_of(t):
        return -(-(-(-t // align)) // num_splits) * align
    chunk = chunk_of(seq_len)
    if max_seq_len > 0:
        chunk = max(chunk, chunk_of(max_seq_len))
    out = []
    for s in range(num_splits):
        lo = min(s * chunk, seq_len)
        out.append((lo, min(lo + chunk, seq_len)))
    return out


def split_partials(
    q: torch.Tensor,
    cache,
    num_splits: int,
    align: int = 32,
    sm_scale: float | None = None,
    max_seq_len: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-split normalised output [B, Hq, S, D] and log2-sum-exp [B, Hq, S].

    For split s over tokens [lo, hi): with x_j = q.k_j * scale * log2(e),
    lse = log2(sum_j 2^x_j) and out = sum_j 2^(x_j - lse) v_j; an empty split
    has lse = -inf and out = 0 (triton_decode.py:169-188).
    """
    qc = q.cpu().float()
    b, hq, d = qc.shape
    hkv = cache.shape.num_kv_heads
    group = hq // hkv
    k, v = gather_contiguous(cache)
    k = k.float()
    v = v.float()
    scale = _softmax_scale(cache, sm_scale) * math.log2(math.e)
    lens = cache.seq_lens.cpu().long().tolist()
    part = torch.zeros((b, hq, num_splits, d), dtype=torch.float32)
    lse = torch.full((b, hq, num_splits), float("-inf"), dtype=torch.float32)
    for bi in range(b):
        for s, (lo, hi) in enumerate(split_ranges(lens[bi], num_splits, align, max_seq_len)):
            if lo >= hi:
                continue
            for h in range(hq):
                kvh = h // group
                x = (k[bi, kvh, lo:hi] @ qc[bi, h]) * scale  # [n]
                m = x.max()
                w = torch.exp2(x - m)
                den = w.sum()
                part[bi, h, s] = (w @ v[bi, kvh, lo:hi]) / den
                lse[bi, h, s] = m + torch.log2(den)
    return part, lse


def flat_segments(seq_lens, flat_splits: int, align: int = 32,
                  seq_cost: int = 0) -> tuple[list[tuple[int, int, int, int]], int]:
    """The flat split's work list and range size: ([(j, b, lo, hi)], per).

    No counterpart in the reference: the HIP build's work-balanced split.
    Sequence b has n_b = ceil(T_b / align) tiles and, when non-empty, weighs
    n_b + seq_cost; sequences are laid end to end in batch order, so b spans
    weights [cw_b, cw_b + seq_cost + n_b) and its tile k sits at weight
    cw_b + seq_cost + k. Range j covers weights [j * per, (j + 1) * per) with
    per = max(1, ceil(W / flat_splits)) over the total weight W and holds the
    tiles whose weights fall inside. Each (j, b, lo, hi) is the token range
    [lo, hi) of sequence b that range j holds, in order. seq_cost = 0 is the
    plain split of the tiles into equal ranges.
    """
    lens = [max(0, int(t)) for t in seq_lens]
    tiles = [-(-t // align) for t in lens]
    weights = [n + seq_cost if n else 0 for n in tiles]
    total = sum(weights)
    per = max(1, -(-total // flat_splits))
    segs = []
    cw = 0
    for b, (t, n) in enumerate(zip(lens, tiles)):
        first = cw + seq_cost  # weight of tile 0
        f = first
        while f < first + n:
            j = f // per
            end = min(first + n, (j + 1) * per)
            segs.append((j, b, (f - first) * align, min((end - first) * align, t)))
            f = end
        cw += weights[b]
    return segs, per


def flat_partials(
    q: torch.Tensor,
    cache,
    flat_splits: int,
    align: int = 32,
    sm_scale: float | None = None,
    seq_cost: int = 0,
) -> tuple[torch.Tensor, torch.Tensor, list[bool]]:
    """The flat decode pass: (part [B + F, Hq, D], lse [B + F, Hq], whole [B]).

    Slot b + j holds the normalised output and log2-sum-exp (as in
    split_partials) of the segment of sequence b in range j; whole[b] is True
    when one range holds all of b (the decode then writes `out` instead of a
    slot). Unused slots stay (0, -inf).
    """
    qc = q.cpu().float()
    b, hq, d = qc.shape
    group = hq // cache.shape.num_kv_heads
    k, v = gather_contiguous(cache)
    k = k.float()
    v = v.float()
    scale = _softmax_scale(cache, sm_scale) * math.log2(math.e)
    lens = cache.seq_lens.cpu().long().tolist()
    segs, _ = flat_segments(lens, flat_splits, align, seq_cost)
    part = torch.zeros((b + flat_splits, hq, d), dtype=torch.float32)
    lse = torch.full((b + flat_splits, hq), float("-inf"), dtype=torch.float32)
    count = [0] * b
    for _, bi, _, _ in segs:
        count[bi] += 1
    for j, bi, lo, hi in segs:
        for h in range(hq):
            kvh = h // group
            x = (k[bi, kvh, lo:hi] @ qc[bi, h]) * scale
            m = x.max()
            w = torch.exp2(x - m)
            den = w.sum()
            part[bi + j, h] = (w @ v[bi, kvh, lo:hi]) / den
            lse[bi + j, h] = m + torch.log2(den)
    return part, lse, [c == 1 for c in count]


def split_merge(part: torch.Tensor, lse: torch.Tensor) -> torch.Tensor:
    """out = sum_s part_s 2^(lse_s - m) / sum_s 2^(lse_s - m). triton_decode.py:221-240.
    Returns fp32 [B, H, D]; rows whose splits are all empty give NaN (0/0),
    as the reference does."""
    m = lse.max(dim=-1, keepdim=True).values
    w = torch.exp2(lse - m)
    w = torch.where(torch.isfinite(lse), w, torch.zeros_like(w))
    return (part * w.unsqueeze(-1)).sum(dim=2) / w.sum(dim=-1, keepdim=True)


def sdpa_math_decode(q: torch.Tensor, cache, sm_scale: float | None = None) -> torch.Tensor:
    """torch SDPA (math backend, enable_gqa) on the gathered cache, fp32.
    The library cross-check of reference.py:57-72 / tests/test_correctness.py:118-122."""
    import torch.nn.functional as F

    k, v = gather_contiguous(cache)
    qf = q.cpu().float().unsqueeze(2)  # [B, Hq, 1, D]
    lens = cache.seq_lens.cpu().long()
    s = k.shape[2]
    mask = (torch.arange(s).view(1, 1, 1, -1) < lens.view(-1, 1, 1, 1))
    with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.MATH):
        o = F.scaled_dot_product_attention(
            qf, k.float(), v.float(), attn_mask=mask,
            enable_gqa=(qf.shape[1] != k.shape[1]),
            scale=_softmax_scale(cache, sm_scale),
        )
    return o.squeeze(2)


def bytes_read_per_decode_step(cache) -> int:
    """K/V (+ scale) bytes inside the sequences. cache.py:90-102, with the
    scale counted at its real element size."""
    n_tok = int(cache.seq_lens.cpu().long().sum().item())
    h, d = cache.shape.num_kv_heads, cache.shape.head_dim
    elem = cache.k_cache.element_size()
    total = 2 * n_tok * h * d * elem
    if cache.kv_dtype == "int8":
        total += 2 * n_tok * h * cache.k_scale.element_size()
    return total


def write_kv(key: torch.Tensor, value: torch.Tensor, cache, slot_mapping: torch.Tensor) -> None:
    """Scatter key/value [n, H_kv, D] (fp16) into a CPU cache at slot_mapping,
    row by row, quantised with `quantize_kv` (cache.py:33-48). Slots < 0 or at
    or past num_blocks * block_size are skipped. Mutates `cache` in place."""
    bs = cache.block_size
    nb = cache.k_cache.shape[0]
    slots = slot_mapping.cpu().long().tolist()
    for t, slot in enumerate(slots):
        if slot < 0 or slot >= nb * bs:
            continue
        blk, off = divmod(slot, bs)
        for src, dst, dst_scale in ((key, cache.k_cache, cache.k_scale), (value, cache.v_cache, cache.v_scale)):
            scale_dtype = dst_scale.dtype if dst_scale is not None else torch.float16
            qv, s = quantize_kv(src[t].cpu().unsqueeze(0), cache.kv_dtype, scale_dtype)
            dst[blk, off] = qv[0]
            if s is not None:
                dst_scale[blk, off] = s[0]
