"""Paged KV cache: the container the decode kernel reads, and a seeded filler.

Layout is vLLM-V1 / FlashInfer "NHD", as in the reference
(ParamThakkar123/paged-decode-attention, pagedattn/cache.py:3-12):

    k_cache, v_cache : [num_blocks, block_size, num_kv_heads, head_dim]
    k_scale, v_scale : [num_blocks, block_size, num_kv_heads]   (int8 only)
    block_table      : [batch, max_blocks] int32 (physical block per page)
    seq_lens         : [batch] int32

head_dim is innermost, so one (block, token, head) row is contiguous and the
HIP kernel reads it with 16-byte loads.

Differences from the reference, all deliberate:
  * `allocate` fills K/V from a CPU generator by default (`fill_device="cpu"`)
    and copies the result to the target device, so a CPU oracle and the GPU
    kernel see identical bytes. `fill_device="cuda"` generates on the GPU
    instead, for pool-scale benchmark caches where parity is checked by
    reading back the blocks under test.
  * int8 scales may be fp16 (the reference's choice, cache.py:45) or fp32
    (`scale_dtype=torch.float32`).
  * `bytes_read_per_decode_step` counts the scale bytes at their real size.
"""

from __future__ import annotations

import dataclasses

import torch

from .config import KVDType, ModelShape, torch_dtype

# e5m2 shares fp16's 5-bit exponent, so fp16 -> e5m2 is a mantissa rounding
# and e5m2 -> fp16 is exact (cache.py:27-30).
FP8_E5M2_MAX = 57344.0
INT8_MAX = 127.0


def quantize_kv(
    x: torch.Tensor, kv_dtype: KVDType, scale_dtype: torch.dtype = torch.float16
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Quantise a [..., num_kv_heads, head_dim] fp16 tensor to the cache dtype.

    Semantics of the reference's `quantize_kv` (cache.py:33-48): fp16/bf16 are
    casts, fp8_e5m2 is torch's round-to-nearest cast, int8 uses one scale per
    (token, head): amax over head_dim clamped to 1e-6, scale = amax / 127
    rounded to `scale_dtype`, q = round_half_even(x / scale) clamped to +-127.
    Returns (stored, scale) with scale None for the unscaled dtypes.
    """
    if kv_dtype in ("fp16", "bf16"):
        return x.to(torch_dtype(kv_dtype)), None
    if kv_dtype == "fp8_e5m2":
        return x.to(torch.float8_e5m2), None
    if kv_dtype == "int8":
        amax = x.abs().amax(dim=-1, keepdim=True).float().clamp_min(1e-6)
        scale = (amax / INT8_MAX).to(scale_dtype)
        q = (x.float() / scale.float()).round().clamp(-INT8_MAX, INT8_MAX).to(torch.int8)
        return q, scale.squeeze(-1)
    raise ValueError(f"unknown kv_dtype {kv_dtype}")


def dequantize_kv(
    q: torch.Tensor, scale: torch.Tensor | None, kv_dtype: KVDType
) -> torch.Tensor:
    """Stored cache rows -> fp16, the values the decode kernel attends over.

    The reference's `dequantize_kv` (cache.py:51-62): fp16 / bf16 / fp8_e5m2
    are casts to fp16 (e5m2 -> fp16 is exact, bf16 -> fp16 rounds to nearest
    even). int8 is `fp16(x * scale)` with one scale per (token, head), i.e.
    `scale` has q's shape without the last (head_dim) axis. The product is
    formed in fp32 and rounded once: for an fp16 scale the product of an
    8-bit integer and an 11-bit significand is exact in fp32, so this equals
    the reference's fp16 multiply bit for bit; for fp32 scales it is the
    single rounding the kernel applies.
    """
    if kv_dtype in ("fp16", "bf16", "fp8_e5m2"):
        return q.to(torch.float16)
    if kv_dtype == "int8":
        if scale is None:
            raise ValueError("int8 rows need their per-(token, head) scales")
        prod = q.to(torch.float32) * scale.to(torch.float32)[..., None]
        return prod.to(torch.float16)
    raise ValueError(f"unknown kv_dtype {kv_dtype}")


@dataclasses.dataclass
class PagedKVCache:
    """The reference's cache dataclass (cache.py:70-102), same field names."""

    shape: ModelShape
    block_size: int
    kv_dtype: KVDType
    k_cache: torch.Tensor  # [num_blocks, block_size, H_kv, D]
    v_cache: torch.Tensor
    k_scale: torch.Tensor | None  # [num_blocks, block_size, H_kv] fp16/fp32, int8 only
    v_scale: torch.Tensor | None
    block_table: torch.Tensor  # [B, max_blocks] int32
    seq_lens: torch.Tensor  # [B] int32

    @property
    def batch(self) -> int:
        return int(self.block_table.shape[0])

    @property
    def num_blocks(self) -> int:
        return int(self.k_cache.shape[0])

    def bytes_read_per_decode_step(self) -> int:
        """K/V (+ scale) bytes a perfect decode kernel must read (cache.py:90-102).

        Counts only tokens inside each sequence. This is the reference's
        bandwidth denominator; `algorithmic_bytes` adds q, out and the block
        table on top.
        """
        n_tok = int(self.seq_lens.sum().item())
        h, d = self.shape.num_kv_heads, self.shape.head_dim
        elem = self.k_cache.element_size()
        total = 2 * n_tok * h * d * elem
        if self.kv_dtype == "int8":
            assert self.k_scale is not None
            total += 2 * n_tok * h * self.k_scale.element_size()
        return total

    def algorithmic_bytes(self, q_elem_bytes: int = 2) -> int:
        """Minimum HBM bytes of one decode call: K/V (+ scales) + q + out + the
        block-table entries actually used."""
        b = self.batch
        hq, d = self.shape.num_q_heads, self.shape.head_dim
        lens = self.seq_lens.to("cpu", torch.int64)
        pages = int(((lens + self.block_size - 1) // self.block_size).sum().item())
        return self.bytes_read_per_decode_step() + 2 * b * hq * d * q_elem_bytes + 4 * pages


def _lens_tensor(batch: int, seq_lens) -> torch.Tensor:
    if isinstance(seq_lens, int):
        t = torch.full((batch,), seq_lens, dtype=torch.int32)
    elif isinstance(seq_lens, (list, tuple)):
        t = torch.tensor(list(seq_lens), dtype=torch.int32)
    else:
        t = seq_lens.to(torch.int32).cpu()
    assert t.numel() == batch, f"seq_lens has {t.numel()} entries for batch {batch}"
    return t


def allocate(
    shape: ModelShape,
    batch: int,
    seq_lens: torch.Tensor | list[int] | int,
    block_size: int = 16,
    kv_dtype: KVDType = "fp16",
    device: str = "cuda",
    shuffle: bool = True,
    seed: int = 0,
    slack_blocks: int = 0,
    scale_dtype: torch.dtype = torch.float16,
    fill_device: str = "cpu",
) -> PagedKVCache:
    """Allocate a paged cache and fill it with a seeded random KV state.

    Follows the reference's `allocate` (cache.py:105-184): pool = sum of
    ceil(T_b / block_size) blocks + `slack_blocks`; K and V are N(0, 1) fp16
    generated in chunks (K then V per chunk) and quantised with `quantize_kv`;
    the used blocks are the first sum(ceil(T_b / P)) entries of a seeded
    `randperm(pool)` (or ascending when `shuffle` is False), dealt out to the
    sequences in order; unused block-table entries are 0.
    """
    gen = torch.Generator(device="cpu").manual_seed(seed)
    seq_lens_t = _lens_tensor(batch, seq_lens)

    blocks_per_seq = ((seq_lens_t + block_size - 1) // block_size).tolist()
    max_blocks = max(1, max(blocks_per_seq) if blocks_per_seq else 1)
    used_blocks = sum(blocks_per_seq)
    total_blocks = max(1, used_blocks + slack_blocks)

    h, d = shape.num_kv_heads, shape.head_dim
    store_dtype = torch_dtype(kv_dtype)
    k_cache = torch.empty((total_blocks, block_size, h, d), dtype=store_dtype, device=device)
    v_cache = torch.empty_like(k_cache)
    need_scale = kv_dtype == "int8"
    k_scale = (
        torch.empty((total_blocks, block_size, h), dtype=scale_dtype, device=device)
        if need_scale
        else None
    )
    v_scale = torch.empty_like(k_scale) if k_scale is not None else None

    fill_gen = torch.Generator(device=fill_device).manual_seed(seed)
    # ~64 MiB of fp16 per chunk
    chunk = max(1, min(total_blocks, (64 << 20) // (block_size * h * d * 2)))
    for start in range(0, total_blocks, chunk):
        stop = min(start + chunk, total_blocks)
        for dst, dst_scale in ((k_cache, k_scale), (v_cache, v_scale)):
            raw = torch.randn(
                (stop - start, block_size, h, d),
                dtype=torch.float16,
                device=fill_device,
                generator=fill_gen,
            )
            qv, s = quantize_kv(raw, kv_dtype, scale_dtype)
            dst[start:stop] = qv.to(device)
            if s is not None:
                assert dst_scale is not None
                dst_scale[start:stop] = s.to(device)
            del raw, qv, s

    perm = (
        torch.randperm(total_blocks, generator=gen)[:used_blocks]
        if shuffle
        else torch.arange(used_blocks)
    )
    block_table = torch.zeros((batch, max_blocks), dtype=torch.int32)
    cursor = 0
    for b, nb in enumerate(blocks_per_seq):
        block_table[b, :nb] = perm[cursor : cursor + nb].to(torch.int32)
        cursor += nb

    return PagedKVCache(
        shape=shape,
        block_size=block_size,
        kv_dtype=kv_dtype,
        k_cache=k_cache,
        v_cache=v_cache,
        k_scale=k_scale,
        v_scale=v_scale,
        block_table=block_table.to(device),
        seq_lens=seq_lens_t.to(device),
    )


def gather_contiguous(cache: PagedKVCache) -> tuple[torch.Tensor, torch.Tensor]:
    """The paged cache as dense [B, H_kv, S_max, D] fp16 K and V tensors.

    The reference's `gather_contiguous` (cache.py:187-215), for callers that
    need a page-free view (dense attention baselines, debugging, the oracle's
    own restatement). It runs on the cache's device with torch indexing and
    is not part of the decode path: the HIP kernels read the pages in place.

    Position s of sequence b reads page `block_table[b, s // P]` at row
    `s % P`, dequantised with `dequantize_kv`. Positions at or past T_b hold
    whatever their page-table entry points at: the column index is clamped
    to the last column of the block table and unused entries are 0, as in
    the reference, so callers mask them by `seq_lens`.
    """
    bt = cache.block_table
    b = int(bt.shape[0])
    h, d = cache.shape.num_kv_heads, cache.shape.head_dim
    dev = cache.k_cache.device
    s_max = int(cache.seq_lens.max().item()) if b else 0
    if b == 0 or s_max <= 0:
        empty = torch.empty((b, h, 0, d), dtype=torch.float16, device=dev)
        return empty, empty.clone()
    page = cache.block_size
    pos = torch.arange(s_max, device=bt.device)
    col = torch.clamp(pos // page, max=int(bt.shape[1]) - 1)
    blocks = bt.index_select(1, col).to(dev, torch.long)        # [B, S] physical block
    rows = (pos % page).to(dev).unsqueeze(0).expand(b, s_max)  # [B, S] row in the page

    def dense(rows_t: torch.Tensor, scale_t: torch.Tensor | None) -> torch.Tensor:
        vals = rows_t[blocks, rows]                            # [B, S, H, D] stored dtype
        sc = None if scale_t is None else scale_t[blocks, rows]  # [B, S, H]
        return dequantize_kv(vals, sc, cache.kv_dtype).transpose(1, 2).contiguous()

    return dense(cache.k_cache, cache.k_scale), dense(cache.v_cache, cache.v_scale)
