"""Input builders and error metrics shared by the CPU and GPU tests."""

from __future__ import annotations

import torch


def seeded_q(batch: int, hq: int, d: int, seed: int, device="cpu") -> torch.Tensor:
    """q ~ N(0, 1) fp16 from a CPU generator (identical on every machine)."""
    g = torch.Generator(device="cpu").manual_seed(10_000 + seed)
    return torch.randn((batch, hq, d), dtype=torch.float16, generator=g).to(device)


def max_abs(got: torch.Tensor, ref: torch.Tensor) -> float:
    return (got.float().cpu() - ref.float().cpu()).abs().max().item()


def rel_err(got: torch.Tensor, ref: torch.Tensor) -> float:
    """The reference's metric: max|got - ref| / max|ref| (test_correctness.py:48-51)."""
    r = ref.float().cpu()
    return (got.float().cpu() - r).abs().max().item() / max(r.abs().max().item(), 1e-6)


def subset_cache(cache, rows):
    """A CPU PagedKVCache-like copy holding only batch rows `rows`, with the
    blocks those rows use copied out and the block table renumbered. Lets the
    CPU oracle check sampled sequences of a pool-scale GPU cache."""
    import types

    bt = cache.block_table.cpu()
    lens = cache.seq_lens.cpu()
    bs = cache.block_size
    sel_bt, sel_lens, blocks = [], [], []
    for r in rows:
        n = int(-(-int(lens[r]) // bs))
        ids = bt[r, :n].long()
        base = sum(len(x) for x in blocks)
        blocks.append(ids)
        row = torch.zeros(max(1, bt.shape[1]), dtype=torch.int32)
        row[:n] = torch.arange(base, base + n, dtype=torch.int32)
        sel_bt.append(row)
        sel_lens.append(int(lens[r]))
    ids = torch.cat(blocks) if blocks else torch.zeros(0, dtype=torch.long)
    if ids.numel() == 0:
        ids = torch.zeros(1, dtype=torch.long)
    dev_ids = ids.to(cache.k_cache.device)
    pick = lambda t: None if t is None else t.index_select(0, dev_ids).cpu()
    return types.SimpleNamespace(
        shape=cache.shape,
        block_size=bs,
        kv_dtype=cache.kv_dtype,
        k_cache=pick(cache.k_cache),
        v_cache=pick(cache.v_cache),
        k_scale=pick(cache.k_scale),
        v_scale=pick(cache.v_scale),
        block_table=torch.stack(sel_bt),
        seq_lens=torch.tensor(sel_lens, dtype=torch.int32),
    )


def golden_case(path):
    """(q, cache, sm_scale, npz) of a fixture written by tests/golden/make_golden.py:
    the reference's NHD cache and fp16 q as CPU tensors (the raw bytes, viewed
    back as their types), the fixture's softmax scale, and the open npz (its
    float64 `out`, and `part` / `lse2` / `num_splits` where present)."""
    import numpy as np

    from pagedattn import ModelShape, PagedKVCache

    z = np.load(path, allow_pickle=False)
    kv_dtype = str(z["kv_dtype"])
    sd = {"fp16": torch.float16, "fp32": torch.float32}.get(str(z["scale_dtype"]))
    store = {"fp16": torch.float16, "fp8_e5m2": torch.float8_e5m2, "int8": torch.int8}[kv_dtype]
    as_t = lambda a, dt: torch.from_numpy(a.copy()).view(dt)
    hq, hkv, d = (int(x) for x in z["heads"])
    shape = ModelShape(hq, hkv, d, "golden")
    k = as_t(z["k_cache"], store)
    v = as_t(z["v_cache"], store)
    ks = as_t(z["k_scale"], sd) if sd is not None else None
    vs = as_t(z["v_scale"], sd) if sd is not None else None
    c = PagedKVCache(shape, int(z["block_size"]), kv_dtype, k, v, ks, vs,
                     torch.from_numpy(z["block_table"].copy()), torch.from_numpy(z["seq_lens"].copy()))
    q = torch.from_numpy(z["q"].copy()).view(torch.float16)
    return q, c, float(z["sm_scale"]), z
