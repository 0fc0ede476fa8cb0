"""Why int8 K must be rounded to fp16 as the reference rounds it (CPU only).

The reference's kernel dequantises every int8 K and V element to
fp16(x * s) (pagedattn/triton_decode.py:145-149, the values of
pagedattn/cache.py:51-62), takes fp16 q . fp16 K with fp32 accumulation
(:155), rounds the probabilities to fp16 before P.V (:165) and the output to
fp16 (:193). The decode's bar compares against the fp32 oracle on the same
dequantised cache (pagedattn/reference.py:28-49 restated), max-abs < 2e-3.

This file emulates that chain tile by tile (64-token tiles, online softmax in
the log2 domain) on the inputs of tests/test_gpu_int8_q_range.py, whose q
heads span magnitudes from 0 to 3x (peaked softmaxes), and checks:
  * the reference's own chain stays within the plain 2e-3 bar on every case,
    so the bar needs no widening for int8;
  * the same chain over the unrounded K, x * s exactly (the arithmetic of an
    integer QK product), moves away from the oracle by more than the
    reference's chain does and beyond 1.5e-3 on these inputs: K's fp16
    rounding is part of the semantics the oracle fixes, so the HIP kernel
    rounds K per element as the reference does (csrc/paged_decode.hip).
"""

from __future__ import annotations

import math

import pytest
import torch

from helpers import seeded_q
from oracle import reference as oracle
from pagedattn import ModelShape, allocate

LENS = [1, 37, 600, 2048, 5, 300]
HEAD_SCALES = [0.0, 1e-3, 0.03, 1.0, 3.0, 1.0, 0.5, 2.0]


def _q(batch, hq, d, seed):
    """tests/test_gpu_int8_q_range.py's q: per-head magnitudes far apart."""
    q = seeded_q(batch, hq, d, seed).float()
    q = q * torch.tensor(HEAD_SCALES * (hq // len(HEAD_SCALES))).view(1, hq, 1)
    q[:, 5, :] *= 0.01
    q[:, 5, 3] = 2.5
    return q.to(torch.float16)


def _dense_int8(cache):
    """[B, H_kv, S, D] int8 values and [B, H_kv, S] scales (float64), gathered
    as the oracle gathers the dequantised rows."""
    bt = cache.block_table.long()
    lens = cache.seq_lens.long()
    s_max = int(lens.max())
    pos = torch.arange(s_max)
    phys = bt[:, (pos // cache.block_size).clamp(max=bt.shape[1] - 1)]
    off = (pos % cache.block_size).unsqueeze(0).expand_as(phys)
    x = cache.k_cache[phys, off].double().permute(0, 2, 1, 3)
    s = cache.k_scale[phys, off].double().permute(0, 2, 1)
    return x, s


def emulate(q, cache, round_k: bool, block_n: int = 64) -> torch.Tensor:
    """The reference kernel's arithmetic, unsplit: fp16(x*s) K when round_k
    (the reference), exact x*s otherwise; V always fp16(x*s); fp32 scores,
    fp16 P, fp32 accumulation, fp16 output."""
    b, hq, d = q.shape
    hkv = cache.shape.num_kv_heads
    g = hq // hkv
    _, v16 = oracle.gather_contiguous(cache)
    x, s = _dense_int8(cache)
    k = (x.float() * s.float()[..., None])  # fp32 product, as the reference forms it
    k = k.to(torch.float16).float() if round_k else (x * s[..., None]).float()
    v = v16.float()
    qk_scale = d ** -0.5 * math.log2(math.e)
    out = torch.empty((b, hq, d), dtype=torch.float16)
    for bi, t in enumerate(cache.seq_lens.tolist()):
        for h in range(hkv):
            qh = q[bi, h * g:(h + 1) * g].float()
            m = torch.full((g,), -math.inf)
            l = torch.zeros(g)
            acc = torch.zeros(g, d)
            for n0 in range(0, t, block_n):
                n1 = min(n0 + block_n, t)
                qk = (qh @ k[bi, h, n0:n1].T) * qk_scale
                m_new = torch.maximum(m, qk.max(dim=1).values)
                alpha = torch.exp2(m - m_new)
                p = torch.exp2(qk - m_new[:, None])
                l = l * alpha + p.sum(dim=1)
                acc = acc * alpha[:, None] + p.to(torch.float16).float() @ v[bi, h, n0:n1]
                m = m_new
            out[bi, h * g:(h + 1) * g] = (acc / l[:, None]).to(torch.float16)
    return out


CASES = [(sdt, d) for sdt in (torch.float16, torch.float32) for d in (32, 64, 128, 256)]


@pytest.mark.parametrize("sdt,d", CASES, ids=[f"s{str(c[0])[-2:]}-d{c[1]}" for c in CASES])
def test_reference_rounding_chain_meets_the_plain_bar(sdt, d):
    hq, hkv, seed = 16, 2, 5100 + d
    c = allocate(ModelShape(hq, hkv, d, name="qrange"), len(LENS), LENS, block_size=16,
                 kv_dtype="int8", seed=seed, scale_dtype=sdt, device="cpu")
    q = _q(len(LENS), hq, d, seed)
    want = oracle.reference_decode(q, c, out_dtype=torch.float32)
    ref_err = (emulate(q, c, round_k=True).float() - want).abs().max().item()
    exact_err = (emulate(q, c, round_k=False).float() - want).abs().max().item()
    print(f"d={d} scale={sdt}: reference chain {ref_err:.2e}, unrounded K {exact_err:.2e}")
    assert ref_err < 2e-3
    # the unrounded K is further from the oracle than the reference's chain
    assert exact_err >= ref_err


def test_unrounded_k_leaves_the_oracle_on_peaked_heads():
    """Over all cases, attending over the exact x * s misses the oracle by
    more than 1.5e-3 somewhere (the reference's chain never does), so a
    kernel that skipped K's fp16 rounding would need a wider bar."""
    worst_ref = worst_exact = 0.0
    for sdt, d in CASES:
        hq, hkv, seed = 16, 2, 5100 + d
        c = allocate(ModelShape(hq, hkv, d, name="qrange"), len(LENS), LENS, block_size=16,
                     kv_dtype="int8", seed=seed, scale_dtype=sdt, device="cpu")
        q = _q(len(LENS), hq, d, seed)
        want = oracle.reference_decode(q, c, out_dtype=torch.float32)
        worst_ref = max(worst_ref, (emulate(q, c, True).float() - want).abs().max().item())
        worst_exact = max(worst_exact, (emulate(q, c, False).float() - want).abs().max().item())
    print(f"worst: reference chain {worst_ref:.2e}, unrounded K {worst_exact:.2e}")
    assert worst_ref < 1.5e-3 < worst_exact
