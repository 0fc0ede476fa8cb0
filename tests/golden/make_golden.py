"""Write the golden fixtures tests/golden/*.npz with the float64 C oracle.

The reference ships no golden vectors (its tests compute a live fp32 oracle),
so these fixtures are this build's own: small seeded caches in the reference's
NHD layout with the float64 output of oracle/pa_oracle.c (and, for some, its
per-split partials). They freeze the oracle's behaviour so a later change to
either restatement shows up as a fixture mismatch.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import pathlib
import sys

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent.parent
for p in (str(ROOT / "paged-decode-attention_amd"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)

from oracle import c_oracle  # noqa: E402
from pagedattn import ModelShape, allocate  # noqa: E402

FIXTURES = [
    # name, (hq, hkv, d), lens, kv_dtype, block_size, scale dtype, sm_scale, splits
    ("qwen_fp16_g7", (14, 2, 64), [32, 192, 77], "fp16", 16, None, None, 3),
    ("llama_fp16_ragged", (32, 8, 128), [1, 65, 140], "fp16", 16, None, None, 4),
    ("llama_e5m2_page32", (32, 8, 128), [70, 33], "fp8_e5m2", 32, None, None, 2),
    ("g8_int8_fp16scale", (16, 2, 64), [129, 7], "int8", 16, torch.float16, None, None),
    ("g8_int8_fp32scale", (64, 8, 128), [50], "int8", 16, torch.float32, 0.05, 2),
    ("mha_d32_page64", (4, 4, 32), [70, 2], "fp16", 64, None, None, None),
]


def _raw(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous()
    if t.element_size() == 1:
        return t.view(torch.uint8).numpy().copy()
    if t.dtype == torch.float16:
        return t.view(torch.int16).numpy().copy()
    return t.numpy().copy()


def main() -> None:
    for i, (name, (hq, hkv, d), lens, kv, bs, sd, sm, splits) in enumerate(FIXTURES):
        shape = ModelShape(hq, hkv, d, name)
        c = allocate(shape, len(lens), lens, block_size=bs, kv_dtype=kv, device="cpu",
                     seed=500 + i, scale_dtype=sd or torch.float16, slack_blocks=3)
        g = torch.Generator().manual_seed(600 + i)
        q = torch.randn((len(lens), hq, d), dtype=torch.float16, generator=g)
        scale = d ** -0.5 if sm is None else sm
        out = c_oracle.decode(q, c, sm_scale=scale).numpy()
        fields = dict(
            heads=np.array([hq, hkv, d], dtype=np.int32),
            kv_dtype=np.array(kv),
            scale_dtype=np.array({None: "none", torch.float16: "fp16", torch.float32: "fp32"}[sd]),
            block_size=np.array(bs, dtype=np.int32),
            sm_scale=np.array(scale, dtype=np.float64),
            q=_raw(q),
            k_cache=_raw(c.k_cache),
            v_cache=_raw(c.v_cache),
            block_table=c.block_table.numpy().copy(),
            seq_lens=c.seq_lens.numpy().copy(),
            out=out,
        )
        if sd is not None:
            fields["k_scale"] = _raw(c.k_scale)
            fields["v_scale"] = _raw(c.v_scale)
        if splits:
            part, lse = c_oracle.split(q, c, splits, align=32, sm_scale=scale)
            fields.update(num_splits=np.array(splits, dtype=np.int32), part=part.numpy(), lse2=lse.numpy())
        np.savez_compressed(HERE / f"{name}.npz", **fields)
        print(f"wrote {name}.npz")


if __name__ == "__main__":
    main()
