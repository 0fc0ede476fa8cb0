"""Build `pagedattn/libpagedattn_hip.so` from csrc/ with hipcc for gfx950.

Usage: python paged-decode-attention_amd/build.py   (or __graft_entry__.build())
The library is written in-tree next to the Python package that loads it.
"""

from __future__ import annotations

import os
import pathlib
import subprocess
import sys

PKG_ROOT = pathlib.Path(__file__).resolve().parent
REPO_ROOT = PKG_ROOT.parent
SOURCES = [PKG_ROOT / "csrc" / "paged_decode.hip", PKG_ROOT / "csrc" / "cache_write.hip"]
OUTPUT = PKG_ROOT / "pagedattn" / "libpagedattn_hip.so"
ARCH = os.environ.get("PAGEDATTN_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # packed-FP32 VALU forms are kept out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = pathlib.Path(rocm) / "bin" / "hipcc"
    return str(cand) if cand.exists() else "hipcc"


def build(verbose: bool = True) -> pathlib.Path:
    tmp = OUTPUT.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{REPO_ROOT / 'include'}", *map(str, SOURCES), "-o", str(tmp)]
    if verbose:
        print("[build]", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build())
