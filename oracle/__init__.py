"""CPU oracle of the paged decode path -- TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
never by the product package (paged-decode-attention_amd/), which has no CPU
path. Two independent restatements of the reference's algorithm live here:

  reference.py  torch fp32, gather-then-attend, as pagedattn/reference.py does
  pa_oracle.c   float64 C, walks the block table page by page (c_oracle.py
                binds it); used to pin reference.py
"""

from __future__ import annotations

import pathlib
import subprocess

ORACLE_DIR = pathlib.Path(__file__).resolve().parent
C_SOURCE = ORACLE_DIR / "pa_oracle.c"
C_LIBRARY = ORACLE_DIR / "libpa_oracle.so"


def build_c_oracle(verbose: bool = True) -> pathlib.Path:
    """Compile pa_oracle.c with gcc into oracle/libpa_oracle.so."""
    tmp = C_LIBRARY.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", str(C_SOURCE), "-o", str(tmp), "-lm"]
    if verbose:
        print("[build]", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed ({res.returncode}):\n{res.stderr}")
    tmp.replace(C_LIBRARY)
    return C_LIBRARY
