"""Build the oracle's C helper (test infrastructure) into oracle/_build/.

    python oracle/build_oracle.py

The reference's own hot-path sources (AIE2 C++ against aie_api, IRON/MLIR-AIE
programs) cannot be compiled with gcc here, so there is no oracle/_ref build;
only this restatement's helper is compiled.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "_build" / "liblfm25_oracle.so"


def build(verbose: bool = False) -> Path:
    OUT.parent.mkdir(exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    cmd = ["gcc", "-O3", "-fopenmp", "-fPIC", "-shared", "-std=c11",
           str(HERE / "lfm25_oracle.c"), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"gcc failed with exit code {proc.returncode}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
