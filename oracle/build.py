"""Build recipe for the oracle's C restatement (test infrastructure only).

``python -m oracle.build`` compiles ``oracle/geo_oracle.c`` into ``oracle/lib/libgeo_oracle.so``
with gcc.  ``-ffp-contract=off`` and ``-fno-fast-math`` keep every float operation a single
IEEE fp32 operation, so the restated distances round like the reference's; ``-fopenmp`` runs
independent queries / targets on several threads.

The reference implementation itself cannot be built here: its kernels are CUDA sources that need
nvcc, CUB and ATen (geoembodied/csrc/*.cu), none of which exist in this image, so there is no
``oracle/_ref`` build.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "geo_oracle.c"
LIB = HERE / "lib" / "libgeo_oracle.so"
CC = os.environ.get("CC", "gcc")
FLAGS = ["-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-fopenmp",
         "-Wall", "-Wextra", "-Wno-unused-parameter"]


def build() -> Path:
    LIB.parent.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [CC, *FLAGS, str(SRC), "-o", str(tmp), "-lm"]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed: {' '.join(cmd)}\n{proc.stdout}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
    sys.exit(0)
