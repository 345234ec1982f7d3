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


# AddressSanitizer + UndefinedBehaviorSanitizer build (CPU checking of the C restatement, written
# to ``out``): every error aborts.  Loaded with gcc's libasan / libubsan preloaded
# (GEO_ORACLE_LIB selects it).
SANITIZE_FLAGS = ["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
                  "-fno-sanitize-recover=all"]


def build(sanitize: bool = False, out: Path | None = None) -> Path:
    lib = Path(out) if out is not None else LIB
    lib.parent.mkdir(parents=True, exist_ok=True)
    tmp = lib.with_suffix(".so.tmp")
    flags = [f for f in FLAGS if f != "-O2"] + SANITIZE_FLAGS if sanitize else FLAGS
    cmd = [CC, *flags, str(SRC), "-o", str(tmp), "-lm"]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed: {' '.join(cmd)}\n{proc.stdout}")
    os.replace(tmp, lib)
    return lib


def sanitizer_runtimes() -> list[str]:
    """gcc's ASan and UBSan runtimes, which must be preloaded into a process that loads the
    sanitizer build."""
    out = []
    for name in ("libasan.so", "libubsan.so"):
        p = subprocess.run([CC, f"-print-file-name={name}"], stdout=subprocess.PIPE, text=True)
        out.append(p.stdout.strip())
    return out


if __name__ == "__main__":
    print(build())
    sys.exit(0)
