"""Build recipe for libgeoembodied_hip.so (gfx950 only).

Compiles every ``gdl_amd/csrc/*.hip`` translation unit with hipcc and links them into
``gdl_amd/lib/libgeoembodied_hip.so``.  Flags:

* ``--offload-arch=gfx950``: MI355X (CDNA4, wave64) is the only target.
* ``-ffp-contract=off``: the geometry kernels must not fuse multiply-adds, because distances
  have to round exactly like the reference's ``(dx*dx + dy*dy) + dz*dz``.
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed fp32 instructions.

Usage: ``python -m gdl_amd.build`` (or ``gdl_amd.build.build()``).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
BUILDDIR = PKG / "_build"
LIBNAME = "libgeoembodied_hip.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

DEVICE_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


# Per-file device flags.  fps.hip: the sampling loops end every iteration with one lane's LDS
# atomic max; the atomic optimizer would wrap it in a single-lane election (mbcnt, compare, exec
# mask) that lengthens the path to the barrier in every wave, every iteration.
FILE_FLAGS = {
    "fps.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}


def lib_path() -> Path:
    return LIBDIR / LIBNAME


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops" not in line and "unused during compilation: '--hip-link'" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(verbose: bool = False, extra_flags: list[str] | None = None,
          out_dir: Path | None = None) -> Path:
    """Compile all HIP sources and link the shared library; returns its path.  ``extra_flags``
    are appended to every compile and link line; with ``out_dir`` the objects and the library
    go there instead of ``_build/`` and ``lib/`` (a checking build beside the one that ships)."""
    if not Path(HIPCC).exists() and shutil.which(HIPCC) is None:
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    extra = list(extra_flags or [])
    builddir = BUILDDIR if out_dir is None else Path(out_dir)
    out = lib_path() if out_dir is None else Path(out_dir) / LIBNAME
    builddir.mkdir(parents=True, exist_ok=True)
    out.parent.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    flags_str = " ".join(DEVICE_FLAGS)
    define = f"-DGEO_BUILD_FLAGS=\"{flags_str}\""

    def compile_one(src: Path) -> Path:
        obj = builddir / (src.stem + ".o")
        cmd = [HIPCC, *DEVICE_FLAGS, *FILE_FLAGS.get(src.name, []), *extra, define, "-c", str(src),
               "-o", str(obj)]
        if verbose:
            print(" ".join(cmd))
        _run(cmd)
        return obj

    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=max(1, workers)) as pool:
        objs = list(pool.map(compile_one, sources))
    tmp = out.with_name(out.name + ".tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *extra, *map(str, objs), "-o",
          str(tmp)])
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
