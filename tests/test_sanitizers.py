"""CPU runs of the oracle's C restatement and of the HIP library's host-side code under
AddressSanitizer + UndefinedBehaviorSanitizer.

* ``oracle/geo_oracle.c`` is built with gcc's sanitizers (oracle/build.py, ``sanitize=True``) and
  the oracle's and golden-vector tests run against that build in a child process that preloads
  gcc's runtimes: every FPS / KNN / radius / CSR restatement call of those tests is checked for
  out-of-bounds accesses, use-after-free, signed overflow, misaligned loads, ...
* ``libgeoembodied_hip.so`` is built with the sanitizers on its host code only (the ABI entry
  points, argument validation, workspace carving and launch set-up; device code is compiled as
  usual) and the C-ABI tests run against it in a child process that preloads clang's ASan
  runtime (which carries the UBSan handlers).  Those tests call every entry point with invalid
  arguments and every workspace-size query, none of which reaches a GPU.

Both builds go to a temporary directory; nothing here touches a GPU.
"""

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
ROCM_CLANG_RT = Path("/opt/rocm/lib/llvm/lib/clang")


def _child_env(preload: list[str], **extra) -> dict:
    env = dict(os.environ)
    # the sanitizer runtime must come first among preloaded libraries; whatever the environment
    # already preloads stays behind it
    old = env.get("LD_PRELOAD")
    env["LD_PRELOAD"] = ":".join(preload + ([old] if old else []))
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    env["PYTHONPATH"] = str(ROOT) + os.pathsep + env.get("PYTHONPATH", "")
    env.update(extra)
    return env


def _pytest(env: dict, *files: str) -> subprocess.CompletedProcess:
    cmd = [sys.executable, "-m", "pytest", "-x", "-q", "-m", "not gpu", "-p", "no:cacheprovider",
           *files]
    return subprocess.run(cmd, cwd=ROOT, env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                          text=True, timeout=600)


def test_oracle_under_asan_ubsan(tmp_path):
    from oracle.build import build, sanitizer_runtimes
    lib = build(sanitize=True, out=tmp_path / "libgeo_oracle_asan.so")
    runtimes = sanitizer_runtimes()
    if not all(Path(r).is_file() for r in runtimes):
        pytest.skip(f"gcc sanitizer runtimes not found: {runtimes}")
    proc = _pytest(_child_env(runtimes, GEO_ORACLE_LIB=str(lib)), "tests/test_oracle.py",
                   "tests/test_golden.py")
    print(proc.stdout[-3000:])
    assert proc.returncode == 0, proc.stdout[-6000:]
    assert "passed" in proc.stdout and "ERROR: AddressSanitizer" not in proc.stdout


def test_hip_host_code_under_asan_ubsan(tmp_path):
    from gdl_amd.build import HIPCC, build
    if not Path(HIPCC).exists():
        pytest.skip("hipcc not available")
    runtimes = sorted(ROCM_CLANG_RT.glob("*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not runtimes:
        pytest.skip("clang ASan runtime not found")
    # host-side sanitizers only: each flag is passed to the host compilation alone
    host_only = ["-Xarch_host", "-fsanitize=address,undefined",
                 "-Xarch_host", "-fno-sanitize-recover=all",
                 "-Xarch_host", "-fno-omit-frame-pointer"]
    lib = build(extra_flags=host_only, out_dir=tmp_path / "hostsan")
    proc = _pytest(_child_env([str(runtimes[-1])], GEOEMBODIED_HIP_LIB=str(lib)),
                   "tests/test_abi.py")
    print(proc.stdout[-3000:])
    assert proc.returncode == 0, proc.stdout[-6000:]
    assert "passed" in proc.stdout and "ERROR: AddressSanitizer" not in proc.stdout
