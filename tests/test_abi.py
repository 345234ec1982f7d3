"""CPU tests of the C ABI: the library loads, exports every entry point declared in
include/geo_api.h, and rejects bad arguments with a status code and message before touching a
GPU (no compute calls here)."""

import ctypes
import re
from pathlib import Path

import pytest

from gdl_amd import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "geo_api.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(geo_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = _declared()
    assert names == sorted(_native.EXPORTED), names


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    for name in _declared():
        assert hasattr(lib, name), name


def test_build_info_and_version():
    info = _native.build_info()
    assert "gfx950" in info and "-ffp-contract=off" in info
    assert _native.lib().geo_abi_version() == 2


def test_workspace_sizes():
    L = _native.lib()
    # the radix sort's intermediate keys and values (three passes at 19-bit keys)
    assert L.geo_csr_workspace_bytes(4_194_304, 262_144) >= 2 * 4 * 4_194_304
    assert L.geo_radius_workspace_bytes(65_536, 16, 32) >= 65_536 * 32 * 4
    assert L.geo_knn_workspace_bytes(16384, 65536, 16, 16) >= 17 * 8
    assert L.geo_fps_workspace_bytes(1, 131072, 131072) >= 131072 * 4
    assert L.geo_fps_workspace_bytes(16, 65536, 4096) == 0
    assert L.geo_csr_workspace_bytes(-1, 5) == 0


def test_se3_fused_tile_size_rule():
    """The fused SE3 forward runs when 16 nodes' aggregate rows (K + 4 floats each; 1 / 3 / 5 rows
    per node for the present output kinds) fit 64 KiB of LDS; larger layers take the two-kernel
    path (geo_se3_aggregate_fwd + geo_se3_gemm)."""
    L = _native.lib()
    assert L.geo_se3_fwd_fused_lds_bytes(64, 16, 0, 80, 96, 96) == 4 * 16 * (84 + 3 * 100)
    assert L.geo_se3_fwd_fused_lds_bytes(70, 10, 4, 112, 128, 112) == 0      # 69,888 bytes
    assert L.geo_se3_fwd_fused_lds_bytes(0, 16, 0, 80, 96, 96) == 4 * 16 * 3 * 100
    assert L.geo_se3_fwd_fused_lds_bytes(-1, 16, 0, 80, 96, 96) == 0


def _err(rc, fragment):
    assert rc != 0
    assert fragment in _native.last_error(), _native.last_error()


def test_invalid_arguments_are_rejected_before_any_launch():
    L = _native.lib()
    nul = None
    _err(L.geo_segment_reduce_fwd(7, 0, nul, nul, nul, nul, 0, 1, 1, nul, nul, 0, nul), "reduce")
    _err(L.geo_segment_reduce_fwd(0, 9, nul, nul, nul, nul, 0, 1, 1, nul, nul, 0, nul), "dtype")
    _err(L.geo_segment_reduce_fwd(0, 0, nul, nul, nul, nul, -1, 1, 1, nul, nul, 0, nul), "negative")
    _err(L.geo_segment_reduce_fwd(2, 0, 8, nul, 8, 8, 1, 1, 4, 8, nul, 0, nul), "arg")
    _err(L.geo_segment_reduce_bwd(2, 0, 8, nul, nul, nul, 8, nul, nul, nul, 1, 1, 1, 8, nul), "max needs")
    _err(L.geo_knn(nul, 1, nul, 1, nul, nul, 1, -1, nul, nul, nul, 0, nul), "k must")
    _err(L.geo_knn(nul, 1, nul, 1, nul, nul, 1, 1000, nul, nul, nul, 0, nul), "null")
    _err(L.geo_radius_count(nul, 10, nul, 0, 10, nul, 0.01, 0.1, 32, 0, nul, nul, 0, nul), "B >= 1")
    _err(L.geo_radius_count(nul, 10, nul, 3, 3, nul, 0.01, 0.1, 32, 0, nul, nul, 0, nul), "points_per_cloud")
    _err(L.geo_radius_count(nul, 10, nul, 1, 10, nul, 0.01, 0.1, 0, 0, nul, nul, 0, nul), "max_num_neighbors")
    _err(L.geo_csr_build(nul, -1, 5, nul, nul, nul, nul, nul, 0, nul), "negative")
    _err(L.geo_fps(nul, 10, nul, nul, 1, 11, nul, nul, 0, nul), "max_cloud")
    # the no-allocation CSR build refuses more edges than its fixed scratch holds
    _err(L.geo_csr_build_noalloc(8, (1 << 20) + 1, 4, 8, 8, 8, 8, nul), "exceed")
    _err(L.geo_csr_build_noalloc(nul, 10, 4, 8, 8, 8, 8, nul), "null edge")
    # fused SE3 forward: row length not a multiple of 16, weights without enough rows, and a
    # tile beyond 64 KiB of LDS
    pc = (ctypes.c_int32 * 9)(*([-1] * 9))

    def fused(Os, Ks, Ws_rows, W=16):
        return L.geo_se3_fwd_fused(nul, nul, nul, 10, 0, 0, 0, nul, nul, nul, nul, 0, nul, nul, 1,
                                   nul, 1, pc, nul, W, Ws_rows, nul, 0, nul, 0, Os, 0, 0, Ks, 16, 16,
                                   nul, nul, nul, 8, nul, nul, nul, nul, nul, nul)
    _err(fused(4, 20, 16), "multiple of 16")
    _err(fused(20, 16, 16), "rows, need 32")
    _err(fused(4, 16, 16, W=4), "16-byte aligned")
    _err(fused(4, 1024, 16), "exceeds")


def test_workspace_too_small_is_reported():
    L = _native.lib()
    rc = L.geo_csr_build(8, 100, 10, 8, 8, 8, 8, None, 0, None)
    assert rc == 3 and "workspace" in _native.last_error()
    rc = L.geo_radius_count(8, 100, None, 1, 100, None, 0.01, 0.1, 32, 0, 8, None, 0, None)
    assert rc == 3 and "workspace" in _native.last_error()


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    import importlib
    monkeypatch.setenv("GEOEMBODIED_HIP_LIB", str(tmp_path / "nope.so"))
    fresh = importlib.reload(_native)
    try:
        assert not fresh.loaded()
        with pytest.raises(RuntimeError, match="nope.so"):
            fresh.lib()
    finally:
        monkeypatch.delenv("GEOEMBODIED_HIP_LIB")
        importlib.reload(_native)
