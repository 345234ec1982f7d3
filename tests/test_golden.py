"""Golden fixtures (tests/golden/*.json, written by tests/golden/make_fixtures.py from closed
forms and exact integer brute force): the oracle (CPU) and the HIP library (GPU) must reproduce
every expected value bit for bit."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def fx(name):
    return json.loads((GOLDEN / f"{name}.json").read_text())


def f32(a):
    return np.asarray(a, dtype=np.float32).reshape(-1, 3) if a else np.zeros((0, 3), np.float32)


# ------------------------------------------------------------------------------ oracle ---

@pytest.mark.parametrize("name", ["fps_line", "fps_lattice"])
def test_oracle_fps_golden(name):
    f = fx(name)
    assert oracle.fps(f32(f["pos"]), f["ptr"], f["k"]).tolist() == f["want"]


def test_oracle_knn_golden():
    f = fx("knn_lattice")
    idx, dist = oracle.knn(f32(f["query"]), f32(f["source"]), f["ptr_q"], f["ptr_s"], f["k"])
    assert idx.tolist() == f["want_idx"]
    np.testing.assert_array_equal(dist, np.asarray(f["want_dist"], np.float32))


@pytest.mark.parametrize("name", ["radius_lattice", "radius_kat_three_points", "radius_kat_batches"])
def test_oracle_radius_golden(name):
    f = fx(name)
    row, col = oracle.radius_graph(f32(f["x"]), f["r"], f["K"], loop=f["loop"], batch=f.get("batch"))
    assert row.tolist() == f["want_row"] and col.tolist() == f["want_col"]


def test_oracle_csr_golden():
    f = fx("csr")
    cs, pm, ns, ne = oracle.sort_and_build_csr(np.asarray(f["col"], np.int64), f["N"])
    assert cs.tolist() == f["col_sorted"] and pm.tolist() == f["perm"]
    assert ns.tolist() == f["start"] and ne.tolist() == f["end"]


@pytest.mark.parametrize("name", ["segment_sum", "segment_mean", "segment_max", "segment_sum_all_to_one"])
def test_oracle_segment_golden(name):
    f = fx(name)
    out, aux = oracle.segment_reduce_fwd(np.asarray(f["msg"], np.float32), f["perm"], f["start"],
                                         f["end"], len(f["start"]), f["reduce"])
    np.testing.assert_array_equal(out, np.asarray(f["want"], np.float64))
    if f["reduce"] == "max":
        assert aux.tolist() == f["want_arg"]


# --------------------------------------------------------------------------------- GPU ---

@pytest.mark.gpu
def test_gpu_golden(dev):
    import geoembodied  # noqa: F401
    from gdl_amd.csrc import fps_cuda, segment_reduce_forward_hip
    from geoembodied.functional.knn import knn
    from geoembodied.functional.radius_graph import radius_graph
    from geoembodied.functional.segment_reduce import sort_and_build_csr

    def t(a, dt=torch.float32):
        return torch.as_tensor(np.asarray(a), dtype=dt, device=dev)

    for name in ("fps_line", "fps_lattice"):
        f = fx(name)
        got = fps_cuda(t(f32(f["pos"])), t(f["ptr"], torch.int64), t(f["k"], torch.int64))
        assert got.cpu().tolist() == f["want"], name
    f = fx("knn_lattice")
    idx, dist = knn(t(f32(f["query"])), t(f32(f["source"])), t(f["ptr_q"], torch.int64),
                    t(f["ptr_s"], torch.int64), f["k"])
    assert idx.cpu().tolist() == f["want_idx"]
    np.testing.assert_array_equal(dist.cpu().numpy(), np.asarray(f["want_dist"], np.float32))
    for name in ("radius_lattice", "radius_kat_three_points", "radius_kat_batches"):
        f = fx(name)
        batch = t(f["batch"], torch.int64) if "batch" in f else None
        row, col = radius_graph(t(f32(f["x"])), f["r"], batch=batch, loop=f["loop"],
                                max_num_neighbors=f["K"])
        assert row.cpu().tolist() == f["want_row"] and col.cpu().tolist() == f["want_col"], name
    f = fx("csr")
    cs, pm, ns, ne = sort_and_build_csr(t(f["col"], torch.int64), f["N"])
    assert cs.cpu().tolist() == f["col_sorted"] and pm.cpu().tolist() == f["perm"]
    assert ns.cpu().tolist() == f["start"] and ne.cpu().tolist() == f["end"]
    for name in ("segment_sum", "segment_mean", "segment_max", "segment_sum_all_to_one"):
        f = fx(name)
        out, arg = segment_reduce_forward_hip(t(f["msg"]), t(f["perm"], torch.int32),
                                              t(f["start"], torch.int32), t(f["end"], torch.int32),
                                              len(f["start"]), f["reduce"])
        np.testing.assert_array_equal(out.cpu().numpy(), np.asarray(f["want"], np.float32), err_msg=name)
        if f["reduce"] == "max":
            assert arg.cpu().tolist() == f["want_arg"]
