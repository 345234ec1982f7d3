"""GPU: spherical harmonics, the fused spatial-graph edge epilogue and SpatialGraph against the
float64 oracle (pinned by quadrature and closed forms in test_oracle.py).

Bars: fp32 values within 2e-6 absolute (directions and SH of unit vectors are O(1); the kernel
rounds each operation once) and distances within 1e-6 relative; topology, CSR arrays and average
degrees exact; gradients with respect to positions within 1e-4 relative of float64 autograd of
the reference's op sequence (fp32 chains through a normalisation).
"""

import numpy as np
import pytest
import torch

import oracle
from sh_torch import sh_torch as _sh_torch

pytestmark = pytest.mark.gpu


def _f():
    import geoembodied  # noqa: F401
    from geoembodied.kernels.triton_sph_harm import spherical_harmonics
    from geoembodied.nn.modules.spatial_graph import SpatialGraph
    return spherical_harmonics, SpatialGraph


@pytest.mark.parametrize("max_l", [0, 1, 2])
@pytest.mark.parametrize("normalize", [False, True])
def test_spherical_harmonics_vs_oracle_and_grad(dev, max_l, normalize):
    sh, _ = _f()
    g = torch.Generator().manual_seed(max_l * 2 + normalize)
    v = torch.randn(5000, 3, generator=g)
    if not normalize:
        v = v / v.norm(dim=1, keepdim=True)
    v[0] = 0.0                                             # zero vector (normalised: clamp)
    vd = v.to(dev).requires_grad_(True)
    Y = sh(vd, max_l=max_l, normalize=normalize)
    assert Y.shape == (5000, (max_l + 1) ** 2)
    np.testing.assert_allclose(Y.detach().cpu().numpy(), oracle.spherical_harmonics(v.numpy(), max_l, normalize),
                               atol=2e-6, rtol=0)
    gY = torch.randn(5000, (max_l + 1) ** 2, generator=g)
    Y.backward(gY.to(dev))
    v64 = v.double().requires_grad_(True)
    u = v64 / v64.norm(dim=-1, keepdim=True).clamp(min=1e-8) if normalize else v64
    if max_l == 0:                                         # Y_0^0 is constant
        want = np.zeros((5000, 3))
    else:
        _sh_torch(u, max_l).backward(gY.double())
        want = v64.grad.numpy()
    got = vd.grad.cpu().numpy()
    ok = np.abs(v.numpy()).sum(1) > 0
    np.testing.assert_allclose(got[ok], want[ok], rtol=1e-4, atol=1e-5)


def _cloud(N, B, seed):
    g = torch.Generator().manual_seed(seed)
    d = torch.randn(N * B, 3, generator=g)
    pos = d / d.norm(dim=1, keepdim=True) + 0.01 * torch.randn(N * B, 3, generator=g)
    return pos, torch.arange(B).repeat_interleave(N)


@pytest.mark.parametrize("B,N,r,K", [(1, 500, 0.3, 16), (4, 1000, 0.15, 32), (16, 4096, 0.1, 32)])
def test_spatial_graph_build_vs_oracle(dev, B, N, r, K):
    _, SpatialGraph = _f()
    pos, batch = _cloud(N, B, N + B)
    graph = SpatialGraph.build(pos.to(dev), r, max_num_neighbors=K, batch=batch.to(dev),
                               num_batch_elements=B)
    wr, wc = oracle.radius_graph(pos.numpy(), r, K, batch=batch.numpy(), num_batch_elements=B)
    np.testing.assert_array_equal(graph.row.cpu().numpy(), wr)
    np.testing.assert_array_equal(graph.col.cpu().numpy(), wc)
    assert graph.E == len(wr) and graph.N == N * B
    cs, pm, ns, ne = oracle.sort_and_build_csr(wc, N * B)
    for got, want in ((graph.col_sorted, cs), (graph.perm, pm), (graph.node_start, ns), (graph.node_end, ne)):
        assert got.dtype == torch.int32
        np.testing.assert_array_equal(got.cpu().numpy(), want)
    d, dist, Y = oracle.edge_geometry(pos.numpy(), wr, wc)
    np.testing.assert_allclose(graph.direction.cpu().numpy(), d, atol=2e-6, rtol=0)
    np.testing.assert_allclose(graph.dist.cpu().numpy(), dist, rtol=1e-6)
    np.testing.assert_allclose(graph.Y.cpu().numpy(), Y, atol=2e-6, rtol=0)
    np.testing.assert_allclose(graph.avg_degree.cpu().numpy(),
                               oracle.graph_avg_degree(ns, ne, batch.numpy(), B), rtol=1e-7)


@pytest.mark.parametrize("layout", ["batch_chunks", "num_batch_elements", "one_cloud", "mask"])
def test_spatial_graph_device_epilogue_matches_exact_sized(dev, layout):
    """SpatialGraph.build without gradients computes its fields on the device behind the radius
    graph's emit pass (bound-sized buffers, views of the first E rows); with gradients it takes
    the exact-sized path after the edge count.  Both must agree bit for bit, for every layout of
    contiguous equal clouds."""
    _, SpatialGraph = _f()
    B = 1 if layout == "one_cloud" else 4
    pos, batch = _cloud(1500, B, 77 + B)
    kw = dict(max_num_neighbors=24)
    if layout == "batch_chunks":
        kw.update(batch=batch.to(dev), num_batch_elements=B)
    elif layout in ("num_batch_elements", "mask"):
        kw.update(num_batch_elements=B)
    if layout == "mask":
        m = torch.ones(pos.shape[0], dtype=torch.bool)
        m[::7] = False
        kw.update(mask=m.to(dev))
    with torch.no_grad():
        fast = SpatialGraph.build(pos.to(dev), 0.12, **kw)
    with torch.enable_grad():
        exact = SpatialGraph.build(pos.to(dev).requires_grad_(True), 0.12, **kw)
    assert fast.E == exact.E > 0
    for name in ("row", "col", "direction", "dist", "Y", "col_sorted", "perm", "node_start",
                 "node_end", "avg_degree"):
        a, b = getattr(fast, name), getattr(exact, name).detach()
        assert a.shape == b.shape and torch.equal(a, b), name


def test_spatial_graph_shuffled_batch_takes_exact_path(dev):
    """A batch vector whose clouds are not contiguous chunks: the device epilogue is skipped (its
    degree formula assumes chunks) and the fields still match the oracle."""
    _, SpatialGraph = _f()
    pos, batch = _cloud(800, 3, 5)
    sh = torch.randperm(pos.shape[0], generator=torch.Generator().manual_seed(1))
    pos, batch = pos[sh], batch[sh]
    graph = SpatialGraph.build(pos.to(dev), 0.2, max_num_neighbors=16, batch=batch.to(dev),
                               num_batch_elements=3)
    wr, wc = oracle.radius_graph(pos.numpy(), 0.2, 16, batch=batch.numpy(), num_batch_elements=3)
    np.testing.assert_array_equal(graph.col.cpu().numpy(), wc)
    cs, pm, ns, ne = oracle.sort_and_build_csr(wc, pos.shape[0])
    np.testing.assert_array_equal(graph.node_start.cpu().numpy(), ns)
    np.testing.assert_allclose(graph.avg_degree.cpu().numpy(),
                               oracle.graph_avg_degree(ns, ne, batch.numpy(), 3), rtol=1e-7)


def _avg_degree_np(row_ptr, batch, B):
    deg = np.diff(row_ptr).astype(np.float64)
    valid = (batch >= 0) & (batch < B)
    s = np.bincount(batch[valid], weights=deg[valid], minlength=B)
    c = np.bincount(batch[valid], minlength=B)
    avg = np.ones(len(deg), np.float32)
    a = (s[batch[valid]] / np.maximum(c[batch[valid]], 1)).astype(np.float32)
    avg[valid] = np.maximum(a, 1.0)
    return avg


@pytest.mark.parametrize("N,B,kind", [
    (10001, 3, "sorted"),      # uneven contiguous clouds, boundaries inside threads and waves
    (9000, 7, "unsorted"),     # every wave mixes clouds
    (5000, 4, "invalid"),      # ids outside [0, B) contribute nothing and get 1
    (16384, 4, "ppc"),         # no batch vector: equal contiguous clouds
    (3, 2, "sorted"),
])
def test_graph_avg_degree_vs_numpy(dev, N, B, kind):
    from gdl_amd.csrc import graph_avg_degree_hip
    rng = np.random.default_rng(N + B)
    deg = rng.integers(0, 40, N)
    row_ptr = np.zeros(N + 1, np.int64)
    row_ptr[1:] = np.cumsum(deg)
    if kind == "sorted":
        batch = np.sort(rng.integers(0, B, N))
    elif kind == "unsorted":
        batch = rng.integers(0, B, N)
    elif kind == "invalid":
        batch = rng.integers(-1, B + 1, N)
    else:
        batch = np.repeat(np.arange(B), N // B)
    got = graph_avg_degree_hip(torch.from_numpy(row_ptr).to(dev), N,
                               None if kind == "ppc" else torch.from_numpy(batch).to(dev), B)
    np.testing.assert_allclose(got.cpu().numpy(), _avg_degree_np(row_ptr, batch, B), rtol=1e-7)


def test_spatial_graph_gradient_and_from_edge_index(dev):
    _, SpatialGraph = _f()
    pos, batch = _cloud(600, 2, 9)
    p = pos.to(dev).requires_grad_(True)
    graph = SpatialGraph.build(p, 0.25, max_num_neighbors=24, batch=batch.to(dev), num_batch_elements=2)
    g = torch.Generator().manual_seed(1)
    w_dir = torch.randn(graph.E, 3, generator=g)
    w_dist = torch.randn(graph.E, generator=g)
    w_Y = torch.randn(graph.E, 9, generator=g)
    loss = (graph.direction * w_dir.to(dev)).sum() + (graph.dist * w_dist.to(dev)).sum() + \
        (graph.Y * w_Y.to(dev)).sum()
    loss.backward()
    p64 = pos.double().requires_grad_(True)
    row, col = graph.row.cpu(), graph.col.cpu()
    diff = p64[col] - p64[row]
    dist = diff.norm(dim=-1, keepdim=True).clamp(min=1e-8)
    direction = diff / dist
    ref = (direction * w_dir.double()).sum() + (dist.squeeze(-1) * w_dist.double()).sum() + \
        (_sh_torch(direction, 2) * w_Y.double()).sum()
    ref.backward()
    np.testing.assert_allclose(p.grad.cpu().numpy(), p64.grad.numpy(), rtol=1e-4, atol=2e-4)
    # the same edges given in shuffled order: identical per-edge geometry and the stable CSR
    sh = torch.randperm(graph.E, generator=g)
    g2 = SpatialGraph.from_edge_index(graph.row[sh.to(dev)], graph.col[sh.to(dev)], pos.to(dev),
                                      graph.N, batch=batch.to(dev), num_batch_elements=2)
    np.testing.assert_array_equal(g2.direction.cpu().numpy(), graph.direction[sh.to(dev)].detach().cpu().numpy())
    np.testing.assert_array_equal(g2.Y.cpu().numpy(), graph.Y[sh.to(dev)].detach().cpu().numpy())
    cs, pm, ns, ne = oracle.sort_and_build_csr(graph.col[sh.to(dev)].cpu().numpy(), graph.N)
    np.testing.assert_array_equal(g2.perm.cpu().numpy(), pm)
    np.testing.assert_array_equal(g2.avg_degree.cpu().numpy(), graph.avg_degree.cpu().numpy())


def test_spatial_graph_empty_and_device_radius(dev):
    _, SpatialGraph = _f()
    pos = torch.randn(100, 3, device=dev) * 100
    g0 = SpatialGraph.build(pos, 1e-3)
    assert g0.E == 0 and g0.Y.shape == (0, 9) and (g0.avg_degree == 1).all()
    from geoembodied.functional.adaptive import adaptive_radius
    p2, _ = _cloud(800, 1, 3)
    r = adaptive_radius(p2.to(dev), torch.tensor([0, 800], device=dev), 3.0)
    ga = SpatialGraph.build(p2.to(dev), r, max_num_neighbors=16)
    gb = SpatialGraph.build(p2.to(dev), float(r), max_num_neighbors=16)
    assert torch.equal(ga.row, gb.row) and torch.equal(ga.Y, gb.Y)
