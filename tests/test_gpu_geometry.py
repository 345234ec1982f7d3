"""GPU parity: FPS, KNN and radius graph vs the oracle — bit-exact indices, distances and edge
sets (ties toward the lower index) — at small sizes, on tie-heavy integer lattices and on the
five BASELINE configurations.  Also restates the reference's own tests
(tests/test_fps_cuda_remote.py:63-202, tests/test_radius_graph_cuda.py:69-232,
tests/test_phase1.py:258-298).
"""

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _f():
    import geoembodied  # noqa: F401
    from geoembodied.functional import fps, knn, radius_graph
    return fps.farthest_point_sampling, knn.knn, knn.knn_self, radius_graph.radius_graph


def _lattice(n_side, seed=0, jitter=False):
    g = np.stack(np.meshgrid(*[np.arange(n_side)] * 3, indexing="ij"), -1).reshape(-1, 3)
    rng = np.random.default_rng(seed)
    g = g[rng.permutation(len(g))].astype(np.float32)
    return torch.from_numpy(g)


def _ptr(sizes):
    p = np.zeros(len(sizes) + 1, dtype=np.int64)
    p[1:] = np.cumsum(sizes)
    return torch.from_numpy(p)


# ----------------------------------------------------------------------------------- FPS ---

def _fps_check(dev, pos, ptr, k):
    from gdl_amd.csrc import fps_cuda
    got = fps_cuda(pos.to(dev), ptr.to(dev), k.to(dev)).cpu().numpy()
    want = oracle.fps(pos.numpy(), ptr.numpy(), k.numpy())
    np.testing.assert_array_equal(got, want)
    return got


@pytest.mark.parametrize("sizes,ks,seed", [
    ([100], [10], 0), ([60, 40], [15, 10], 1), ([1000, 1000], [250, 250], 42),
    ([2048, 1024, 4096, 512], [512, 256, 1024, 128], 3), ([1, 2, 3, 300], [1, 2, 5, 0], 4),
    ([257, 511, 1025, 3000], [257, 100, 1024, 2999], 5), ([9000], [300], 6),
    ([16384, 100], [500, 50], 7), ([20000, 5000], [200, 100], 8),
])
def test_fps_vs_oracle(dev, sizes, ks, seed):
    g = torch.Generator().manual_seed(seed)
    pos = torch.randn(sum(sizes), 3, generator=g)
    _fps_check(dev, pos, _ptr(sizes), torch.tensor(ks))


def test_fps_large_clouds(dev):
    """Clouds above 16384 points take the Hilbert-bucket path with points in the workspace:
    several clouds, empty and tiny clouds, points outside every cloud, k = n and k = 0."""
    g = torch.Generator().manual_seed(11)
    pos = torch.randn(47100, 3, generator=g) * torch.tensor([30.0, 5.0, 1.0])
    ptr = torch.tensor([50, 50, 30050, 30060, 47000])  # first 50 / last 100 points in no cloud
    _fps_check(dev, pos, ptr, torch.tensor([5, 1000, 10, 500]))
    _fps_check(dev, pos, ptr, torch.tensor([0, 20, 10, 16940]))     # k = 0 and k = n
    _fps_check(dev, pos[:20000], _ptr([20000]), torch.tensor([4000]))


@pytest.mark.parametrize("n,k", [(8192, 300), (8193, 300), (16384, 300), (16385, 300),
                                 (196608, 48), (196609, 48)])
def test_fps_kernel_boundaries(dev, n, k):
    """One cloud at each kernel-selection boundary: the bucketed kernel's largest cloud (8192),
    the register kernel's smallest and largest (8193, 16384), the large kernel's smallest and its
    full capacity (16385; 196,608 = 3 slots x 1024 lanes x 64 points), and the streaming kernel
    above it (196,609)."""
    g = torch.Generator().manual_seed(n)
    pos = torch.randn(n, 3, generator=g) * torch.tensor([4.0, 2.0, 1.0])
    _fps_check(dev, pos, _ptr([n]), torch.tensor([k]))


def test_fps_large_tie_lattice(dev):
    pos = _lattice(30, 3)  # 27,000 integer points: exact distances, ties at every step
    _fps_check(dev, pos, _ptr([27000]), torch.tensor([3000]))


def test_fps_duplicate_points(dev):
    """Exact duplicates: once every distinct location is taken, every remaining point has min
    distance 0 and the lowest index among them must be taken next.  This drives the bucket
    records through ties at equal maxima (the point holding a bucket's maximum falls while an
    equal value at a higher index stays), in the bucketed kernel (4096 points) and the
    Hilbert-bucket kernel for large clouds (24,576 points)."""
    g = torch.Generator().manual_seed(21)
    base = torch.randn(1024, 3, generator=g)
    pos = base[torch.randint(0, 1024, (4096,), generator=g)]
    _fps_check(dev, pos, _ptr([4096]), torch.tensor([1500]))
    big = torch.randn(3000, 3, generator=g)
    pos2 = big[torch.randint(0, 3000, (24576,), generator=g)]
    _fps_check(dev, pos2, _ptr([24576]), torch.tensor([4000]))


def test_fps_tie_lattice(dev):
    pos = _lattice(8)  # 512 integer points: exact distances, many ties
    _fps_check(dev, pos, _ptr([512]), torch.tensor([200]))
    pos2 = torch.cat([_lattice(6, 1), _lattice(7, 2)])
    _fps_check(dev, pos2, _ptr([216, 343]), torch.tensor([216, 100]))


def test_fps_reference_kat(dev):
    """tests/test_fps_cuda_remote.py:63-90: 25 int64 indices, batch isolation, no duplicates."""
    from gdl_amd.csrc import fps_cuda
    pos = torch.randn(100, 3, device=dev)
    idx = fps_cuda(pos, torch.tensor([0, 60, 100], device=dev), torch.tensor([15, 10], device=dev))
    assert idx.shape == (25,) and idx.dtype == torch.int64 and idx.is_cuda
    assert (idx[:15] < 60).all() and (idx[15:] >= 60).all()
    assert idx.unique().numel() == 25


def test_fps_spread_beats_random(dev):
    """tests/test_fps_cuda_remote.py:141-167."""
    fps, *_ = _f()
    torch.manual_seed(0)
    pos = torch.randn(4096, 3, device=dev)
    sel = pos[fps(pos, 256)]
    rnd = np.mean([torch.cdist(p, p).mean().item()
                   for p in (pos[torch.randperm(4096, device=dev)[:256]] for _ in range(10))])
    assert torch.cdist(sel, sel).mean().item() > rnd


def test_fps_api_variants(dev):
    fps, *_ = _f()
    g = torch.Generator().manual_seed(9)
    pos = torch.randn(300, 3, generator=g)
    d = pos.to(dev)
    assert torch.equal(fps(d, 500).cpu(), torch.arange(300))
    np.testing.assert_array_equal(fps(d, 40).cpu().numpy(), oracle.fps(pos.numpy(), [0, 300], [40]))
    ptr = torch.tensor([0, 100, 300])
    np.testing.assert_array_equal(fps(d, 30, ptr=ptr.to(dev)).cpu().numpy(),
                                  oracle.fps(pos.numpy(), ptr.numpy(), [30, 30]))
    # legacy batch vector, clouds interleaved: cloud b is the points with batch == b in order
    batch = torch.from_numpy(np.random.default_rng(0).integers(0, 3, 300))
    got = fps(d, 25, batch=batch.to(dev)).cpu().numpy()
    want = []
    for b in range(3):
        members = np.nonzero(batch.numpy() == b)[0]
        loc = oracle.fps(pos.numpy()[members], [0, len(members)], [min(25, len(members))])
        want.append(members[loc])
    np.testing.assert_array_equal(got, np.concatenate(want))


@pytest.mark.parametrize("sizes,k", [
    ([4096] * 4, 1024),                 # every cloud the average size: the early launch is right
    ([100, 3000], 700),                 # average 1550 -> 2048-point variant; 3000 needs the next
    ([5000, 20, 0, 7], 9),              # empty and tiny clouds, k >= n for some
    ([9000, 100], 64),                  # average above 8192 points: no early launch
    ([12000, 3000, 3000], 100),         # average in range, largest cloud beyond the bucket kernels
    ([300, 300], 0),                    # nothing selected
    ([64, 64, 64], 64),                 # k == n everywhere
])
def test_fps_ptr_path_vs_oracle(dev, sizes, k):
    """The ptr path launches the sampling kernel for the average cloud size before the host has
    read the prepare summary; the kernel must do nothing when a cloud is larger, and the host then
    runs the right variant."""
    fps, *_ = _f()
    g = torch.Generator().manual_seed(sum(sizes) + k)
    pos = torch.randn(sum(sizes), 3, generator=g)
    ptr = _ptr(sizes)
    got = fps(pos.to(dev), k, ptr=ptr.to(dev))
    want = oracle.fps(pos.numpy(), ptr.numpy(), np.minimum(np.diff(ptr.numpy()), k))
    assert got.dtype == torch.int64 and got.is_contiguous()
    np.testing.assert_array_equal(got.cpu().numpy(), want)


def test_fps_ptr_path_invalid_and_repeated(dev):
    fps, *_ = _f()
    pos = torch.randn(5000, 3, device=dev)
    with pytest.raises(ValueError):
        fps(pos, 4, ptr=torch.tensor([0, 4000, 3000, 5000], device=dev))
    with pytest.raises(ValueError):
        fps(pos, 4, ptr=torch.tensor([0, 2000, 5001], device=dev))
    # valid calls right after, with a smaller problem second: nothing stale from the earlier ones
    cpu = pos.cpu().numpy()
    for ptr, k in (([0, 2500, 5000], 300), ([0, 10, 40], 5)):
        got = fps(pos, k, ptr=torch.tensor(ptr, device=dev)).cpu().numpy()
        want = oracle.fps(cpu, np.array(ptr), np.minimum(np.diff(ptr), k))
        np.testing.assert_array_equal(got, want)


def test_fps_invalid_ptr_raises(dev):
    from gdl_amd.csrc import fps_cuda
    pos = torch.randn(10, 3, device=dev)
    with pytest.raises(ValueError):
        fps_cuda(pos, torch.tensor([0, 8, 5], device=dev), torch.tensor([2, 2], device=dev))
    with pytest.raises(ValueError):
        fps_cuda(pos, torch.tensor([0, 11], device=dev), torch.tensor([2], device=dev))


# ----------------------------------------------------------------------------------- KNN ---

def _knn_check(dev, q, s, pq, ps, k):
    _, knn, _, _ = _f()
    gi, gd = knn(q.to(dev), s.to(dev), pq.to(dev), ps.to(dev), k)
    wi, wd = oracle.knn(q.numpy(), s.numpy(), pq.numpy(), ps.numpy(), k)
    np.testing.assert_array_equal(gi.cpu().numpy(), wi)
    np.testing.assert_array_equal(gd.cpu().numpy().view(np.uint32), wd.view(np.uint32))


@pytest.mark.parametrize("k", [1, 2, 3, 4, 5, 8, 9, 16, 17, 33, 64, 100, 128])
def test_knn_vs_oracle(dev, k):
    g = torch.Generator().manual_seed(k)
    qs, ss = [30, 0, 200, 77, 5], [50, 10, 1500, 0, 3]
    q = torch.randn(sum(qs), 3, generator=g)
    s = torch.randn(sum(ss), 3, generator=g)
    _knn_check(dev, q, s, _ptr(qs), _ptr(ss), k)


def _knn_grid_problem(kind, g):
    """Source clouds of >= 1024 points on average (the grid search); queries in and around them."""
    if kind == "cube":
        ss, qs = [5000, 3000, 8000], [700, 0, 900]
        s = torch.rand(sum(ss), 3, generator=g) * torch.tensor([4.0, 1.0, 0.25])
        q = (torch.rand(sum(qs), 3, generator=g) * 3 - 1) * torch.tensor([4.0, 1.0, 0.25])
    elif kind == "lattice":  # integer points: exact distances, ties everywhere
        s = _lattice(20, 1)
        q = _lattice(8, 2) * 2.5 - 1.0
        ss, qs = [8000], [512]
    elif kind == "sphere":
        d = torch.randn(12000, 3, generator=g)
        s = d / d.norm(dim=1, keepdim=True)
        q = s[torch.randperm(12000, generator=g)[:1500]] * 1.01
        ss, qs = [4000, 4000, 4000], [500, 500, 500]
    elif kind == "plane":    # zero extent in z: one cell layer
        s = torch.cat([torch.rand(6000, 2, generator=g), torch.zeros(6000, 1)], 1)
        q = torch.rand(800, 3, generator=g) - 0.25
        ss, qs = [6000], [800]
    elif kind == "small_cloud":  # a cloud with fewer sources than k, an empty one
        s = torch.randn(6005, 3, generator=g)
        q = torch.randn(600, 3, generator=g)
        ss, qs = [6000, 5, 0], [300, 200, 100]
    elif kind == "uncovered":  # queries before the first and after the last cloud: padding
        s = torch.randn(9000, 3, generator=g)
        q = torch.randn(800, 3, generator=g)
        return q, s, torch.tensor([50, 300, 300, 700]), _ptr([4000, 3000, 2000])
    elif kind == "scene":    # one 70,000-point cloud, density varying ~1000x (32 lanes per query)
        dense = torch.randn(20000, 3, generator=g) * 0.05
        ring = torch.rand(30000, generator=g) * 6.2832
        rad = 1.0 + 9.0 * torch.rand(30000, generator=g)
        rings = torch.stack([rad * ring.cos(), rad * ring.sin(), 0.02 * torch.randn(30000, generator=g)], 1)
        sparse = (torch.rand(20000, 3, generator=g) - 0.5) * torch.tensor([40.0, 40.0, 4.0])
        s = torch.cat([dense, rings, sparse])
        q = torch.cat([s[torch.randperm(70000, generator=g)[:500]], torch.randn(100, 3, generator=g) * 8])
        ss, qs = [70000], [600]
    else:                    # "nonfinite": one source at inf -> the cloud falls back to one cell
        s = torch.randn(5000, 3, generator=g)
        s[17] = float("inf")
        q = torch.randn(300, 3, generator=g)
        ss, qs = [5000], [300]
    return q, s, _ptr(qs), _ptr(ss)


@pytest.mark.parametrize("kind", ["cube", "lattice", "sphere", "plane", "small_cloud", "uncovered",
                                  "nonfinite", "scene"])
@pytest.mark.parametrize("k", [1, 3, 8, 16, 17, 32])
def test_knn_grid_vs_oracle(dev, kind, k):
    g = torch.Generator().manual_seed(k * 31 + len(kind))
    q, s, pq, ps = _knn_grid_problem(kind, g)
    _knn_check(dev, q, s, pq, ps, k)


def test_knn_lattice_ties(dev):
    s = _lattice(7)
    q = _lattice(4, 3) + 0.5 * (torch.arange(64).reshape(-1, 1) % 2)  # some half-integer queries
    _knn_check(dev, q, s, _ptr([64]), _ptr([343]), 27)
    _, _, knn_self, _ = _f()
    idx, d = knn_self(s.to(dev), _ptr([343]).to(dev), 7)
    assert torch.equal(idx[:, 0].cpu(), torch.arange(343)) and (d[:, 0] == 0).all()


def test_knn_bad_args(dev):
    _, knn, _, _ = _f()
    x = torch.randn(5, 3, device=dev)
    with pytest.raises(ValueError):
        knn(x, x, torch.tensor([0, 5], device=dev), torch.tensor([0, 2, 5], device=dev), 2)
    with pytest.raises(ValueError):
        knn(x, x, torch.tensor([0, 5], device=dev), torch.tensor([0, 5], device=dev), -1)


@pytest.mark.parametrize("k", [129, 200, 256, 300, 513])
def test_knn_large_k_vs_oracle(dev, k):
    """k above 128 is listed in passes of 128 columns, each admitting only keys (d, j) above the
    previous pass's last: clouds larger and smaller than k (padding), an empty cloud, and a
    lattice with ties everywhere; the reference path accepts any k (csrc/__init__.py:484-486)."""
    g = torch.Generator().manual_seed(k)
    qs, ss = [40, 0, 90, 7, 33], [600, 10, 2500, 0, 150]
    q = torch.randn(sum(qs), 3, generator=g)
    s = torch.randn(sum(ss), 3, generator=g)
    _knn_check(dev, q, s, _ptr(qs), _ptr(ss), k)
    lat = _lattice(9)                        # 729 integer points: equal distances in runs
    ql = _lattice(3, 4) + 0.5 * (torch.arange(27).reshape(-1, 1) % 2)
    _knn_check(dev, ql, lat, _ptr([27]), _ptr([729]), k)


# -------------------------------------------------------------------------- radius graph ---

def _rg_check(dev, x, r, K=32, loop=False, mask=None, batch=None, nb=None):
    *_, rg = _f()
    row, col = rg(x.to(dev), r, max_num_neighbors=K, loop=loop,
                  mask=None if mask is None else mask.to(dev),
                  batch=None if batch is None else batch.to(dev), num_batch_elements=nb)
    wr, wc = oracle.radius_graph(x.numpy(), r, K, loop,
                                 mask=None if mask is None else mask.numpy(),
                                 batch=None if batch is None else batch.cpu().numpy(),
                                 num_batch_elements=nb)
    assert row.dtype == torch.int64 and col.dtype == torch.int64
    np.testing.assert_array_equal(col.cpu().numpy(), wc)
    np.testing.assert_array_equal(row.cpu().numpy(), wr)
    return row, col


@pytest.mark.parametrize("N,r", [(50, 0.5), (100, 0.3), (200, 0.2), (500, 0.15), (1000, 0.1)])
@pytest.mark.parametrize("K", [4, 16, 300])
def test_radius_vs_oracle(dev, N, r, K):
    torch.manual_seed(42)
    x = torch.randn(N, 3)
    _rg_check(dev, x, r * 4, K)   # dense: K caps bind (selection path)
    _rg_check(dev, x, r, K)


def test_radius_lattice_boundary(dev):
    """Integer lattice, r = 1: neighbours at distance exactly 1 are excluded (d < r2)."""
    x = _lattice(6)
    r, c = _rg_check(dev, x, 1.0, 32)
    assert r.numel() == 0
    r, c = _rg_check(dev, x, 1.5, 32)     # 6-neighbourhood
    r, c = _rg_check(dev, x, 1.5, 3)      # ties at d = 1 broken toward lower index
    r, c = _rg_check(dev, x, 2.0, 100, loop=True)


def test_radius_masks_batches(dev):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(600, 3, generator=g)
    mask = torch.rand(600, generator=g) > 0.3
    batch = torch.randint(0, 5, (600,), generator=g)          # unsorted cloud ids
    _rg_check(dev, x, 0.6, 16, mask=mask)
    _rg_check(dev, x, 0.6, 16, batch=batch)
    _rg_check(dev, x, 0.6, 16, batch=batch, mask=mask, loop=True)
    _rg_check(dev, x, 0.6, 16, nb=4)                          # contiguous equal chunks
    _rg_check(dev, x, 0.6, 16, batch=batch.sort().values, nb=5)


def test_radius_reference_kats(dev):
    """tests/test_phase1.py:258-298 and tests/test_radius_graph_cuda.py:105-192."""
    *_, rg = _f()
    x = torch.tensor([[0.0, 0, 0], [0.1, 0, 0], [10.0, 0, 0]], device=dev)
    row, col = rg(x, r=1.0)
    assert row.numel() == 2 and 2 not in row.tolist() and 2 not in col.tolist()
    xr = torch.randn(20, 3, device=dev)
    row, col = rg(xr, r=100.0)
    assert not (row == col).any() and row.numel() == 20 * 19
    row, col = rg(torch.tensor([[0.0, 0, 0], [0.1, 0, 0]], device=dev), r=100.0,
                  batch=torch.tensor([0, 1], device=dev))
    assert row.numel() == 0
    assert rg(torch.randn(20, 3, device=dev) * 10, r=0.001)[0].numel() == 0
    m = torch.ones(200, dtype=torch.bool, device=dev)
    m[150:] = False
    row, col = rg(torch.randn(200, 3, device=dev), 0.4, max_num_neighbors=16, mask=m)
    assert (row < 150).all() and (col < 150).all()
    assert rg(torch.randn(100, 3, device=dev), 1.0, mask=torch.zeros(100, dtype=torch.bool,
                                                                     device=dev))[0].numel() == 0
    row, col = rg(torch.randn(50, 3, device=dev), 10.0, max_num_neighbors=64, loop=True)
    assert (row == col).sum() == 50
    assert rg(torch.randn(1, 3, device=dev), 1.0)[0].numel() == 0
    assert rg(torch.tensor([[0.0, 0, 0], [100.0, 0, 0]], device=dev), 1.0)[0].numel() == 0
    assert rg(torch.tensor([[0.0, 0, 0], [0.1, 0, 0]], device=dev), 0.5)[0].numel() == 2
    assert rg(torch.randn(100, 3, device=dev), 0.0)[0].numel() == 0
    from geoembodied.functional.radius_graph import compute_edge_vectors
    diff, dist, direction = compute_edge_vectors(torch.tensor([[0.0, 0, 0], [3.0, 4, 0]], device=dev),
                                                 torch.tensor([0], device=dev),
                                                 torch.tensor([1], device=dev))
    assert torch.allclose(dist.cpu(), torch.tensor([5.0]))
    assert torch.allclose(direction.cpu(), torch.tensor([[0.6, 0.8, 0.0]]))
    from geoembodied.csrc import get_radius_graph_backend
    assert get_radius_graph_backend() == "cuda"


@pytest.mark.parametrize("layout", ["chunks", "shuffled", "unequal", "foreign_id"])
def test_radius_batch_layouts(dev, layout):
    """A batch vector with N % B == 0 first takes the per-cloud front end, which checks on the
    device that batch[i] == i // (N / B); any other layout is reported with the edge count and
    redone on the general path.  Every layout must give the oracle's graph."""
    B, n = 6, 700
    N = B * n
    g = torch.Generator().manual_seed(len(layout))
    x = torch.randn(N, 3, generator=g) * 0.7
    batch = torch.arange(B).repeat_interleave(n)
    if layout == "shuffled":                  # equal counts, interleaved
        batch = batch[torch.randperm(N, generator=g)]
    elif layout == "unequal":                 # sorted, unequal sizes
        batch = torch.repeat_interleave(torch.arange(B), torch.tensor([900, 500, 700, 800, 600, 700]))
    elif layout == "foreign_id":              # one entry outside [0, B) (excluded point)
        batch[1234] = B + 2
    _rg_check(dev, x, 0.3, 12, batch=batch, nb=B)
    _rg_check(dev, x, 0.3, 12, loop=True, batch=batch, nb=B)
    from gdl_amd.csrc import _BATCH_NOT_CHUNKED, radius_graph_hip
    bd = batch.to(dev)
    radius_graph_hip(x.to(dev), 0.3, max_num_neighbors=12, batch=bd, num_batch_elements=B)
    # a layout the device rejected is remembered for the same unchanged tensor, so the next
    # call goes straight to the general path (and still gives the oracle's graph)
    assert (bd in _BATCH_NOT_CHUNKED) == (layout != "chunks")
    _rg_check(dev, x, 0.3, 12, batch=bd, nb=B)


def test_radius_outputs_exact_size(dev):
    """A sparse graph (E well below N * max_num_neighbors) comes back in exact-sized tensors, not
    as views of the bound-sized scratch; a dense one may share the scratch."""
    from gdl_amd.csrc import radius_graph_hip
    g = torch.Generator().manual_seed(2)
    x = (torch.rand(3000, 3, generator=g) * 4).to(dev)
    row, col = radius_graph_hip(x, 0.2, max_num_neighbors=32)
    assert row.numel() < 3000 * 16
    for t in (row, col):
        assert t.untyped_storage().nbytes() == 8 * t.numel()
    xd = (torch.rand(3000, 3, generator=g) * 0.01).to(dev)   # every target has > K sources
    row, col = radius_graph_hip(xd, 0.2, max_num_neighbors=8)
    assert row.numel() == 3000 * 8


@pytest.mark.parametrize("ppc", [1, 63, 1000, 4096])
def test_radius_per_cloud_front_masks_and_caps(dev, ppc):
    """Contiguous clouds given by num_batch_elements (the per-cloud front end up to 4096 points):
    masked points leave holes in the cell-ordered slots; loops, K caps with ties (integer
    lattice) and clouds with no valid point."""
    B = 5
    g = torch.Generator().manual_seed(ppc)
    x = torch.randn(B * ppc, 3, generator=g) * 0.5
    mask = torch.rand(B * ppc, generator=g) > 0.3
    mask[:ppc] = False                                   # cloud 0 entirely masked
    _rg_check(dev, x, 0.25, 9, mask=mask, nb=B)
    _rg_check(dev, x, 0.25, 9, loop=True, mask=mask, nb=B)
    lat = _lattice(16, 5)[: B * min(ppc, 800)]
    if lat.shape[0] >= B:
        _rg_check(dev, lat, 1.5, 7, nb=B)                # d^2 in {1, 2}: ties at the cap


@pytest.mark.parametrize("N", [10000, 50000])
def test_radius_large(dev, N):
    torch.manual_seed(N)
    x = torch.randn(N, 3) * 0.5
    _rg_check(dev, x, 0.05, 32)


def test_radius_degenerate_extent(dev):
    """All points on a line far longer than r: the per-axis cell cap grows the cells."""
    t = torch.linspace(0, 1000, 5000)
    x = torch.stack([t, torch.zeros_like(t), torch.zeros_like(t)], 1)
    _rg_check(dev, x, 0.5, 8)
    x2 = torch.zeros(300, 3)   # all coincident
    _rg_check(dev, x2, 0.1, 7)
    _rg_check(dev, x2, 0.1, 400, loop=True)


def test_radius_dense_blob_wave_selection_paths(dev):
    """Targets with more than K in-radius sources are selected by a whole wave: up to 1024 of
    them kept in LDS, beyond that re-scanned from the cell lists; K above 1024 compacts into the
    global list.  A 2500-point blob (every pair within r) beside a sparse cloud, with exact-tie
    lattice points, checked at K = 20 and K = 1100."""
    g = torch.Generator().manual_seed(17)
    blob = torch.rand(2500, 3, generator=g) * 0.01
    lat = _lattice(8, 3) * 0.004 + 0.02       # 512 points, many equal distances
    sparse = torch.rand(1500, 3, generator=g) * 4 + 1
    x = torch.cat([blob, lat, sparse])
    _rg_check(dev, x, 0.05, 20)
    _rg_check(dev, x, 0.05, 1100)
    _rg_check(dev, x, 0.05, 1100, loop=True)


@pytest.mark.parametrize("per,r", [(1025, 0.13), (5000, 0.078)])
def test_radius_without_lists(dev, per, r):
    """When N x K exceeds the per-target lists the workspace holds (2^28 entries), the rows come
    from the emit kernel, which re-scans each target's stencil: rows sorted in LDS for K <= 256,
    the K-th distance and the index threshold found by binary search for targets above K.
    About 1.05 M points with K = 256, in clouds of 1025 points (the per-cloud front end) or of
    5000 (the general grid build), each cloud in its own unit cube (~10 sources per target);
    three clouds are blobs 0.02 across, where every target has more than K sources."""
    K = 256
    B = -(-1049600 // per)
    N = B * per
    assert N * K > (1 << 28)
    g = torch.Generator().manual_seed(per)
    x = torch.rand(N, 3, generator=g)
    x[: 3 * per] *= 0.02
    _rg_check(dev, x, r, K, nb=B)


# ------------------------------------------------------------------------ BASELINE configs ---

def test_config_c1(dev):
    """C1: FPS 2048 -> 512, radius graph over the centres, then the C = 32 segment sum of the
    centre features over that graph, forward and backward."""
    import bench
    from seg_legs import reduce_leg_oracle
    fps, _, _, rg = _f()
    c = bench.make_c1()
    idx = fps(c["pos"].to(dev), c["M"]).cpu().numpy()
    np.testing.assert_array_equal(idx, oracle.fps(c["pos"].numpy(), [0, 2048], [512]))
    cen = c["pos"][torch.from_numpy(idx)]
    row, col = _rg_check(dev, cen, c["r"], c["K"])
    assert row.numel() > 0   # 178 edges: the 512 centres are spread by FPS
    msg = c["feat"][row.cpu()]
    reduce_leg_oracle(dev, msg, col, c["M"], "sum", seed=1)


def test_config_c2(dev):
    import bench
    fps, knn, _, rg = _f()
    c = bench.make_c2()
    pos, ptr = c["pos"], c["ptr"]
    idx = fps(pos.to(dev), c["M"], ptr=ptr.to(dev)).cpu().numpy()
    np.testing.assert_array_equal(idx, oracle.fps(pos.numpy(), ptr.numpy(), [c["M"]] * c["B"]))
    row, col = _rg_check(dev, pos, c["r"], c["K"], batch=c["batch"], nb=c["B"])
    assert row.numel() > 600000
    cen = pos[torch.from_numpy(idx)]
    pq = torch.arange(c["B"] + 1) * c["M"]
    _knn_check(dev, cen, pos, pq, ptr, c["k"])
    _rg_check(dev, cen, c["r"], c["K"], nb=c["B"])


def test_config_c4(dev):
    import bench
    fps, _, _, rg = _f()
    c = bench.make_c4()
    pos, ptr = c["pos"], c["ptr"]
    i1 = fps(pos.to(dev), 512, ptr=ptr.to(dev)).cpu().numpy()
    np.testing.assert_array_equal(i1, oracle.fps(pos.numpy(), ptr.numpy(), [512] * c["B"]))
    q1 = pos[torch.from_numpy(i1)]
    p1 = torch.arange(c["B"] + 1) * 512
    i2 = fps(q1.to(dev), 128, ptr=p1.to(dev)).cpu().numpy()
    np.testing.assert_array_equal(i2, oracle.fps(q1.numpy(), p1.numpy(), [128] * c["B"]))
    q2 = q1[torch.from_numpy(i2)]
    # pooling at each level: segment max and mean of N(0, 1) features gathered over the radius
    # graph (C = 64 on the 512-level r = 0.2 graph, C = 128 on the 128-level r = 0.4 graph),
    # forward and backward
    from seg_legs import reduce_leg_oracle
    g = torch.Generator().manual_seed(4)
    for pts, r, C in ((q1, 0.2, 64), (q2, 0.4, 128)):
        row, col = _rg_check(dev, pts, r, 64, nb=c["B"])
        feat = torch.randn(pts.shape[0], C, generator=g)
        msg = feat[row.cpu()]
        for red in ("max", "mean"):
            reduce_leg_oracle(dev, msg, col, pts.shape[0], red, seed=C)


def test_config_c5(dev):
    import bench
    fps, knn, _, rg = _f()
    c = bench.make_c5()
    pos = c["pos"]
    N = pos.shape[0]
    idx = fps(pos.to(dev), c["M"]).cpu().numpy()
    np.testing.assert_array_equal(idx, oracle.fps(pos.numpy(), [0, N], [c["M"]]))
    cen = pos[torch.from_numpy(idx)]
    # the radius graph over the 16,384 centres is empty at r = 0.5 m: FPS spreads them about a
    # metre apart over the 80 m scene, so its segment sum is all zeros
    row, col = _rg_check(dev, cen, c["r"], c["K"])
    from seg_legs import reduce_leg_oracle
    feat = torch.randn(c["M"], c["C"], generator=torch.Generator().manual_seed(5))
    out = reduce_leg_oracle(dev, feat[row.cpu()], col, c["M"], "sum", seed=5)
    assert row.numel() == 0 and torch.all(out == 0)
    # every one of the 16,384 centres against all 131,072 sources (k = 8)
    _knn_check(dev, cen, pos, torch.tensor([0, c["M"]]), torch.tensor([0, N]), c["k"])


def test_config_c5_all_points(dev):
    """C5's radius graph over all 131,072 lidar points (r = 0.5 m, at most 64 neighbours: 5.3 M
    edges, dense near the sensor, sparse far away), bit-exact against the oracle, and the C = 32
    segment sum over it, forward and backward, against float64 sums."""
    import bench
    from seg_legs import csr_checked, reduce_leg_fp64
    c = bench.make_c5()
    pos = c["pos"]
    N = pos.shape[0]
    row, col = _rg_check(dev, pos, c["r"], c["K"])
    assert row.numel() > 5_000_000
    cs, pm, ns, ne = csr_checked(dev, col, N)
    g = torch.Generator(device=dev).manual_seed(5)
    feat = torch.randn(N, c["C"], device=dev, generator=g)
    msg = feat[row]
    grad = torch.randn(N, c["C"], device=dev, generator=g)
    reduce_leg_fp64(msg, cs, pm, ns, ne, N, "sum", grad)
