"""Pins the CPU oracle (oracle/) independently of its own formulas.

Each oracle function is checked against at least one of:
  * the reference's own known-answer tests (tests/test_phase1.py:258-298,
    tests/test_radius_graph_cuda.py:105-192, tests/test_fps_cuda_remote.py:63-90,
    tests/test_segment_reduce.py:118-141);
  * exact brute force in pure-Python integers on integer lattices, where every fp32 operation
    of the oracle is exact, so a dropped term, a wrong index or a wrong tie rule shows;
  * library routines (numpy stable argsort / add.at, scipy cKDTree, torch scatter ops and
    autograd);
  * the restated reference CPU path (oracle/ref_cpu_path.py: the reference's torch op sequences).
"""

import itertools

import numpy as np
import pytest
import torch
from scipy.spatial import cKDTree

import oracle
from oracle import ref_cpu_path


def _lattice(n_side, seed=0, scale=1):
    g = np.array(list(itertools.product(range(n_side), repeat=3)), dtype=np.int64) * scale
    return g[np.random.default_rng(seed).permutation(len(g))]


def _d2(a, b):
    return sum((int(x) - int(y)) ** 2 for x, y in zip(a, b))


# ----------------------------------------------------------------------------------- FPS ---

def _fps_int(pts, k):
    """Greedy max-min in exact integers: lowest index on ties."""
    n = len(pts)
    sel = [0]
    md = [None] * n
    for _ in range(k - 1):
        c = pts[sel[-1]]
        for i in range(n):
            d = _d2(pts[i], c)
            md[i] = d if md[i] is None else min(md[i], d)
        best = max(md)
        sel.append(md.index(best))
    return sel


@pytest.mark.parametrize("n_side,k,seed", [(4, 20, 0), (5, 60, 1), (6, 100, 2)])
def test_fps_matches_exact_integer_greedy(n_side, k, seed):
    pts = _lattice(n_side, seed)
    got = oracle.fps(pts.astype(np.float32), [0, len(pts)], [k])
    assert got.tolist() == _fps_int(pts.tolist(), k)


def test_fps_line_closed_form():
    x = np.zeros((11, 3), np.float32)
    x[:, 0] = np.arange(11)
    # 0, then the far end 10, then the middle 5, then the lowest of the tied quarter points
    assert oracle.fps(x, [0, 11], [5]).tolist() == [0, 10, 5, 2, 7]


def test_fps_reference_kat_and_clamping():
    g = np.random.default_rng(0)
    pos = g.standard_normal((100, 3)).astype(np.float32)
    idx = oracle.fps(pos, [0, 60, 100], [15, 10])
    assert len(idx) == 25 and len(set(idx.tolist())) == 25
    assert (idx[:15] < 60).all() and (idx[15:] >= 60).all()
    assert idx[0] == 0 and idx[15] == 60
    assert oracle.fps(pos, [0, 100], [100]).tolist() == list(range(100))
    assert oracle.fps(pos, [0, 100], [500]).tolist() == list(range(100))
    assert oracle.fps(pos, [0, 100], [0]).size == 0


def test_fps_greedy_property_fp64():
    """Each pick attains the max fp64 min-distance up to fp32 rounding."""
    g = np.random.default_rng(1)
    pos = g.standard_normal((700, 3)).astype(np.float32)
    idx = oracle.fps(pos, [0, 700], [60])
    p64 = pos.astype(np.float64)
    md = np.full(700, np.inf)
    for i in range(1, 60):
        md = np.minimum(md, ((p64 - p64[idx[i - 1]]) ** 2).sum(1))
        assert md[idx[i]] >= md.max() * (1 - 1e-6)


def test_fps_matches_reference_cpu_path():
    """The reference's torch op sequence (ref_cpu_path.fps) gives identical picks."""
    g = torch.Generator().manual_seed(3)
    pos = torch.randn(900, 3, generator=g)
    ptr = torch.tensor([0, 400, 900])
    k = torch.tensor([70, 120])
    assert ref_cpu_path.fps(pos, ptr, k).tolist() == oracle.fps(pos.numpy(), ptr.numpy(), k.numpy()).tolist()


# ----------------------------------------------------------------------------------- KNN ---

def _knn_int(q, s, k):
    out = []
    for a in q:
        keys = sorted((_d2(a, b), j) for j, b in enumerate(s))[:k]
        out.append([j for _, j in keys] + [-1] * (k - len(keys)))
    return out


def test_knn_exact_integer_lattice():
    s = _lattice(5, 1)
    q = _lattice(3, 2) * 2 - 1
    idx, dist = oracle.knn(q.astype(np.float32), s.astype(np.float32), [0, len(q)], [0, len(s)], 10)
    assert idx.tolist() == _knn_int(q.tolist(), s.tolist(), 10)
    want_d = [[_d2(a, s[j]) for j in row] for a, row in zip(q.tolist(), idx.tolist())]
    assert dist.tolist() == want_d


def test_knn_padding_and_batches():
    s = np.arange(12, dtype=np.float32).reshape(4, 3)
    q = s[:3] + 0.5
    idx, dist = oracle.knn(q, s, [0, 1, 1, 3], [0, 2, 2, 4], 3)
    assert idx[0].tolist()[:2] == [0, 1] and idx[0, 2] == -1 and dist[0, 2] == np.float32(1e30)
    assert set(idx[1].tolist()) <= {2, 3, -1} and idx[1, 2] == -1


def test_knn_distances_match_numpy_formula_and_kdtree():
    g = np.random.default_rng(4)
    s = g.standard_normal((800, 3)).astype(np.float32)
    q = g.standard_normal((50, 3)).astype(np.float32)
    idx, dist = oracle.knn(q, s, [0, 50], [0, 800], 12)
    diff = q[:, None, :] - s[None, :, :]
    full = (diff * diff).sum(-1, dtype=np.float32)      # the reference formula, numpy fp32
    np.testing.assert_array_equal(dist, np.take_along_axis(full, idx, 1))
    d64, j64 = cKDTree(s.astype(np.float64)).query(q.astype(np.float64), k=12)
    assert np.allclose(np.sqrt(dist), d64, rtol=1e-5)
    assert (np.sort(idx, 1) == np.sort(j64, 1)).mean() > 0.99


def test_knn_matches_reference_cpu_path_values():
    g = torch.Generator().manual_seed(5)
    q = torch.randn(60, 3, generator=g)
    s = torch.randn(300, 3, generator=g)
    pq, ps = torch.tensor([0, 20, 60]), torch.tensor([0, 100, 300])
    ri, rd = ref_cpu_path.knn(q, s, pq, ps, 9)
    oi, od = oracle.knn(q.numpy(), s.numpy(), pq.numpy(), ps.numpy(), 9)
    np.testing.assert_array_equal(rd.numpy(), od)          # same distances, same order
    np.testing.assert_array_equal(np.sort(ri.numpy(), 1), np.sort(oi, 1))


# -------------------------------------------------------------------------- radius graph ---

def _radius_int(pts, r2, K, loop=False, cloud=None):
    n = len(pts)
    rows, cols = [], []
    for i in range(n):
        cand = []
        for j in range(n):
            if (not loop and i == j) or (cloud is not None and (cloud[i] != cloud[j] or cloud[i] < 0)):
                continue
            d = _d2(pts[i], pts[j])
            if d < r2:
                cand.append((d, j))
        keep = sorted(j for _, j in sorted(cand)[:K])
        rows += keep
        cols += [i] * len(keep)
    return rows, cols


@pytest.mark.parametrize("r,K,loop", [(1.5, 32, False), (1.5, 3, False), (2.0, 100, True), (1.0, 8, False)])
def test_radius_exact_integer_lattice(r, K, loop):
    pts = _lattice(4, 7)
    row, col = oracle.radius_graph(pts.astype(np.float32), r, K, loop)
    wr, wc = _radius_int(pts.tolist(), r * r, K, loop)
    assert row.tolist() == wr and col.tolist() == wc


def test_radius_batch_and_mask_exact():
    pts = _lattice(4, 8)
    g = np.random.default_rng(2)
    batch = g.integers(0, 3, len(pts))
    mask = g.random(len(pts)) > 0.25
    row, col = oracle.radius_graph(pts.astype(np.float32), 1.8, 6, batch=batch, mask=mask)
    cloud = np.where(mask, batch, -1)
    wr, wc = _radius_int(pts.tolist(), 1.8 * 1.8, 6, cloud=cloud.tolist())
    assert row.tolist() == wr and col.tolist() == wc


def test_radius_reference_kats():
    x = np.array([[0, 0, 0], [0.1, 0, 0], [10, 0, 0]], np.float32)
    row, col = oracle.radius_graph(x, 1.0)
    assert len(row) == 2 and 2 not in row and 2 not in col
    xr = np.random.default_rng(0).standard_normal((20, 3)).astype(np.float32)
    row, col = oracle.radius_graph(xr, 100.0)
    assert not (row == col).any()
    row, _ = oracle.radius_graph(np.array([[0, 0, 0], [0.1, 0, 0]], np.float32), 100.0, batch=[0, 1])
    assert len(row) == 0
    assert len(oracle.radius_graph(xr * 10, 0.001)[0]) == 0
    assert len(oracle.radius_graph(xr[:1], 1.0)[0]) == 0
    assert len(oracle.radius_graph(np.array([[0, 0, 0], [100, 0, 0]], np.float32), 1.0)[0]) == 0
    assert len(oracle.radius_graph(np.array([[0, 0, 0], [0.1, 0, 0]], np.float32), 0.5)[0]) == 2
    assert len(oracle.radius_graph(xr, 0.0)[0]) == 0
    row, col = oracle.radius_graph(xr, 10.0, 64, loop=True)
    assert (row == col).sum() == 20
    m = np.ones(20, bool)
    m[15:] = False
    row, col = oracle.radius_graph(xr, 1.5, 16, mask=m)
    assert (row < 15).all() and (col < 15).all()
    assert len(oracle.radius_graph(xr, 1.5, 16, mask=np.zeros(20, bool))[0]) == 0


def test_radius_vs_kdtree_and_threshold():
    """Edge set == scipy query_pairs(r) away from the r boundary; threshold is fl32(r*r)."""
    g = np.random.default_rng(9)
    x = g.standard_normal((1500, 3)).astype(np.float32)
    r = 0.2
    row, col = oracle.radius_graph(x, r, 10_000)
    got = set(zip(row.tolist(), col.tolist()))
    pairs = cKDTree(x.astype(np.float64)).query_pairs(r)
    want = {(a, b) for a, b in pairs} | {(b, a) for a, b in pairs}
    x64 = x.astype(np.float64)
    for a, b in got ^ want:
        d = ((x64[a] - x64[b]) ** 2).sum()
        assert abs(d - r * r) < 1e-6 * r * r
    assert oracle.fp32_radius_sq(0.1) == float(np.float32(0.1 * 0.1))
    assert oracle.fp32_radius_sq(0.1) != float(np.float32(0.1)) ** 2  # 1 ulp below fl32(r)^2


def test_radius_vs_reference_cpu_path():
    """Same edges as the reference's cdist/topk CPU path except pairs in cdist's error band."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2 * 600, 3, generator=g) * 0.6
    rr, rc = ref_cpu_path.radius_graph(x, 0.25, 2, 1000)
    orow, ocol = oracle.radius_graph(x.numpy(), 0.25, 1000, num_batch_elements=2)
    a = set(zip(rr.tolist(), rc.tolist()))
    b = set(zip(orow.tolist(), ocol.tolist()))
    x64 = x.double().numpy()
    diff = a ^ b
    assert len(diff) <= 10
    for i, j in diff:
        assert abs(((x64[i] - x64[j]) ** 2).sum() - 0.0625) < 3e-2 * 0.0625


def test_c2_disagreement_with_reference_cdist_path():
    """The survey's D3 diagnostic on the real C2 batch (16 x 4096 points, r = 0.1, K = 32): the
    exact edge set against the reference's cdist/topk CPU path (radius_graph.py:204-275).  They
    differ only in pairs whose exact squared distance lies within cdist's rounding band of r2:
    cdist forms |x|^2 + |y|^2 - 2 x.y in fp32, so its error is a few ulps of |x|^2 + |y|^2
    (bound used: 4 * 2^-24 * (|x_i|^2 + |x_j|^2)).  On this batch: 4 directed edges (2 pairs)
    of 657,154."""
    import bench
    c = bench.make_c2()
    x = c["pos"]
    rr, rc = ref_cpu_path.radius_graph(x, c["r"], c["B"], c["K"])
    orow, ocol = oracle.radius_graph(x.numpy(), c["r"], c["K"], batch=c["batch"].numpy(),
                                     num_batch_elements=c["B"])
    a = set(zip(rr.tolist(), rc.tolist()))
    b = set(zip(orow.tolist(), ocol.tolist()))
    assert len(b) == 657_154
    diff = a ^ b
    x64 = x.double().numpy()
    r2 = oracle.fp32_radius_sq(c["r"])
    for i, j in diff:
        d = ((x64[i] - x64[j]) ** 2).sum()
        band = 4 * 2.0 ** -24 * ((x64[i] ** 2).sum() + (x64[j] ** 2).sum())
        assert abs(d - r2) <= band, (i, j, d)
        assert ((i, j) in b) == (d < r2)        # the exact set is on the right side of r2
    print(f"C2 disagreement with the cdist path: {len(diff)} directed edges of {len(b)}")
    assert len(diff) == 4


# ---------------------------------------------------------------------------- CSR build ---

@pytest.mark.parametrize("E,N", [(0, 5), (1, 1), (1000, 17), (5000, 4000)])
def test_csr_matches_numpy_stable_sort(E, N):
    g = np.random.default_rng(E + N)
    col = g.integers(-2, N + 2, E)
    cs, pm, ns, ne = oracle.sort_and_build_csr(col, N)
    key = np.where((col >= 0) & (col < N), col, N)
    order = np.argsort(key, kind="stable")
    np.testing.assert_array_equal(pm, order)
    np.testing.assert_array_equal(cs, key[order])
    counts = np.bincount(key, minlength=N + 1)[:N]
    np.testing.assert_array_equal(ne - ns, counts)
    np.testing.assert_array_equal(ns, np.concatenate([[0], np.cumsum(counts)[:-1]]))


# ------------------------------------------------------------------------ segment reduce ---

def _csr_problem(E, N, C, seed, ties=False):
    g = np.random.default_rng(seed)
    col = g.integers(0, N, E)
    msg = g.standard_normal((E, C))
    if ties:
        msg = np.round(msg * 2) / 2 + 0.25
    cs, pm, ns, ne = oracle.sort_and_build_csr(col, N)
    return col, msg.astype(np.float32), cs, pm, ns, ne


def test_segment_sum_mean_vs_add_at():
    col, msg, cs, pm, ns, ne = _csr_problem(3000, 400, 7, 0)
    ref = np.zeros((400, 7))
    np.add.at(ref, col, msg.astype(np.float64))
    out, scale = oracle.segment_reduce_fwd(msg, pm, ns, ne, 400, "sum")
    np.testing.assert_allclose(out, ref, rtol=0, atol=1e-12)
    absum = np.zeros((400, 7))
    np.add.at(absum, col, np.abs(msg.astype(np.float64)))
    np.testing.assert_allclose(scale, absum, atol=1e-12)
    cnt = np.bincount(col, minlength=400)
    mean, _ = oracle.segment_reduce_fwd(msg, pm, ns, ne, 400, "mean")
    np.testing.assert_allclose(mean, ref / np.maximum(cnt, 1)[:, None], atol=1e-12)


def test_segment_max_vs_torch_scatter_reduce():
    col, msg, cs, pm, ns, ne = _csr_problem(3000, 400, 5, 1, ties=True)
    t = torch.zeros(400, 5).scatter_reduce(0, torch.from_numpy(col).unsqueeze(1).expand(-1, 5),
                                           torch.from_numpy(msg), "amax", include_self=False)
    out, arg = oracle.segment_reduce_fwd(msg, pm, ns, ne, 400, "max")
    np.testing.assert_array_equal(out.astype(np.float32), t.numpy())
    # arg: unique maxima point at a sorted position holding the max; ties report -count
    for s in range(0, 400, 7):
        for c in range(5):
            seg = msg[pm[ns[s]:ne[s]], c]
            if len(seg) == 0:
                assert arg[s, c] == -1
            elif (seg == seg.max()).sum() == 1:
                assert msg[pm[arg[s, c]], c] == seg.max() and ns[s] <= arg[s, c] < ne[s]
            else:
                assert arg[s, c] == -(seg == seg.max()).sum()
    _, first = oracle.segment_reduce_fwd(msg, pm, ns, ne, 400, "max", tie_mode=1)
    nz = ne > ns
    assert (first[nz] >= 0).all()


def test_segment_backward_vs_torch_autograd():
    col, msg, cs, pm, ns, ne = _csr_problem(2000, 300, 4, 2, ties=True)
    E = len(col)
    idx = torch.from_numpy(col).unsqueeze(1).expand(-1, 4)
    g = torch.from_numpy(np.random.default_rng(5).standard_normal((300, 4)).astype(np.float32))
    for red in ("sum", "mean", "max"):
        m = torch.from_numpy(msg).requires_grad_(True)
        if red == "sum":
            y = torch.zeros(300, 4).scatter_add(0, idx, m)
        elif red == "mean":
            cnt = torch.bincount(torch.from_numpy(col), minlength=300).clamp(min=1)
            y = torch.zeros(300, 4).scatter_add(0, idx, m) / cnt.unsqueeze(1)
        else:
            y = torch.zeros(300, 4).scatter_reduce(0, idx, m, "amax", include_self=False)
        y.backward(g)
        out, arg = oracle.segment_reduce_fwd(msg, pm, ns, ne, 300, red)
        want = oracle.segment_reduce_bwd(g.numpy(), cs, pm, ns, ne, E, red, msg=msg, out=out,
                                         arg=arg if red == "max" else None)
        np.testing.assert_allclose(want, m.grad.numpy(), rtol=1e-6, atol=1e-7)


def test_segment_reference_kats():
    # all edges into node 0 sum to E (tests/test_segment_reduce.py:131-141)
    cs, pm, ns, ne = oracle.sort_and_build_csr(np.zeros(10, np.int64), 1)
    out, _ = oracle.segment_reduce_fwd(np.ones((10, 4), np.float32), pm, ns, ne, 1, "sum")
    assert out.tolist() == [[10.0] * 4]
    # E = 0 gives zeros (:118-129)
    cs, pm, ns, ne = oracle.sort_and_build_csr(np.zeros(0, np.int64), 10)
    out, _ = oracle.segment_reduce_fwd(np.zeros((0, 8), np.float32), pm, ns, ne, 10, "sum")
    assert out.shape == (10, 8) and not out.any()
    # backward of sum() is all ones (:74-89)
    col, msg, cs, pm, ns, ne = _csr_problem(200, 50, 8, 3)
    gm = oracle.segment_reduce_bwd(np.ones((50, 8)), cs, pm, ns, ne, 200, "sum")
    assert (gm == 1).all()


def test_bf16_round_matches_torch():
    g = np.random.default_rng(0)
    x = np.concatenate([g.standard_normal(10000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, 3.4e38], np.float32)])
    want = torch.from_numpy(x).bfloat16().float().numpy()
    got = oracle.bf16_round(x)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    np.testing.assert_array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))


# ----------------------------------------------------------------------- segment softmax ---

def test_sparse_softmax_vs_reference_op_sequence_and_closed_forms():
    """The oracle equals the reference's own torch op sequence (invariant_attention.py:202-230,
    restated in ref_cpu_path.sparse_softmax) in float64, and the closed forms hold: equal scores
    give 1/degree, a lone edge gives 1, every segment sums to 1, a constant shift changes
    nothing."""
    g = np.random.default_rng(4)
    N, E, H = 40, 300, 3
    index = g.integers(0, N, E)
    x = g.standard_normal((E, H)) * 3
    w = oracle.sparse_softmax(x, index, N)
    ref = ref_cpu_path.sparse_softmax(torch.from_numpy(x), torch.from_numpy(index), N).numpy()
    np.testing.assert_allclose(w, ref, rtol=1e-13, atol=1e-15)
    sums = np.zeros((N, H))
    np.add.at(sums, index, w)
    deg = np.bincount(index, minlength=N)
    np.testing.assert_allclose(sums[deg > 0], 1.0, rtol=1e-13)
    np.testing.assert_allclose(oracle.sparse_softmax(x + 7.5, index, N), w, rtol=1e-12, atol=1e-15)
    eq = oracle.sparse_softmax(np.ones((E, H)), index, N)
    np.testing.assert_allclose(eq, (1.0 / deg[index])[:, None].repeat(H, 1), rtol=1e-15)
    assert oracle.sparse_softmax(np.array([[-3.0]]), np.array([2]), 5).tolist() == [[1.0]]
    # NaN makes its segment NaN, as torch's amax does
    xn = np.array([[1.0], [np.nan], [2.0]])
    wn = oracle.sparse_softmax(xn, np.array([0, 0, 1]), 2)
    assert np.isnan(wn[:2]).all() and wn[2, 0] == 1.0


def test_sparse_softmax_backward_vs_torch_autograd():
    g = np.random.default_rng(5)
    N, E, H = 25, 200, 2
    index = g.integers(0, N, E)
    x = torch.from_numpy(g.standard_normal((E, H))).requires_grad_(True)
    gr = g.standard_normal((E, H))
    ref_cpu_path.sparse_softmax(x, torch.from_numpy(index), N).backward(torch.from_numpy(gr))
    w = oracle.sparse_softmax(x.detach().numpy(), index, N)
    np.testing.assert_allclose(oracle.sparse_softmax_bwd(gr, w, index, N), x.grad.numpy(),
                               rtol=1e-10, atol=1e-13)


# ----------------------------------------------------------- neighbourhood gather-sum ---

def test_idw_interpolation_vs_reference_op_sequence_and_closed_forms():
    """oracle idw_weights + gather_weighted_sum equal the reference's interpolation op sequence
    (equivariant_interp.py:95-125, restated in ref_cpu_path.idw_interpolate) in float64; equal
    distances give 1/(valid neighbours); a lone valid neighbour gets weight 1; all-padding rows
    are 0; the sum is linear in the features."""
    g = np.random.default_rng(7)
    Ns, No, K, C = 50, 30, 4, 6
    idx = g.integers(0, Ns, (No, K))
    idx[3, 1:] = -1
    idx[4] = -1
    dist = g.random((No, K)) * 2
    dist[5] = 0.7
    feat = g.standard_normal((Ns, C))
    w = oracle.idw_weights(idx, dist)
    out, _ = oracle.gather_weighted_sum(feat, idx, w)
    ref = ref_cpu_path.idw_interpolate(torch.from_numpy(feat), torch.from_numpy(idx),
                                       torch.from_numpy(dist)).numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(w[5], 0.25, rtol=1e-15)
    assert w[3].tolist() == [1.0, 0.0, 0.0, 0.0] and (out[4] == 0).all()
    out2, _ = oracle.gather_weighted_sum(2 * feat + 1, idx, w)
    np.testing.assert_allclose(out2, 2 * out + w.sum(1, keepdims=True) * (idx >= 0).any(1, keepdims=True),
                               rtol=1e-12, atol=1e-12)


def test_gather_weighted_sum_backward_vs_torch_autograd():
    g = np.random.default_rng(8)
    Ns, No, K, C = 40, 25, 5, 3
    idx = g.integers(-1, Ns, (No, K))
    f = torch.from_numpy(g.standard_normal((Ns, C))).requires_grad_(True)
    w = torch.from_numpy(g.standard_normal((No, K))).requires_grad_(True)
    ok = torch.from_numpy(idx >= 0)
    out = ((w * ok).unsqueeze(-1) * f[torch.from_numpy(idx).clamp(min=0)]).sum(1)
    go = g.standard_normal((No, C))
    out.backward(torch.from_numpy(go))
    gf, gw = oracle.gather_weighted_sum_bwd(go, f.detach().numpy(), idx, w.detach().numpy())
    np.testing.assert_allclose(gf, f.grad.numpy(), rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(gw, w.grad.numpy(), rtol=1e-12, atol=1e-14)


# ------------------------------------------------------------ adaptive radius statistic ---

def test_knn_radius_stat_vs_reference_expressions():
    """The oracle statistic equals the reference's expressions evaluated by torch on the same
    KNN distances: the mean up to float32 summation order, the median exactly."""
    g = np.random.default_rng(11)
    d = (g.random((5001, 2)) ** 2).astype(np.float32)
    d[:, 0] = 0.0
    d[7, 1] = 1e30   # padding distance: clamped at 1e20
    d[9, 1] = 0.0    # duplicate point: clamped at 1e-8 / 1e-12
    t = torch.from_numpy(d)
    ref_mean = t[:, 1].clamp(max=1e20).clamp(min=1e-8).sqrt().mean().item() * 4.0
    assert oracle.knn_radius_stat(d, 1, "mean", 4.0) == pytest.approx(ref_mean, rel=1e-6)
    ref_med = t[:, -1].clamp(min=1e-12).sqrt().median().item() * 2.5
    assert oracle.knn_radius_stat(d, 1, "median", 2.5) == ref_med
    even = d[:5000]
    assert oracle.knn_radius_stat(even, 1, "median", 1.0) == \
        torch.from_numpy(even)[:, -1].clamp(min=1e-12).sqrt().median().item()
    d[3, 1] = np.nan
    assert np.isnan(oracle.knn_radius_stat(d, 1, "median", 1.0))


# -------------------------------------------------- spherical harmonics / edge geometry ---

def test_spherical_harmonics_orthonormal_and_addition_theorem():
    """Gauss-Legendre x uniform-phi quadrature (exact for these degrees) gives the identity Gram
    matrix, and sum_m Y_lm(u)^2 = (2l+1)/(4 pi) on unit vectors: both pin every constant and
    formula independently of how the oracle writes them."""
    t, wt = np.polynomial.legendre.leggauss(12)
    phi = np.arange(24) * (2 * np.pi / 24)
    ct, P = np.meshgrid(t, phi, indexing="ij")
    st = np.sqrt(1 - ct ** 2)
    u = np.stack([st * np.cos(P), st * np.sin(P), ct], -1).reshape(-1, 3)
    w = (wt[:, None] * np.full(24, 2 * np.pi / 24)[None, :]).reshape(-1)
    Y = oracle.spherical_harmonics(u, 2)
    np.testing.assert_allclose((Y * w[:, None]).T @ Y, np.eye(9), atol=1e-12)
    g = np.random.default_rng(0).standard_normal((100, 3))
    Yn = oracle.spherical_harmonics(g, 2, normalize=True)
    for l, sl in ((0, slice(0, 1)), (1, slice(1, 4)), (2, slice(4, 9))):
        np.testing.assert_allclose((Yn[:, sl] ** 2).sum(1), (2 * l + 1) / (4 * np.pi), rtol=1e-12)
    assert oracle.spherical_harmonics(g, 1).shape == (100, 4)


def test_edge_geometry_and_avg_degree_closed_forms():
    g = np.random.default_rng(1)
    pos = g.standard_normal((30, 3))
    row, col = g.integers(0, 30, 80), g.integers(0, 30, 80)
    row[0] = col[0]                       # zero-length edge: dist clamps to 1e-8
    d, dist, Y = oracle.edge_geometry(pos, row, col)
    ref = pos[col] - pos[row]
    loops = row == col
    np.testing.assert_allclose(dist, np.maximum(np.sqrt((ref ** 2).sum(1)), 1e-8), rtol=1e-14)
    assert (dist[loops] == 1e-8).all() and (d[loops] == 0).all()
    np.testing.assert_allclose(np.linalg.norm(d[~loops], axis=1), 1.0, rtol=1e-14)
    ns = np.array([0, 2, 2, 5, 9])
    ne = np.array([2, 2, 5, 9, 9])
    np.testing.assert_allclose(oracle.graph_avg_degree(ns, ne, [0, 0, 1, 1, 1], 2),
                               [1.0, 1.0, 7 / 3, 7 / 3, 7 / 3])
    np.testing.assert_allclose(oracle.graph_avg_degree(ns, ne), 1.8)
