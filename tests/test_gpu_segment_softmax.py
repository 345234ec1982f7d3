"""GPU parity of the segment softmax (drop-in for _sparse_softmax,
geoembodied/nn/modules/invariant_attention.py:202-230) against the float64 oracle.

Bars: float32 |w - ref| <= 2e-6 + 1e-5 |ref| (exp and division are correctly rounded or within
a few ulp; the segment sum adds deg roundings); float64 1e-12 relative; the backward likewise
against the oracle's analytic gradient, which test_oracle.py pins to torch autograd of the
reference's op sequence.
"""

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _ops():
    import geoembodied  # noqa: F401
    from geoembodied.functional.segment_softmax import segment_softmax, sparse_softmax
    return segment_softmax, sparse_softmax


def _check(got, ref, dtype):
    got = got.detach().cpu().double().numpy()
    if dtype == torch.float64:
        np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-15)
    else:
        assert np.all(np.abs(got - ref) <= 2e-6 + 1e-5 * np.abs(ref)), float(np.max(np.abs(got - ref)))


@pytest.mark.parametrize("E,N,H", [(1, 1, 1), (500, 40, 1), (3000, 200, 4), (20000, 3000, 8),
                                   (70000, 4000, 3)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_sparse_softmax_vs_oracle(dev, E, N, H, dtype):
    _, sparse_softmax = _ops()
    g = torch.Generator().manual_seed(E + H)
    index = torch.randint(0, N, (E,), generator=g)
    x = (torch.randn(E, H, generator=g, dtype=torch.float64) * 4).to(dtype)
    xg = x.to(dev).requires_grad_(True)
    w = sparse_softmax(xg, index.to(dev), N)
    assert w.shape == (E, H) and w.dtype == dtype
    ref = oracle.sparse_softmax(x.double().numpy(), index.numpy(), N)
    _check(w, ref, dtype)
    gr = torch.randn(E, H, generator=g, dtype=torch.float64).to(dtype)
    w.backward(gr.to(dev))
    want = oracle.sparse_softmax_bwd(gr.double().numpy(), w.detach().cpu().double().numpy(),
                                     index.numpy(), N)
    _check(xg.grad, want, dtype)


def test_segment_softmax_csr_identity_perm_and_1d(dev):
    segment_softmax, _ = _ops()
    deg = torch.tensor([3, 0, 1, 5, 2])
    ne = deg.cumsum(0).int()
    ns = ne - deg.int()
    E = int(deg.sum())
    index = torch.repeat_interleave(torch.arange(5), deg)
    x = torch.randn(E, dtype=torch.float64)
    w = segment_softmax(x.to(dev), None, ns.to(dev), ne.to(dev), 5)
    assert w.shape == (E,)
    _check(w, oracle.sparse_softmax(x.numpy(), index.numpy(), 5), torch.float64)


def test_softmax_special_values_and_unlisted_rows(dev):
    _, sparse_softmax = _ops()
    x = torch.tensor([[1.0], [float("nan")], [2.0], [float("-inf")], [0.5], [float("inf")], [3.0]])
    index = torch.tensor([0, 0, 1, 1, 2, 3, 3])
    w = sparse_softmax(x.to(dev), index.to(dev), 5).cpu().numpy()
    ref = oracle.sparse_softmax(x.double().numpy(), index.numpy(), 5)
    np.testing.assert_array_equal(np.isnan(w), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_allclose(w[ok], ref[ok], rtol=1e-6)
    # rows of edges outside every segment are 0 (the CSR build sorts them last)
    from gdl_amd.csrc import segment_softmax_forward_hip
    ns = torch.tensor([0, 2], dtype=torch.int32, device=dev)
    ne = torch.tensor([2, 3], dtype=torch.int32, device=dev)
    out = segment_softmax_forward_hip(torch.ones(5, 2, device=dev), None, ns, ne, 2)
    assert out.cpu().tolist() == [[0.5, 0.5], [0.5, 0.5], [1.0, 1.0], [0.0, 0.0], [0.0, 0.0]]


@pytest.mark.parametrize("H,dtype", [(1, torch.float32), (2, torch.float32), (4, torch.float32),
                                     (8, torch.float32), (3, torch.float32), (12, torch.float32),
                                     (4, torch.float64)])
def test_sparse_softmax_out_of_range_targets_zero_without_fill(dev, H, dtype):
    """sparse_softmax allocates its output and gradient unfilled: the kernels themselves write 0
    to the rows of targets outside [0, N) (the CSR build sorts them after the last segment), on
    every kernel path (vector rows, runtime-H rows, one thread per head, float64); with N = 0
    every row is such a row."""
    _, sparse_softmax = _ops()
    E, N = 5000, 300
    g = torch.Generator().manual_seed(H)
    index = torch.randint(0, N, (E,), generator=g)
    index[::37] = -1
    index[5::41] = N + 3
    valid = ((index >= 0) & (index < N)).numpy()
    x = (torch.randn(E, H, generator=g, dtype=torch.float64) * 3).to(dtype)
    gr = torch.randn(E, H, generator=g, dtype=torch.float64).to(dtype)
    for n_nodes in (N, 0):
        xg = x.to(dev).requires_grad_(True)
        w = sparse_softmax(xg, index.to(dev), n_nodes)
        w.backward(gr.to(dev))
        ref = np.zeros((E, H))
        want = np.zeros((E, H))
        if n_nodes:
            ref[valid] = oracle.sparse_softmax(x.double().numpy()[valid], index.numpy()[valid], N)
            want[valid] = oracle.sparse_softmax_bwd(gr.double().numpy()[valid],
                                                    w.detach().cpu().double().numpy()[valid],
                                                    index.numpy()[valid], N)
        _check(w, ref, dtype)
        _check(xg.grad, want, dtype)
        assert np.all(w.detach().cpu().numpy()[~valid] == 0)


def test_softmax_bf16_input_promoted(dev):
    _, sparse_softmax = _ops()
    x = torch.randn(1000, 2).bfloat16()
    index = torch.randint(0, 50, (1000,))
    w = sparse_softmax(x.to(dev), index.to(dev), 50)
    assert w.dtype == torch.float32
    _check(w, oracle.sparse_softmax(x.double().numpy(), index.numpy(), 50), torch.float32)


def test_softmax_gradcheck_fp64(dev):
    _, sparse_softmax = _ops()
    g = torch.Generator().manual_seed(1)
    index = torch.randint(0, 7, (40,), generator=g).to(dev)
    x = torch.randn(40, 2, generator=g, dtype=torch.float64).to(dev).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda t: sparse_softmax(t, index, 7), (x,))


@pytest.mark.parametrize("H", [1, 2, 4, 8])
@pytest.mark.parametrize("short", [False, True])
def test_segment_softmax_vector_rows_long_segments(dev, H, short):
    """Head counts with vector-row kernels, forward and backward, shuffled permutation.
    short=False: segments of 0..100 edges (average 50: 16 lanes per segment, chunks past the
    second re-read from memory).  short=True: mostly 0..8 edges with every 25th segment 33..70
    long (average <= 12: 8 lanes per segment, chunks past the fourth re-read)."""
    from gdl_amd.csrc import segment_softmax_backward_hip, segment_softmax_forward_hip
    g = torch.Generator().manual_seed(40 + H + 100 * short)
    N = 700
    if short:
        deg = torch.randint(0, 9, (N,), generator=g)
        deg[::25] = torch.randint(33, 71, (deg[::25].numel(),), generator=g)
        assert int(deg.sum()) <= 12 * N
    else:
        deg = torch.randint(0, 101, (N,), generator=g)
    deg[::7] = 0
    index = torch.repeat_interleave(torch.arange(N), deg)
    E = index.numel()
    sh = torch.randperm(E, generator=g)
    index = index[sh]
    x = torch.randn(E, H, generator=g) * 3
    x[5 % E, 0] = float("nan")
    order = torch.sort(index, stable=True).indices
    cnt = torch.bincount(index, minlength=N)
    ne = cnt.cumsum(0).int()
    ns = (ne - cnt.int())
    pm = order.int().to(dev)
    w = segment_softmax_forward_hip(x.to(dev), pm, ns.to(dev), ne.to(dev), N)
    ref = oracle.sparse_softmax(x.double().numpy(), index.numpy(), N)
    got = w.cpu().double().numpy()
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.all(np.abs(got[ok] - ref[ok]) <= 2e-6 + 1e-5 * np.abs(ref[ok]))
    gr = torch.randn(E, H, generator=g)
    dx = segment_softmax_backward_hip(gr.to(dev), w, pm, ns.to(dev), ne.to(dev), N)
    want = oracle.sparse_softmax_bwd(gr.double().numpy(), got, index.numpy(), N)
    got_dx = dx.cpu().double().numpy()
    fin = np.isfinite(want)
    assert np.all(np.abs(got_dx[fin] - want[fin]) <= 2e-6 + 1e-5 * np.abs(want[fin]))


def test_segment_softmax_misaligned_rows_match_aligned(dev):
    """Rows not aligned to the vector width take the runtime-H kernel (16 lanes per segment;
    the aligned rows here take 8): both within the oracle bar and within a few ulp of each
    other."""
    from gdl_amd.csrc import segment_softmax_forward_hip
    g = torch.Generator().manual_seed(3)
    E, N, H = 5000, 600, 4
    index = torch.sort(torch.randint(0, N, (E,), generator=g)).values
    cnt = torch.bincount(index, minlength=N)
    ne = cnt.cumsum(0).int().to(dev)
    ns = ne - cnt.int().to(dev)
    x = torch.randn(E, H, generator=g).to(dev)
    buf = torch.empty(E * H + 1, device=dev)
    buf[1:] = x.reshape(-1)
    xm = buf[1:].view(E, H)
    assert xm.data_ptr() % 16 != 0
    a = segment_softmax_forward_hip(x, None, ns, ne, N)
    b = segment_softmax_forward_hip(xm, None, ns, ne, N)
    ref = oracle.sparse_softmax(x.cpu().double().numpy(), index.numpy(), N)
    _check(a, ref, torch.float32)
    _check(b, ref, torch.float32)
    torch.testing.assert_close(a, b, rtol=1e-6, atol=1e-7)


def _contiguous_case(g, N, deg, H, tail):
    """Shuffled edges with target degrees ``deg`` plus ``tail`` edges whose target is N (outside
    every segment: the CSR puts them after the last one); perm = stable sort by target."""
    index = torch.cat([torch.repeat_interleave(torch.arange(N), deg),
                       torch.full((tail,), N, dtype=torch.int64)])
    index = index[torch.randperm(index.numel(), generator=g)]
    perm = torch.sort(index, stable=True).indices
    cnt = torch.bincount(index[index < N], minlength=N)
    ne = cnt.cumsum(0).int()
    ns = ne - cnt.int()
    x = torch.randn(index.numel(), H, generator=g) * 3
    return index, perm, ns, ne, x


@pytest.mark.parametrize("H", [1, 2, 4, 8])
@pytest.mark.parametrize("kind", ["graph", "long", "bad_perm"])
def test_segment_softmax_contiguous_csr_short_segments(dev, H, kind):
    """A contiguous CSR whose segments average at most 12 edges (a radius graph's: 8 lanes per
    segment), called with contiguous_csr=True, so the kernel writes the rows after the last
    segment itself and its permutation entries are loaded together before they are checked.
    graph: degrees 0..20, a NaN score, edges after the last segment (written as 0).
    long: short segments with some of 600..1200 edges (chunks past the fourth re-read).
    bad_perm: permutation entries outside [0, E) at some positions: those are skipped."""
    from gdl_amd.csrc import segment_softmax_forward_hip
    g = torch.Generator().manual_seed(7 + 11 * H + len(kind))
    N = 4000
    if kind == "long":
        deg = torch.randint(0, 8, (N,), generator=g)
        deg[0::320] = torch.randint(600, 1201, (deg[0::320].numel(),), generator=g)
        deg[45::300] = torch.randint(600, 1201, (deg[45::300].numel(),), generator=g)
    else:
        deg = torch.randint(0, 21, (N,), generator=g)
    deg[3::17] = 0
    tail = 0 if kind == "bad_perm" else 333
    index, perm, ns, ne, x = _contiguous_case(g, N, deg, H, tail)
    E = index.numel()
    assert E - tail <= 12 * N
    x[int(perm[int(ns[5])]), 0] = float("nan")
    pos_ok = torch.ones(E, dtype=torch.bool)
    if kind == "bad_perm":
        bad = torch.randperm(E, generator=g)[:E // 50]
        pos_ok[bad] = False
        perm_dev = perm.clone()
        perm_dev[bad[0::2]] = -1
        perm_dev[bad[1::2]] = E + 5
    else:
        perm_dev = perm
    w = segment_softmax_forward_hip(x.to(dev), perm_dev.int().to(dev), ns.to(dev), ne.to(dev), N,
                                    contiguous_csr=True).cpu().double().numpy()
    seg_of_pos = torch.sort(index, stable=True).values
    use = pos_ok & (seg_of_pos < N)
    rows = perm[use]
    ref = oracle.sparse_softmax(x[rows].double().numpy(), seg_of_pos[use].numpy(), N)
    got = w[rows.numpy()]
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.all(np.abs(got[ok] - ref[ok]) <= 2e-6 + 1e-5 * np.abs(ref[ok]))
    if tail:
        assert np.all(w[perm[seg_of_pos >= N].numpy()] == 0)


@pytest.mark.parametrize("H", [1, 4])
def test_sparse_softmax_of_radius_graph_targets(dev, H):
    """sparse_softmax over a radius graph's own target tensor takes the graph's row pointer as the
    CSR (identity permutation, no CSR build): bit-identical to the same targets through the CSR
    build, forward and backward, and against the oracle; an in-place change of the targets
    drops back to the CSR build."""
    from gdl_amd.csrc import target_bounds
    from gdl_amd.functional.radius_graph import radius_graph
    _, sparse_softmax = _ops()
    g = torch.Generator().manual_seed(3)
    pos = torch.rand(3000, 3, generator=g).to(dev)
    row, col = radius_graph(pos, 0.08, max_num_neighbors=20)
    N, E = pos.shape[0], col.numel()
    assert target_bounds(col, N) is not None and target_bounds(col.clone(), N) is None
    x = torch.randn(E, H, generator=g, dtype=torch.float64).float().to(dev)
    xa = x.clone().requires_grad_(True)
    xb = x.clone().requires_grad_(True)
    wa = sparse_softmax(xa, col, N)
    wb = sparse_softmax(xb, col.clone(), N)
    assert torch.equal(wa, wb)
    gr = torch.randn(E, H, generator=g).to(dev)
    wa.backward(gr)
    wb.backward(gr)
    assert torch.equal(xa.grad, xb.grad)
    _check(wa, oracle.sparse_softmax(x.double().cpu().numpy(), col.cpu().numpy(), N), torch.float32)
    col_mod = col
    col_mod[0] = col_mod[-1]  # in place: the cached row pointer no longer describes it
    assert target_bounds(col_mod, N) is None
    w2 = sparse_softmax(x, col_mod, N)
    assert torch.equal(w2, sparse_softmax(x, col_mod.clone(), N))
