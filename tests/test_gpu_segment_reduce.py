"""GPU parity: CSR build and segment sum / mean / max (forward and backward) vs the oracle.

Bars: CSR arrays, segment max values + argmax records and every backward value bit-exact;
sum / mean within 1e-5 * sum|msg| (fp32), 2e-2 * sum|msg| (bf16), 1e-12 * sum|msg| (fp64)
per element.  Also restates the reference's own segment-reduce tests
(tests/test_segment_reduce.py:34-159).
"""

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float64: 1e-12}
NP_DT = {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float64: "float64"}


def _ops():
    import geoembodied  # noqa: F401
    from geoembodied.functional.segment_reduce import segment_reduce, sort_and_build_csr
    return segment_reduce, sort_and_build_csr


def _problem(E, N, C, dtype, seed, ties=False, sorted_col=False):
    g = torch.Generator().manual_seed(seed)
    col = torch.randint(0, max(N, 1), (E,), generator=g)
    if sorted_col:
        col = col.sort().values
    msg = torch.randn(E, C, generator=g, dtype=torch.float64)
    if ties:
        msg = (msg * 2).round() / 2  # few distinct values -> many tied maxima
    return col, msg.to(dtype)


def _np(t):
    return t.detach().cpu().float().numpy() if t.dtype == torch.bfloat16 else t.detach().cpu().numpy()


# ----------------------------------------------------------------------------- CSR build ---

@pytest.mark.parametrize("E,N,seed", [(1, 1, 0), (1000, 10, 1), (5000, 300, 2), (70000, 70000, 3),
                                      (200000, 5000, 4), (300000, 20_000_000, 5),
                                      # either side of the one-workgroup path (E <= 2048, N <= 16384)
                                      (2048, 16384, 6), (2049, 16384, 7), (2048, 16385, 8),
                                      (2048, 3, 9)])
def test_csr_matches_oracle(dev, E, N, seed):
    _, csr = _ops()
    g = torch.Generator().manual_seed(seed)
    col = torch.randint(0, N, (E,), generator=g)
    if E > 10:
        col[::97] = -3          # out-of-range targets sort last
        col[5::101] = N + 7
    cs, pm, ns, ne = csr(col.to(dev), N)
    r = oracle.sort_and_build_csr(col.numpy(), N)
    for got, want, name in zip((cs, pm, ns, ne), r, ("col_sorted", "perm", "node_start", "node_end")):
        assert got.dtype == torch.int32, name
        np.testing.assert_array_equal(got.cpu().numpy(), want, err_msg=name)


@pytest.mark.parametrize("kind", ["sorted", "sorted_invalid_last", "invalid_first", "one_descent",
                                  "constant", "reversed"])
@pytest.mark.parametrize("E,N", [(3000, 500), (200000, 300000)])   # one and two radix passes
def test_csr_sorted_input_detection(dev, kind, E, N):
    """Targets that arrive sorted take the identity path (one pass); anything out of order, however
    little, takes the full sort.  Both must give the oracle's stable CSR."""
    _, csr = _ops()
    g = torch.Generator().manual_seed(E + len(kind))
    col = torch.sort(torch.randint(0, N, (E,), generator=g)).values
    if kind == "sorted_invalid_last":
        col[-7:] = N + 3               # clamped to N: still sorted
    elif kind == "invalid_first":
        col[0] = -1                    # clamped to N at the front: out of order
    elif kind == "one_descent":
        i = E // 2 + 5
        col[i] = col[i - 1] - 1 if col[i - 1] > 0 else col[i]
        col[i - 1] = col[i - 1] if col[i - 1] > 0 else N - 1
    elif kind == "constant":
        col[:] = N // 2
    elif kind == "reversed":
        col = col.flip(0)
    cs, pm, ns, ne = csr(col.to(dev), N)
    r = oracle.sort_and_build_csr(col.numpy(), N)
    for got, want, name in zip((cs, pm, ns, ne), r, ("col_sorted", "perm", "node_start", "node_end")):
        np.testing.assert_array_equal(got.cpu().numpy(), want, err_msg=name)


@pytest.mark.parametrize("E,N,seed", [(4_194_304, 262_144, 11),      # C3 size, two passes
                                      (1_000_000, 1_000, 12),        # ~1000 equal keys per target
                                      (500_000, 40_000_000, 13),     # 26-bit keys, three passes
                                      (4097, 5_000, 14), (12_289, 2, 15)])  # ragged last tiles
@pytest.mark.parametrize("order", ["shuffled", "sorted"])
def test_csr_radix_paths(dev, E, N, seed, order):
    """The multi-tile radix sort (look-back over 4096-key tiles) and the identity path of sorted
    input, on sizes that give one, two and three digit passes, partial last tiles and targets
    sparser than the edges (whose node bounds fall back to a binary search)."""
    _, csr = _ops()
    g = torch.Generator().manual_seed(seed)
    col = torch.randint(0, N, (E,), generator=g)
    if order == "sorted":
        col = col.sort().values
    cs, pm, ns, ne = csr(col.to(dev), N)
    r = oracle.sort_and_build_csr(col.numpy(), N)
    for got, want, name in zip((cs, pm, ns, ne), r, ("col_sorted", "perm", "node_start", "node_end")):
        np.testing.assert_array_equal(got.cpu().numpy(), want, err_msg=name)


@pytest.mark.parametrize("gaps", [(4, 5), (64, 65), (4096, 4097), (4160, 20_000), (1, 300_000)])
def test_csr_sorted_gaps(dev, gaps):
    """Sorted targets with runs of empty nodes between them: gaps of up to four nodes are written
    by one thread, longer ones by the whole wave, and a wave whose long gaps exceed its budget of
    64 steps of 64 nodes hands every bound to the binary-search kernel."""
    _, csr = _ops()
    g = torch.Generator().manual_seed(sum(gaps))
    E = 60_000
    step = torch.randint(0, 2, (E,), generator=g)            # 0 or 1: repeats and unit steps
    big = torch.randint(0, E, (40,), generator=g)
    step[big] = torch.tensor(gaps)[torch.arange(40) % 2]     # a few long runs of empty nodes
    col = torch.cumsum(step, 0)
    N = int(col[-1]) + gaps[1]                               # empty nodes after the last target too
    cs, pm, ns, ne = csr(col.to(dev), N)
    r = oracle.sort_and_build_csr(col.numpy(), N)
    for got, want, name in zip((cs, pm, ns, ne), r, ("col_sorted", "perm", "node_start", "node_end")):
        np.testing.assert_array_equal(got.cpu().numpy(), want, err_msg=name)


def test_csr_of_radius_graph_targets(dev):
    """The targets of a radius graph are already in CSR order: their CSR build comes from the
    graph's row pointer.  It must equal the oracle's stable CSR; a different node count, or the
    targets changed in place, take the sort instead and still match the oracle."""
    import geoembodied  # noqa: F401
    from geoembodied.functional.radius_graph import radius_graph
    _, csr = _ops()
    g = torch.Generator().manual_seed(21)
    pos = torch.rand(3000, 3, generator=g)
    row, col = radius_graph(pos.to(dev), 0.12, max_num_neighbors=16)
    N = pos.shape[0]
    for n_nodes in (N, N + 5):
        got = csr(col, n_nodes)
        want = oracle.sort_and_build_csr(col.cpu().numpy(), n_nodes)
        for g_, w_, name in zip(got, want, ("col_sorted", "perm", "node_start", "node_end")):
            np.testing.assert_array_equal(g_.cpu().numpy(), w_, err_msg=f"{name} N={n_nodes}")
    col[0] = N - 1          # in place: no longer the graph's targets, nor sorted
    got = csr(col, N)
    want = oracle.sort_and_build_csr(col.cpu().numpy(), N)
    for g_, w_, name in zip(got, want, ("col_sorted", "perm", "node_start", "node_end")):
        np.testing.assert_array_equal(g_.cpu().numpy(), w_, err_msg=f"{name} after in-place change")


def test_csr_empty(dev):
    _, csr = _ops()
    cs, pm, ns, ne = csr(torch.empty(0, dtype=torch.long, device=dev), 7)
    assert cs.numel() == 0 and pm.numel() == 0
    assert ns.tolist() == [0] * 7 and ne.tolist() == [0] * 7


# ------------------------------------------------------------------------- forward / bwd ---

CASES = [
    # E, N, C, dtype
    (3000, 500, 32, torch.float32),
    (4000, 300, 1, torch.float32),
    (4000, 300, 3, torch.float32),
    (5000, 700, 112, torch.float32),
    (5000, 256, 128, torch.float32),
    (3000, 200, 300, torch.float32),
    (5000, 700, 128, torch.bfloat16),
    (4000, 300, 7, torch.bfloat16),
    (3000, 400, 64, torch.float64),
    (2000, 100, 5, torch.float64),
]


@pytest.mark.parametrize("E,N,C,dtype", CASES)
@pytest.mark.parametrize("reduce", ["sum", "mean", "max"])
def test_forward_backward_vs_oracle(dev, E, N, C, dtype, reduce):
    seg, csr = _ops()
    col, msg = _problem(E, N, C, dtype, seed=E + C, ties=reduce == "max")
    cs, pm, ns, ne = csr(col.to(dev), N)
    m = msg.to(dev).requires_grad_(True)
    out = seg(m, cs, pm, ns, ne, N, reduce=reduce)
    assert out.shape == (N, C) and out.dtype == dtype
    ref, aux = oracle.segment_reduce_fwd(_np(msg), pm.cpu().numpy(), ns.cpu().numpy(),
                                         ne.cpu().numpy(), N, reduce)
    got = _np(out).astype(np.float64)
    if reduce == "max":
        np.testing.assert_array_equal(got, ref)
    else:
        bound = TOL[dtype] * aux + 1e-30
        if dtype == torch.bfloat16:
            bound = bound + np.abs(ref) * 2.0 ** -8  # final rounding to bf16
        assert np.all(np.abs(got - ref) <= bound), float(np.max(np.abs(got - ref) - bound))
    grad = torch.randn(N, C, generator=torch.Generator().manual_seed(7), dtype=torch.float64).to(dtype)
    out.backward(grad.to(dev))
    from gdl_amd.csrc import segment_reduce_forward_hip
    arg = None
    if reduce == "max":
        _, arg_t = segment_reduce_forward_hip(msg.to(dev), pm, ns, ne, N, "max")
        np.testing.assert_array_equal(arg_t.cpu().numpy(), aux)
        arg = aux
    want = oracle.segment_reduce_bwd(_np(grad), cs.cpu().numpy(), pm.cpu().numpy(),
                                     ns.cpu().numpy(), ne.cpu().numpy(), E, reduce,
                                     msg=_np(msg), out=ref, arg=arg, dtype=NP_DT[dtype])
    np.testing.assert_array_equal(_np(m.grad).astype(np.float64), want)


def test_max_first_mode_and_identity_perm(dev):
    seg, _ = _ops()
    from gdl_amd.csrc import segment_reduce_forward_hip
    E, N, C = 3000, 200, 16
    col, msg = _problem(E, N, C, torch.float32, 11, ties=True, sorted_col=True)
    counts = torch.bincount(col, minlength=N)
    ne = counts.cumsum(0).int()
    ns = ne - counts.int()
    perm = torch.arange(E, dtype=torch.int32)
    out, arg = segment_reduce_forward_hip(msg.to(dev), None, ns.to(dev), ne.to(dev), N, "max", 1)
    ref, aux = oracle.segment_reduce_fwd(msg.numpy(), perm.numpy(), ns.numpy(), ne.numpy(), N, "max",
                                         tie_mode=1)
    np.testing.assert_array_equal(out.cpu().numpy(), ref)
    np.testing.assert_array_equal(arg.cpu().numpy(), aux)
    m = msg.to(dev).requires_grad_(True)
    o = seg(m, col.int().to(dev), perm.to(dev), ns.to(dev), ne.to(dev), N, reduce="max", max_ties="first")
    o.sum().backward()
    g = m.grad.cpu()
    # each non-empty (segment, channel) routes exactly one unit of gradient
    assert g.sum().item() == float((counts > 0).sum().item() * C)


def test_empty_segments_and_special_values(dev):
    seg, csr = _ops()
    N, C = 6, 4
    col = torch.tensor([1, 1, 3, 3, 3])
    msg = torch.tensor([[-0.0, 1.0, float("nan"), -float("inf")],
                        [0.0, 1.0, 2.0, -float("inf")],
                        [5.0, -1.0, 2.0, 3.0],
                        [5.0, -2.0, float("nan"), 3.0],
                        [4.0, -1.0, 1.0, 3.0]])
    cs, pm, ns, ne = csr(col.to(dev), N)
    for red in ("sum", "mean", "max"):
        out = seg(msg.to(dev), cs, pm, ns, ne, N, reduce=red).cpu()
        assert torch.all(out[[0, 2, 4, 5]] == 0), red
    out = seg(msg.to(dev), cs, pm, ns, ne, N, reduce="max").cpu()
    ref, _ = oracle.segment_reduce_fwd(msg.numpy(), pm.cpu().numpy(), ns.cpu().numpy(),
                                       ne.cpu().numpy(), N, "max")
    np.testing.assert_array_equal(out.numpy().view(np.uint32), ref.astype(np.float32).view(np.uint32))


# ----------------------------------------------- reference tests restated (test_segment_reduce) ---

def test_matches_scatter_add(dev):
    seg, csr = _ops()
    torch.manual_seed(42)
    N, E, C = 500, 3000, 32
    col = torch.randint(0, N, (E,), device=dev)
    msg = torch.randn(E, C, device=dev)
    ref = torch.zeros(N, C, device=dev).scatter_add_(0, col.unsqueeze(-1).expand(E, C), msg)
    out = seg(msg, *csr(col, N), N)
    assert torch.allclose(out, ref, atol=1e-5)


def test_bit_exact_determinism(dev):
    seg, csr = _ops()
    torch.manual_seed(0)
    N, E, C = 100, 500, 8
    col = torch.randint(0, N, (E,), device=dev)
    msg = torch.randn(E, C, device=dev)
    args = csr(col, N)
    ref = seg(msg, *args, N)
    for _ in range(19):
        assert torch.equal(seg(msg, *args, N), ref)


def test_backward_ones(dev):
    seg, csr = _ops()
    torch.manual_seed(42)
    N, E, C = 50, 200, 8
    col = torch.randint(0, N, (E,), device=dev)
    msg = torch.randn(E, C, device=dev, requires_grad=True)
    seg(msg, *csr(col, N), N).sum().backward()
    assert torch.equal(msg.grad, torch.ones_like(msg))


@pytest.mark.parametrize("reduce", ["sum", "mean", "max"])
def test_gradcheck_fp64(dev, reduce):
    seg, csr = _ops()
    torch.manual_seed(3)
    N, E, C = 10, 30, 4
    col = torch.randint(0, N, (E,), device=dev)
    args = csr(col, N)
    msg = torch.randn(E, C, device=dev, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda m: seg(m, *args, N, reduce=reduce), (msg,), atol=1e-6)


def test_empty_edges(dev):
    seg, csr = _ops()
    N, C = 10, 8
    out = seg(torch.empty(0, C, device=dev), *csr(torch.empty(0, dtype=torch.long, device=dev), N), N)
    assert out.shape == (N, C) and out.abs().sum() == 0


def test_single_node(dev):
    seg, csr = _ops()
    E, C = 10, 4
    out = seg(torch.ones(E, C, device=dev), *csr(torch.zeros(E, dtype=torch.long, device=dev), 1), 1)
    assert torch.equal(out, torch.full((1, C), float(E), device=dev))


@pytest.mark.parametrize("C", [1, 16, 32, 64])
def test_channel_widths(dev, C):
    seg, csr = _ops()
    torch.manual_seed(C)
    N, E = 30, 150
    col = torch.randint(0, N, (E,), device=dev)
    msg = torch.randn(E, C, device=dev)
    ref = torch.zeros(N, C, device=dev).scatter_add_(0, col.unsqueeze(-1).expand(E, C), msg)
    assert torch.allclose(seg(msg, *csr(col, N), N), ref, atol=1e-4)


def test_mean_and_max_match_reference_call_sites(dev):
    """mean == global_mean_pool (scatter_add / bincount.clamp(1)); max == scatter_reduce amax
    with include_self=False on zeros; both with fp32 inputs (nn/modules/se3_net.py:226-270,
    nn/modules/invariant_attention.py:212-219)."""
    seg, csr = _ops()
    torch.manual_seed(5)
    N, E, C = 64, 900, 24
    col = torch.randint(0, N - 4, (E,), device=dev)  # last 4 targets empty
    msg = torch.randn(E, C, device=dev)
    args = csr(col, N)
    s = torch.zeros(N, C, device=dev).scatter_add_(0, col.unsqueeze(1).expand(E, C), msg)
    mean_ref = s / torch.bincount(col, minlength=N).clamp(min=1).unsqueeze(1)
    assert torch.allclose(seg(msg, *args, N, reduce="mean"), mean_ref, atol=1e-5)
    mx_ref = torch.zeros(N, C, device=dev).scatter_reduce_(0, col.unsqueeze(1).expand(E, C), msg,
                                                           reduce="amax", include_self=False)
    assert torch.equal(seg(msg, *args, N, reduce="max"), mx_ref)
    # gradient of max with ties split evenly, as scatter_reduce's backward.  Values sit on a
    # 0.5 grid offset by 0.25 so that no segment maximum is exactly 0: for such segments
    # PyTorch's backward also counts the zero-initialised output as a tie (grad / (count + 1)),
    # which this implementation deliberately does not reproduce.
    mt = ((msg * 2).round() / 2 + 0.25).requires_grad_(True)
    mr = mt.detach().clone().requires_grad_(True)
    g = torch.randn(N, C, device=dev)
    seg(mt, *args, N, reduce="max").backward(g)
    torch.zeros(N, C, device=dev).scatter_reduce(0, col.unsqueeze(1).expand(E, C), mr,
                                                 reduce="amax", include_self=False).backward(g)
    assert torch.allclose(mt.grad, mr.grad, atol=1e-6)


def test_max_backward_exact_zero_maximum_differs_from_torch_by_design(dev):
    """The one deliberate difference from the reference's scatter_reduce('amax',
    include_self=False) on a zero-initialised output: when a segment's maximum is exactly 0.0,
    PyTorch's backward also counts the initial 0 of the output as a tied maximum and gives each
    tied input grad / (count + 1); this build gives grad / count (the gradient of the inputs'
    maximum).  Segments whose maximum is not 0 agree exactly."""
    seg, csr = _ops()
    vals = torch.tensor([0.0, -1.0, 0.0,      # segment 0: maximum 0 attained twice
                         0.0, -2.0,           # segment 1: maximum 0 attained once
                         0.5, 0.5, -3.0,      # segment 2: maximum 0.5, two ties
                         -0.0, -4.0],         # segment 3: maximum -0.0 (equal to 0)
                        device=dev).unsqueeze(1)
    col = torch.tensor([0, 0, 0, 1, 1, 2, 2, 2, 3, 3], device=dev)
    g = torch.tensor([[6.0], [4.0], [2.0], [8.0]], device=dev)
    ours = vals.clone().requires_grad_(True)
    seg(ours, *csr(col, 4), 4, reduce="max").backward(g)
    ref = vals.clone().requires_grad_(True)
    torch.zeros(4, 1, device=dev).scatter_reduce(0, col.unsqueeze(1), ref, reduce="amax",
                                                 include_self=False).backward(g)
    want_ours = [3.0, 0.0, 3.0, 4.0, 0.0, 1.0, 1.0, 0.0, 8.0, 0.0]
    want_torch = [2.0, 0.0, 2.0, 2.0, 0.0, 1.0, 1.0, 0.0, 4.0, 0.0]
    assert ours.grad.squeeze(1).tolist() == want_ours
    assert ref.grad.squeeze(1).tolist() == want_torch


# ------------------------------------------------------------- many-segment forward path ---
# S >= 4096 segments of average length <= 128 take the merge-path kernel: a wave's rows are
# split evenly over its lane groups, so segments cross group boundaries and are completed from
# partial results.  Layouts cover every group count R = 64 / L from 1 to 64.

MERGE_LAYOUTS = [  # C, dtype  (lanes per row L)
    (1, torch.float32),      # L = 1, R = 64
    (3, torch.float32),      # L = 4
    (32, torch.float32),     # L = 8
    (128, torch.float32),    # L = 32
    (300, torch.float32),    # L = 64, two column passes
    (128, torch.bfloat16),   # L = 16
    (7, torch.bfloat16),     # L = 8, 2-byte vectors
    (64, torch.float64),     # L = 32
]


def _merge_sizes(kind, S, rng):
    if kind == "zipf":
        sz = np.minimum(rng.zipf(1.3, S), 64)
        sz[rng.random(S) < 0.4] = 0
    elif kind == "long":   # a few segments spanning many groups and waves' worth of rows
        sz = rng.integers(0, 6, S)
        sz[rng.choice(S, 8, replace=False)] = rng.integers(300, 3000, 8)
    else:                  # "ones": every segment a single row
        sz = np.ones(S, dtype=np.int64)
    return sz.astype(np.int64)


@pytest.mark.parametrize("C,dtype", MERGE_LAYOUTS)
@pytest.mark.parametrize("kind", ["zipf", "long", "ones"])
@pytest.mark.parametrize("reduce", ["sum", "mean", "max"])
def test_merge_path_vs_oracle(dev, C, dtype, kind, reduce):
    from gdl_amd.csrc import segment_reduce_forward_hip
    rng = np.random.default_rng(C * 7 + len(kind))
    S = 6000
    sz = _merge_sizes(kind, S, rng)
    ne = np.cumsum(sz)
    ns = ne - sz
    E = int(ne[-1])
    assert E <= 128 * S
    perm = rng.permutation(E).astype(np.int32)
    msg = torch.from_numpy(rng.standard_normal((E, C)))
    if reduce == "max":
        msg = (msg * 2).round() / 2
    msg = msg.to(dtype)
    for p in (perm, None):
        out, arg = segment_reduce_forward_hip(
            msg.to(dev), None if p is None else torch.from_numpy(p).to(dev),
            torch.from_numpy(ns.astype(np.int32)).to(dev),
            torch.from_numpy(ne.astype(np.int32)).to(dev), S, reduce)
        ref, aux = oracle.segment_reduce_fwd(_np(msg), p, ns, ne, S, reduce)
        got = _np(out).astype(np.float64)
        if reduce == "max":
            np.testing.assert_array_equal(got, ref)
            np.testing.assert_array_equal(arg.cpu().numpy(), aux)
        else:
            bound = TOL[dtype] * aux + 1e-30
            if dtype == torch.bfloat16:
                bound = bound + np.abs(ref) * 2.0 ** -8
            assert np.all(np.abs(got - ref) <= bound), float(np.max(np.abs(got - ref) - bound))


# ------------------------------------------------------------------- full-size C3 properties ---

def test_c3_full_size(dev):
    """C3 at full size: oracle on a sample of segments, linearity and total-sum checks on all."""
    import bench
    seg, _ = _ops()
    off = bench.make_c3_offsets()
    S, E, C = off.shape[0] - 1, int(off[-1]), 128
    ns = torch.from_numpy(off[:-1].astype(np.int32)).to(dev)
    ne = torch.from_numpy(off[1:].astype(np.int32)).to(dev)
    cs = torch.repeat_interleave(torch.arange(S, device=dev, dtype=torch.int32), (ne - ns).long())
    perm = torch.arange(E, device=dev, dtype=torch.int32)
    gen = torch.Generator(device=dev).manual_seed(0)
    msg = torch.randn(E, C, device=dev, generator=gen)
    out = seg(msg, cs, perm, ns, ne, S)
    # sampled oracle comparison
    sample = np.random.default_rng(3).choice(S, 2000, replace=False)
    rows = np.concatenate([np.arange(off[s], off[s + 1]) for s in sample])
    sub = msg[torch.from_numpy(rows).to(dev)].cpu().numpy()
    loc = np.zeros(len(sample) + 1, dtype=np.int64)
    loc[1:] = np.cumsum(off[sample + 1] - off[sample])
    ref, scale = oracle.segment_reduce_fwd(sub, None, loc[:-1], loc[1:], len(sample), "sum")
    got = out[torch.from_numpy(sample).to(dev)].cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got - ref) <= 1e-5 * scale + 1e-30)
    # empty segments are exactly zero
    empty = (ne - ns) == 0
    assert torch.all(out[empty] == 0)
    # column totals: sum over segments == sum over edges (fp64 on both sides)
    tot_seg = out.double().sum(0)
    tot_edge = msg.double().sum(0)
    assert torch.allclose(tot_seg, tot_edge, rtol=0, atol=1e-5 * msg.abs().double().sum(0).max().item())
    # max at full size: exact against torch's segment reduction on the sorted rows
    mx = seg(msg, cs, perm, ns, ne, S, reduce="max")
    ref_mx = torch.segment_reduce(msg, "max", lengths=(ne - ns).long(), unsafe=True)
    ref_mx = torch.where((ne - ns).unsqueeze(1) > 0, ref_mx, torch.zeros_like(ref_mx))
    assert torch.equal(mx, ref_mx)


@pytest.mark.parametrize("reduce,dtype", [("sum", torch.float32), ("mean", torch.float32),
                                          ("max", torch.float32), ("sum", torch.bfloat16),
                                          ("mean", torch.bfloat16), ("max", torch.bfloat16)])
def test_c3_full_size_every_leg(dev, reduce, dtype):
    """Every C3 leg at full size (E = 4,194,304, S = 262,144, C = 128), forward and backward,
    against float64 library routines on the GPU: sum / mean within TOL * sum|msg| of an fp64
    index_add, max and its tie-split backward equal to scatter_reduce('amax') and its autograd
    backward, sum / mean backward equal to the gather formula; the segment order is permuted
    (perm is not the identity) for the mean and max legs."""
    import bench
    from seg_legs import reduce_leg_fp64
    off = bench.make_c3_offsets()
    S, E, C = off.shape[0] - 1, int(off[-1]), 128
    ns = torch.from_numpy(off[:-1].astype(np.int32)).to(dev)
    ne = torch.from_numpy(off[1:].astype(np.int32)).to(dev)
    cs = torch.repeat_interleave(torch.arange(S, device=dev, dtype=torch.int32), (ne - ns).long())
    gen = torch.Generator(device=dev).manual_seed(3)
    if reduce == "sum":
        perm = torch.arange(E, device=dev, dtype=torch.int32)
    else:
        perm = torch.randperm(E, device=dev, generator=gen).to(torch.int32)
    msg = torch.randn(E, C, device=dev, generator=gen).to(dtype)
    grad = torch.randn(S, C, device=dev, generator=gen).to(dtype)
    out = reduce_leg_fp64(msg, cs, perm, ns, ne, S, reduce, grad)
    assert torch.all(out[(ne - ns) == 0] == 0)
