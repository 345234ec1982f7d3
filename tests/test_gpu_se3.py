"""GPU: fused SE3Conv message passing against the float64 oracle (oracle/se3.py, pinned by closed
forms and rotation equivariance in test_oracle_se3.py).

Bars (fp32 arithmetic with the sums reordered: aggregate first, then the weights):
  outputs     |got - want| <= 2e-4 |want| + 2e-5 max|want|
  gradients   |got - want| <= 5e-4 |want| + 5e-5 max|want|     (per tensor)
"""

import numpy as np
import pytest
import torch

from oracle import se3 as ose3

pytestmark = pytest.mark.gpu

SPEC = lambda Cs, Cv, Ct, Os, Ov, Ot: {  # noqa: E731
    "w_ss": (Os, Cs), "w_sv": (Ov, Cs), "w_vv_scalar": (Ov, Cv), "w_vs": (Os, Cv),
    "w_vv_cross": (Ov, Cv), "w_st2": (Ot, Cs), "w_t2t2": (Ot, Ct), "w_vt2": (Ot, Cv), "w_t2s": (Os, Ct)}


def _close(got, want, rtol, arel):
    got = got.detach().double().cpu().numpy()
    want = want.detach().double().cpu().numpy()
    scale = max(float(np.abs(want).max()) if want.size else 0.0, 1e-30)
    np.testing.assert_allclose(got, want, rtol=rtol, atol=arel * scale)


def test_gemm_kernel_vs_torch(dev):
    from gdl_amd.se3_conv import _gemm, _pad64
    g = torch.Generator().manual_seed(0)
    for (N, G, K, O) in [(1000, 1, 80, 64), (333, 3, 96, 16), (257, 5, 48, 23), (64, 1, 16, 100)]:
        A = torch.randn(N * G, K, generator=g)
        B = torch.zeros(_pad64(O), K)
        B[:O] = torch.randn(O, K, generator=g)
        avg = torch.rand(N, generator=g) + 0.5
        bias = torch.randn(O, generator=g) if G == 1 else None
        mask = torch.rand(N, generator=g) > 0.3
        out = torch.full((N, O, G), float("nan"), device=dev)
        _gemm(A.to(dev), N * G, K, B.to(dev), O, G, out, O * G, avg.to(dev),
              None if bias is None else bias.to(dev), mask.to(dev).view(torch.uint8))
        want = (A.double() @ B[:O].double().t()).view(N, G, O).permute(0, 2, 1) / avg.double().view(N, 1, 1)
        if bias is not None:
            want = want + bias.double().view(1, O, 1)
        want = want * mask.double().view(N, 1, 1)
        _close(out, want, 1e-5, 1e-6)


def test_gemm_tn_kernel_vs_torch(dev):
    """Weight-gradient GEMM out[o][k] = sum_r A[r][o] B[r][k] (rows split over up to 512
    workgroups, the four waves of a workgroup added in LDS, partials added in a fixed order):
    O and K off the 16-tiles, several tile groups along O and K, M below one 16-row step, M not a
    multiple of 16, and a long M with strided rows (lda > O, ldb > K)."""
    from gdl_amd import _native as nat
    L = nat.lib()
    g = torch.Generator().manual_seed(5)
    for (M, O, K, lda, ldb) in [(7, 5, 9, 5, 9), (1000, 64, 80, 64, 80), (196611, 16, 96, 20, 100),
                                (5000, 100, 200, 100, 200), (65536, 33, 17, 48, 32), (0, 8, 8, 8, 8)]:
        A = torch.randn(M, lda, generator=g)
        B = torch.randn(M, ldb, generator=g)
        out = torch.full((O, K + 3), float("nan"), device=dev)
        nbytes = L.geo_se3_gemm_tn_workspace_bytes(M, O, K)
        ws = nat.workspace(nbytes, torch.device(dev))
        Ad, Bd = A.to(dev), B.to(dev)
        nat.check(L.geo_se3_gemm_tn(nat.ptr(Ad), M, lda, O, nat.ptr(Bd), ldb, K, nat.ptr(out), K + 3,
                                    nat.ptr(ws), nbytes, nat.stream_of(torch.device(dev))),
                  "geo_se3_gemm_tn")
        want = A[:, :O].double().t() @ B[:, :K].double()
        _close(out[:, :K], want, 1e-5, 1e-6)
        assert torch.isnan(out[:, K:]).all()  # columns past K untouched


def test_gemm_tn_split_writes_each_part_bitwise(dev):
    """geo_se3_gemm_tn_split: the product's column ranges written as separate row-major matrices
    equal the unsplit result bit for bit (same partials, same order); a NULL part is skipped and
    its neighbours' memory is untouched."""
    import ctypes
    from gdl_amd import _native as nat
    L = nat.lib()
    g = torch.Generator().manual_seed(7)
    for (M, O, K, cuts) in [(65536, 64, 112, (0, 64, 80, 112)), (1000, 16, 40, (0, 16, 40)),
                            (333, 5, 9, (0, 9)), (4097, 33, 50, (0, 10, 10, 50))]:
        A = torch.randn(M, O, generator=g).to(dev)
        B = torch.randn(M, K, generator=g).to(dev)
        nbytes = L.geo_se3_gemm_tn_workspace_bytes(M, O, K)
        ws = nat.workspace(nbytes, torch.device(dev))
        st = nat.stream_of(torch.device(dev))
        full = torch.empty(O, K, device=dev)
        nat.check(L.geo_se3_gemm_tn(nat.ptr(A), M, O, O, nat.ptr(B), K, K, nat.ptr(full), K,
                                    nat.ptr(ws), nbytes, st), "geo_se3_gemm_tn")
        n = len(cuts) - 1
        parts = [torch.full((O, cuts[j + 1] - cuts[j]), float("nan"), device=dev) for j in range(n)]
        skip = n - 1 if n > 1 else -1   # the last part of a multi-part split is not requested
        cols = (ctypes.c_int32 * (n + 1))(*cuts)
        outs = (ctypes.c_void_p * n)(*[None if j == skip else parts[j].data_ptr() for j in range(n)])
        nat.check(L.geo_se3_gemm_tn_split(nat.ptr(A), M, O, O, nat.ptr(B), K, K, n, cols, outs,
                                          nat.ptr(ws), nbytes, st), "geo_se3_gemm_tn_split")
        for j in range(n):
            if j == skip:
                assert torch.isnan(parts[j]).all()
            else:
                assert torch.equal(parts[j], full[:, cuts[j]:cuts[j + 1]])


def test_colsum_bias_gradient(dev):
    """geo_se3_colsum: column sums over the unmasked rows (fixed order: bitwise equal on a
    repeat), against a float64 sum; N = 0 gives zeros."""
    from gdl_amd import _native as nat
    L = nat.lib()
    g = torch.Generator().manual_seed(9)
    st = nat.stream_of(torch.device(dev))
    for (N, O, masked) in [(65536, 64, False), (65536, 64, True), (1000, 130, True), (3, 5, False),
                           (0, 7, False)]:
        x = torch.randn(N, O, generator=g)
        mask = (torch.rand(N, generator=g) > 0.3) if masked else None
        xd = x.to(dev)
        md = mask.to(dev).view(torch.uint8) if masked else None
        nbytes = L.geo_se3_colsum_workspace_bytes(N, O)
        ws = nat.workspace(nbytes, torch.device(dev))
        outs = []
        for _ in range(2):
            out = torch.full((O,), float("nan"), device=dev)
            nat.check(L.geo_se3_colsum(nat.ptr(xd), N, O, nat.ptr(md), nat.ptr(out), nat.ptr(ws),
                                       nbytes, st), "geo_se3_colsum")
            outs.append(out)
        assert torch.equal(outs[0], outs[1])
        want = (x.double() * (mask.double().view(N, 1) if masked else 1.0)).sum(0)
        scale = x.abs().double().sum(0).clamp(min=1e-30)
        assert ((outs[0].double().cpu() - want).abs() <= 1e-5 * scale + 1e-30).all()


def _graph(N, B, r, K, seed, shuffle):
    from gdl_amd.graph import SpatialGraph
    g = torch.Generator().manual_seed(seed)
    pos = torch.rand(N * B, 3, generator=g)
    batch = torch.arange(B).repeat_interleave(N)
    gr = SpatialGraph.build(pos.cuda(), r, max_num_neighbors=K, batch=batch.cuda(), num_batch_elements=B)
    if shuffle:
        p = torch.randperm(gr.E, generator=g).cuda()
        gr = SpatialGraph.from_edge_index(gr.row[p], gr.col[p], pos.cuda(), gr.N, batch=batch.cuda(),
                                          num_batch_elements=B)
    return gr


CONFIGS = [
    # Cs, Cv, Ct, Os, Ov, Ot, type2-in, type2-out
    (8, 4, 0, 8, 4, 0),
    (64, 16, 0, 64, 16, 0),
    (80, 20, 6, 70, 10, 4),
    (0, 4, 0, 3, 2, 0),
    (5, 0, 2, 4, 0, 3),
    (12, 6, 0, 10, 5, 3),      # type-2 output from scalars and vectors only
]


def _inputs(cfg, gr, seed, dev):
    Cs, Cv, Ct, Os, Ov, Ot = cfg
    g = torch.Generator().manual_seed(seed)
    N, E = gr.N, gr.E
    s = torch.randn(N, Cs, generator=g)
    v = torch.randn(N, Cv, 3, generator=g)
    t = torch.randn(N, Ct, 5, generator=g) if Ct > 0 else None
    W = {k: (torch.randn(*sh, generator=g) / max(sh[1], 1) ** 0.5 if sh[0] > 0 and sh[1] > 0 else None)
         for k, sh in SPEC(*cfg).items()}
    pc = ose3.path_columns(W, t is not None, True, Ot)
    P = max(sum(1 for x in pc if x >= 0), 1) + 1          # one spare column, as in the module
    R = torch.randn(E, P, generator=g)
    bias = torch.randn(Os, generator=g) if Os > 0 else None
    mask = torch.rand(N, generator=g) > 0.2
    return s, v, t, W, R, bias, mask


@pytest.mark.parametrize("cfg", CONFIGS, ids=[str(c) for c in CONFIGS])
@pytest.mark.parametrize("shuffle", [False, True])
def test_forward_and_gradients_vs_oracle(dev, cfg, shuffle):
    from gdl_amd.se3_conv import se3_message_aggregate
    Cs, Cv, Ct, Os, Ov, Ot = cfg
    gr = _graph(300, 2, 0.22, 24, sum(cfg) + shuffle, shuffle)
    s, v, t, W, R, bias, mask = _inputs(cfg, gr, 1 + shuffle, dev)
    d = gr.direction.detach()
    Y = gr.Y.detach()
    leaves = {"s": s, "v": v, "R": R, "d": d.cpu(), "Y": Y.cpu()}
    if t is not None:
        leaves["t"] = t
    if bias is not None:
        leaves["bias"] = bias
    for k, w in W.items():
        if w is not None:
            leaves[k] = w
    gpu = {k: x.detach().to(dev).requires_grad_(True) for k, x in leaves.items()}
    cpu = {k: x.detach().double().requires_grad_(True) for k, x in leaves.items()}

    class G:  # the graph with differentiable direction / Y
        pass
    gg = G()
    for k in ("row", "col", "perm", "node_start", "node_end", "avg_degree", "N", "E"):
        setattr(gg, k, getattr(gr, k))
    gg.direction, gg.Y = gpu["d"], gpu["Y"]
    Wg = {k: gpu.get(k) for k in W}
    outs = se3_message_aggregate(gpu["s"], gpu["v"], gg, gpu["R"], Wg, Os, Ov, Ot, type2=gpu.get("t"),
                                 bias=gpu.get("bias"), mask=mask.to(dev), return_type2=True)
    Wc = {k: cpu.get(k) for k in W}
    want = ose3.se3_conv(cpu["s"], cpu["v"], cpu.get("t"), gr.row.cpu(), gr.col.cpu(), cpu["d"], cpu["Y"],
                         cpu["R"], Wc, ose3.cg_11_2_cartesian(), Os, Ov, Ot, gr.avg_degree.cpu(),
                         bias=cpu.get("bias"), mask=mask)
    for o, w in zip(outs, want):
        if w is None:
            assert o is None or o.numel() == 0
            continue
        _close(o, w, 2e-4, 2e-5)
    gen = torch.Generator().manual_seed(5)
    loss_g, loss_c = 0, 0
    for o, w in zip(outs, want):
        if w is None or w.numel() == 0:
            continue
        c = torch.randn(w.shape, generator=gen, dtype=torch.float64)
        loss_g = loss_g + (o * c.to(dev).float()).sum()
        loss_c = loss_c + (w * c).sum()
    loss_g.backward()
    loss_c.backward()
    for k in leaves:
        wg = cpu[k].grad
        gg_ = gpu[k].grad
        if wg is None:
            assert gg_ is None or gg_.numel() == 0 or float(gg_.abs().max()) == 0.0, k
            continue
        assert gg_ is not None, k
        _close(gg_, wg, 5e-4, 5e-5)


def test_se3conv_module_end_to_end(dev):
    """The module on a SpatialGraph: outputs and parameter / feature / position gradients vs the
    oracle fed with the module's own radial weights (float64 on the CPU)."""
    from gdl_amd.graph import SpatialGraph
    from gdl_amd.se3_conv import SE3Conv
    torch.manual_seed(0)
    conv = SE3Conv(16, 8, 12, 6, in_type2_channels=4, out_type2_channels=3, radius=0.3).to(dev)
    with torch.no_grad():
        conv.scalar_bias.normal_()
    g = torch.Generator().manual_seed(3)
    pos = torch.rand(500, 3, generator=g)
    s = torch.randn(500, 16, generator=g)
    v = torch.randn(500, 8, 3, generator=g)
    t = torch.randn(500, 4, 5, generator=g)
    p_gpu = pos.to(dev).requires_grad_(True)
    gr = SpatialGraph.build(p_gpu, 0.3, max_num_neighbors=20)
    sg, vg, tg = (x.to(dev).requires_grad_(True) for x in (s, v, t))
    out = conv(sg, vg, gr, type2=tg)
    assert len(out) == 3
    gen = torch.Generator().manual_seed(1)
    cs = [torch.randn(o.shape, generator=gen) for o in out]
    sum((o * c.to(dev)).sum() for o, c in zip(out, cs)).backward()

    import copy
    from sh_torch import sh_torch
    ref = copy.deepcopy(conv).cpu().double()
    ref.zero_grad(set_to_none=True)
    p64 = pos.double().requires_grad_(True)
    row, col = gr.row.cpu(), gr.col.cpu()
    diff = p64[col] - p64[row]
    dist = diff.norm(dim=-1, keepdim=True).clamp(min=1e-8)
    direction = diff / dist
    Y = sh_torch(direction, 2)
    rb = ref.radial_basis
    R = ose3.radial_basis(dist.squeeze(-1), rb.freqs, rb.cutoff, rb.mlp[0].weight, rb.mlp[0].bias,
                          rb.mlp[2].weight, rb.mlp[2].bias)
    W = {k: (getattr(ref, k).weight if getattr(ref, k) is not None else None) for k in ose3.PATH_NAMES}
    s64, v64, t64 = (x.double().requires_grad_(True) for x in (s, v, t))
    want = ose3.se3_conv(s64, v64, t64, row, col, direction, Y, R, W, ref.cg_11_2, 12, 6, 3,
                         gr.avg_degree.cpu(), bias=ref.scalar_bias)
    for o, w in zip(out, want):
        _close(o, w, 2e-4, 2e-5)
    sum((w * c.double()).sum() for w, c in zip(want, cs)).backward()
    for got, wnt in ((sg.grad, s64.grad), (vg.grad, v64.grad), (tg.grad, t64.grad), (p_gpu.grad, p64.grad)):
        _close(got, wnt, 1e-3, 1e-4)
    for (name, pg), (_, pr) in zip(conv.named_parameters(), ref.named_parameters()):
        assert pg.grad is not None, name
        _close(pg.grad, pr.grad, 1e-3, 1e-4)


def test_se3conv_empty_graph(dev):
    from gdl_amd.graph import SpatialGraph
    from gdl_amd.se3_conv import SE3Conv
    conv = SE3Conv(4, 2, 3, 2).to(dev)
    with torch.no_grad():
        conv.scalar_bias.fill_(0.5)
    pos = torch.randn(20, 3, device=dev) * 100
    gr = SpatialGraph.build(pos, 1e-3)
    s = torch.randn(20, 4, device=dev, requires_grad=True)
    so, vo = conv(s, torch.randn(20, 2, 3, device=dev), gr)
    assert torch.equal(so, torch.full((20, 3), 0.5, device=dev)) and not vo.any()
    so.sum().backward()
    assert s.grad is not None and not s.grad.any()


def _rot(seed):
    q, _ = np.linalg.qr(np.random.default_rng(seed).normal(size=(3, 3)))
    return q * np.sign(np.linalg.det(q))


def _wigner_d2(Q):
    import oracle
    u = np.random.default_rng(7).normal(size=(64, 3))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    A = oracle.spherical_harmonics(u, 2, False)[:, 4:9]
    B = oracle.spherical_harmonics(u @ Q.T, 2, False)[:, 4:9]
    D, *_ = np.linalg.lstsq(A, B, rcond=None)
    return D.T


@pytest.mark.parametrize("seed", [0, 1])
def test_se3conv_rotation_equivariance(dev, seed):
    """f(R x) = R . f(x) for all three feature types (the reference's SE3Conv equivariance test,
    tests/test_se3conv_equivariance.py:186-300, with type-2 features added): the same edge set is
    used for both poses so that no edge flips at the radius boundary."""
    from gdl_amd.graph import SpatialGraph
    from gdl_amd.se3_conv import SE3Conv
    torch.manual_seed(seed)
    conv = SE3Conv(8, 4, 6, 5, in_type2_channels=3, out_type2_channels=2, radius=0.4).to(dev)
    g = torch.Generator().manual_seed(seed)
    pos = torch.rand(400, 3, generator=g)
    s = torch.randn(400, 8, generator=g)
    v = torch.randn(400, 4, 3, generator=g)
    t = torch.randn(400, 3, 5, generator=g)
    gr1 = SpatialGraph.build(pos.to(dev), 0.4, max_num_neighbors=24)
    Q = torch.from_numpy(_rot(seed)).float()
    D2 = torch.from_numpy(_wigner_d2(_rot(seed))).float()
    pr = pos @ Q.T
    gr2 = SpatialGraph.from_edge_index(gr1.row, gr1.col, pr.to(dev), 400)
    s1, v1, t1 = conv(s.to(dev), v.to(dev), gr1, type2=t.to(dev))
    s2, v2, t2 = conv(s.to(dev), (v @ Q.T).to(dev), gr2, type2=(t @ D2.T).to(dev))
    _close(s2, s1, 1e-4, 1e-4)
    _close(v2, v1 @ Q.T.to(dev), 1e-4, 1e-4)
    _close(t2, t1 @ D2.T.to(dev), 1e-4, 1e-4)


def test_se3conv_dtypes_and_autocast(dev):
    """Outputs keep the input dtype (fp64 module and inputs, as tests/test_dtype_preservation.py:
    10-30 asks; half inputs computed in fp32 and returned as half) and stay fp32 under autocast
    (:74-103)."""
    from gdl_amd.graph import SpatialGraph
    from gdl_amd.se3_conv import SE3Conv
    torch.manual_seed(0)
    pos = torch.rand(200, 3, device=dev)
    gr = SpatialGraph.build(pos, 0.3, max_num_neighbors=32)
    conv = SE3Conv(16, 4, 16, 4, radius=0.3).to(dev)
    s = torch.randn(200, 16, device=dev)
    v = torch.randn(200, 4, 3, device=dev)
    s32, v32 = conv(s, v, gr)
    c64 = SE3Conv(16, 4, 16, 4, radius=0.3).to(dev)
    c64.load_state_dict(conv.state_dict())
    c64 = c64.double()
    sd = s.double().requires_grad_(True)
    s64, v64 = c64(sd, v.double(), gr)
    assert s64.dtype == torch.float64 and v64.dtype == torch.float64
    _close(s64, s32, 1e-6, 1e-6)
    (s64.sum() + v64.sum()).backward()
    assert sd.grad.dtype == torch.float64
    assert all(p.grad is not None and p.grad.dtype == torch.float64 for p in c64.parameters())
    s16, v16 = conv(s.half(), v.half(), gr)
    assert s16.dtype == torch.float16 and v16.dtype == torch.float16
    with torch.autocast("cuda"):
        sa, va = conv(s, v, gr)
    assert sa.dtype == torch.float32 and va.dtype == torch.float32
    _close(sa, s32, 0, 0)


@pytest.mark.parametrize("type2", [False, True])
def test_se3conv_run_to_run_bitwise(dev, type2):
    """Five forward + backward passes of one layer on the full C2 graph (16 clouds x 4096 points,
    r = 0.1, K = 32, 657,154 edges; positions, features and weights all require grad) give
    bit-identical outputs and gradients every time, as the reference asks of its own layer
    (tests/test_segment_reduce.py:274-283): every sum here has a fixed order (CSR walks, per-block
    partials added in block order), none depends on atomics or scheduling."""
    import bench
    from gdl_amd.graph import SpatialGraph
    from gdl_amd.se3_conv import SE3Conv
    c = bench.make_c2()
    torch.manual_seed(0)
    ct = 4 if type2 else 0
    conv = SE3Conv(64, 16, 64, 16, in_type2_channels=ct, out_type2_channels=ct,
                   radius=c["r"]).to(dev)
    with torch.no_grad():
        conv.scalar_bias.normal_()
    g = torch.Generator().manual_seed(5)
    N = c["pos"].shape[0]
    s = torch.randn(N, 64, generator=g).to(dev)
    v = torch.randn(N, 16, 3, generator=g).to(dev)
    t = torch.randn(N, 4, 5, generator=g).to(dev) if type2 else None
    outs_ref = None
    for rep in range(5):
        conv.zero_grad(set_to_none=True)
        p = c["pos"].to(dev).requires_grad_(True)
        gr = SpatialGraph.build(p, c["r"], max_num_neighbors=c["K"], batch=c["batch"].to(dev),
                                num_batch_elements=c["B"])
        assert gr.E == 657_154
        xs = [s.clone().requires_grad_(True), v.clone().requires_grad_(True)]
        if type2:
            xs.append(t.clone().requires_grad_(True))
        out = conv(xs[0], xs[1], gr, type2=xs[2] if type2 else None)
        gen = torch.Generator(device=dev).manual_seed(11)
        cot = [torch.randn(o.shape, device=dev, generator=gen) for o in out]
        torch.autograd.backward(list(out), cot)
        got = [o.detach().clone() for o in out] + [x.grad.clone() for x in xs] + [p.grad.clone()] + \
              [q.grad.clone() for q in conv.parameters()]
        assert all(torch.isfinite(x).all() for x in got)
        if outs_ref is None:
            outs_ref = got
            print(f"[se3 determinism] E={gr.E} type2={type2}: {len(got)} tensors", flush=True)
        else:
            for i, (a, b) in enumerate(zip(got, outs_ref)):
                assert torch.equal(a, b), (rep, i)


# Fused forward (aggregate tile in LDS, weights applied there) against the two-kernel path
# (geo_se3_aggregate_fwd + geo_se3_gemm): both add a node's edges in CSR order with the same
# per-edge arithmetic and the same MFMA k order, so outputs and kept aggregates are bit-identical.
FUSED_CONFIGS = [
    # Cs, Cv, Ct, Os, Ov, Ot
    (64, 16, 0, 64, 16, 0),    # the C2 layer
    (8, 4, 0, 8, 4, 0),
    (96, 8, 0, 40, 8, 0),      # two 64-channel chunks, three scalar column blocks
    (12, 6, 0, 10, 5, 3),      # type-2 output from scalars and vectors only
    (5, 0, 2, 4, 0, 3),
    (0, 4, 0, 3, 2, 0),
    (16, 4, 3, 16, 4, 2),      # every path
    (60, 13, 0, 33, 7, 0),     # one node per 16-lane row: partial lanes in both kinds
    (64, 0, 0, 32, 0, 0),      # scalars only
    (4, 1, 0, 5, 3, 0),
]


def _abi_forward(cfg, gr, s, v, t, W, R, bias, mask, fused, keep, dev):
    import ctypes
    from gdl_amd import _native as nat
    from gdl_amd.se3_conv import PATH_NAMES, _Plan, _cg_on, _gemm, _pack, _pad64, path_columns
    Cs, Cv, Ct, Os, Ov, Ot = cfg
    N, E = gr.N, gr.E
    pc = path_columns(W, t is not None, True, Ot)
    p = _Plan(Cs, Cv, Ct, Os, Ov, Ot, pc, R.shape[1], gr.Y.shape[1], Ot > 0)
    Wl = [W[k] for k in PATH_NAMES]
    Ws, Wv, Wt = _pack(p, Wl, [(0, _pad64(p.Os), p.Ks), (1, _pad64(p.Ov), p.Kv),
                               (2, _pad64(p.Ot), p.Kt)], dev)
    f32 = dict(dtype=torch.float32, device=dev)
    so = torch.full((N, Os), float("nan"), **f32)
    vo = torch.full((N, Ov, 3), float("nan"), **f32)
    to = torch.full((N, Ot, 5), float("nan"), **f32)
    Xs = torch.full((N, p.Ks), float("nan"), **f32) if Os > 0 and keep else None
    Xv = torch.full((N, 3, p.Kv), float("nan"), **f32) if Ov > 0 and keep else None
    Xt = torch.full((N, 5, p.Kt), float("nan"), **f32) if Ot > 0 and keep else None
    perm = None if getattr(gr, "_perm_identity", False) else gr.perm
    cg = _cg_on(dev) if pc[7] >= 0 else None
    avg, mask_u8 = gr.avg_degree, mask.view(torch.uint8)
    L, st = nat.lib(), nat.stream_of(dev)
    common = (nat.ptr(s), nat.ptr(v), nat.ptr(t), N, Cs, Cv, Ct, nat.ptr(gr.row), nat.ptr(perm),
              nat.ptr(gr.node_start), nat.ptr(gr.node_end), E, nat.ptr(gr.direction), nat.ptr(gr.Y),
              gr.Y.shape[1], nat.ptr(R), R.shape[1], p.pc_c, nat.ptr(cg))
    if fused:
        assert L.geo_se3_fwd_fused_lds_bytes(Os, Ov, Ot, p.Ks, p.Kv, p.Kt) > 0
        nat.check(L.geo_se3_fwd_fused(
            *common, nat.ptr(Ws), Ws.shape[0], nat.ptr(Wv), Wv.shape[0], nat.ptr(Wt), Wt.shape[0],
            Os, Ov, Ot, p.Ks, p.Kv, p.Kt, nat.ptr(avg), nat.ptr(bias), nat.ptr(mask_u8),
            nat.ptr(so), nat.ptr(vo), nat.ptr(to), nat.ptr(Xs), nat.ptr(Xv), nat.ptr(Xt), st),
            "geo_se3_fwd_fused")
    else:
        nat.check(L.geo_se3_aggregate_fwd(*common, nat.ptr(Xs), p.Ks, nat.ptr(Xv), p.Kv,
                                          nat.ptr(Xt), p.Kt, st), "geo_se3_aggregate_fwd")
        _gemm(Xs, N, p.Ks, Ws, Os, 1, so, Os, avg, bias, mask_u8)
        _gemm(Xv, 3 * N, p.Kv, Wv, Ov, 3, vo, 3 * Ov, avg, None, mask_u8)
        _gemm(Xt, 5 * N, p.Kt, Wt, Ot, 5, to, 5 * Ot, avg, None, mask_u8)
    torch.cuda.synchronize()
    return (so, vo, to), (Xs, Xv, Xt)


@pytest.mark.parametrize("cfg", FUSED_CONFIGS, ids=[str(c) for c in FUSED_CONFIGS])
@pytest.mark.parametrize("graph", ["sorted", "shuffled", "dense"])
def test_fused_forward_bitwise_vs_two_kernel_path(dev, cfg, graph):
    """Also covers partial tiles (N = 600 and 250 are not multiples of 16), nodes without edges,
    and (dense: K = 100) nodes whose edges fill more than one 64-edge staging round."""
    if graph == "dense":
        gr = _graph(250, 1, 0.45, 100, 7, False)
        assert int((gr.node_end - gr.node_start).max()) > 64
    else:
        gr = _graph(300, 2, 0.22, 24, sum(cfg), graph == "shuffled")
    s, v, t, W, R, bias, mask = _inputs(cfg, gr, 3, dev)
    s, v, R, mask = s.to(dev), v.to(dev), R.to(dev), mask.to(dev)
    t = t.to(dev) if t is not None else None
    bias = bias.to(dev) if bias is not None else None
    W = {k: (w.to(dev) if w is not None else None) for k, w in W.items()}
    print(f"[se3 fused] cfg={cfg} graph={graph} N={gr.N} E={gr.E}", flush=True)
    want, Xw = _abi_forward(cfg, gr, s, v, t, W, R, bias, mask, False, True, dev)
    got, Xg = _abi_forward(cfg, gr, s, v, t, W, R, bias, mask, True, True, dev)
    got0, _ = _abi_forward(cfg, gr, s, v, t, W, R, bias, mask, True, False, dev)
    for a, b, c in zip(got, got0, want):
        assert torch.isfinite(c).all()
        assert torch.equal(a, c) and torch.equal(b, c)
    for a, b in zip(Xg, Xw):
        assert (a is None) == (b is None)
        if a is not None:
            assert torch.equal(a, b)


def _abi_src_backward(cfg, gr, W, R, fused, dev, seed):
    """Feature gradients from prepared output gradients (random rows, zero padding) through the
    C ABI: geo_se3_bwd_src_fused, or geo_se3_bwd_src + geo_se3_gemm.  Returns (ds, dv) (NaN where
    nothing was written), or None when the fused entry point declines the layer."""
    from gdl_amd import _native as nat
    from gdl_amd.csrc import source_csr
    from gdl_amd.se3_conv import PATH_NAMES, _Plan, _cg_on, _gemm, _pack, _pad64, path_columns
    Cs, Cv, Ct, Os, Ov, Ot = cfg
    N, E = gr.N, gr.E
    pc = path_columns(W, Ct > 0, True, Ot)
    p = _Plan(Cs, Cv, Ct, Os, Ov, Ot, pc, R.shape[1], gr.Y.shape[1], Ot > 0)
    g = torch.Generator().manual_seed(seed)
    f32 = dict(dtype=torch.float32, device=dev)
    Gs = torch.zeros(N, p.OsP)
    Gs[:, :Os] = torch.randn(N, Os, generator=g)
    Gv = torch.zeros(N, 3, p.OvP)
    Gv[:, :, :Ov] = torch.randn(N, 3, Ov, generator=g)
    Gs, Gv = (Gs.to(dev) if Os > 0 else None), (Gv.to(dev) if Ov > 0 else None)
    Wl = [W[k] for k in PATH_NAMES]
    Bs, Bv = _pack(p, Wl, [(6, _pad64(Cs), p.KZs if Cs > 0 else 0),
                           (7, _pad64(Cv), p.KZv if Cv > 0 else 0)], dev)
    ds = torch.full((N, Cs), float("nan"), **f32) if Cs > 0 else None
    dv = torch.full((N, Cv, 3), float("nan"), **f32) if Cv > 0 else None
    perm_r, ns_r, ne_r = source_csr(gr.row, N)
    cg = _cg_on(dev) if pc[7] >= 0 else None
    L, st = nat.lib(), nat.stream_of(dev)
    graph = (N, nat.ptr(gr.col), nat.ptr(perm_r), nat.ptr(ns_r), nat.ptr(ne_r), E,
             nat.ptr(gr.direction), nat.ptr(gr.Y), gr.Y.shape[1], nat.ptr(R), R.shape[1], p.pc_c,
             nat.ptr(cg))
    if fused:
        rc = L.geo_se3_bwd_src_fused(nat.ptr(Gs), Os, p.OsP, nat.ptr(Gv), Ov, p.OvP, *graph, p.KZs,
                                     p.KZv, nat.ptr(Bs), Bs.shape[0], Cs, nat.ptr(ds), nat.ptr(Bv),
                                     Bv.shape[0], Cv, nat.ptr(dv), st)
        torch.cuda.synchronize()
        if rc == nat.GEO_ERR_UNSUPPORTED:
            for o in (ds, dv):  # declined: nothing written
                assert o is None or torch.isnan(o).all()
            return None
        nat.check(rc, "geo_se3_bwd_src_fused")
    else:
        Zs = torch.empty(N, p.KZs, **f32) if Cs > 0 else None
        Zv = torch.empty(N, 3, p.KZv, **f32) if Cv > 0 else None
        nat.check(L.geo_se3_bwd_src(nat.ptr(Gs), Os, p.OsP, nat.ptr(Gv), Ov, p.OvP, None, 0, 0,
                                    *graph, nat.ptr(Zs), p.KZs, nat.ptr(Zv), p.KZv, None, 0, None, 0,
                                    st), "geo_se3_bwd_src")
        if Cs > 0:
            _gemm(Zs, N, p.KZs, Bs, Cs, 1, ds, Cs)
        if Cv > 0:
            _gemm(Zv, 3 * N, p.KZv, Bv, Cv, 3, dv, 3 * Cv)
        torch.cuda.synchronize()
    return ds, dv


SRC_FUSED_CONFIGS = [
    # Cs, Cv, Ct, Os, Ov, Ot
    (64, 16, 0, 64, 16, 0),    # the C2 layer
    (8, 4, 0, 8, 4, 0),
    (96, 8, 0, 40, 8, 0),      # six scalar column blocks of ds
    (0, 4, 0, 3, 2, 0),        # no scalar input: only dv
    (20, 0, 0, 6, 0, 0),       # no vector channels: only ds
]


@pytest.mark.parametrize("cfg", SRC_FUSED_CONFIGS, ids=[str(c) for c in SRC_FUSED_CONFIGS])
@pytest.mark.parametrize("graph", ["sorted", "shuffled", "dense"])
def test_fused_source_backward_bitwise_vs_two_step_path(dev, cfg, graph):
    """geo_se3_bwd_src_fused (source-side sums kept in LDS, multiplied there by the transposed
    weights) equals geo_se3_bwd_src + geo_se3_gemm bit for bit: the same sums in the same order,
    the same MFMA accumulation.  Partial tiles (N not a multiple of 16), sources without edges and
    (dense) sources with more than 16 edges per staging round."""
    if graph == "dense":
        gr = _graph(250, 1, 0.45, 100, 7, False)
    else:
        gr = _graph(300, 2, 0.22, 24, sum(cfg), graph == "shuffled")
    _, _, _, W, R, _, _ = _inputs(cfg, gr, 5, dev)
    R = R.to(dev)
    W = {k: (w.to(dev) if w is not None else None) for k, w in W.items()}
    print(f"[se3 src fused] cfg={cfg} graph={graph} N={gr.N} E={gr.E}", flush=True)
    got = _abi_src_backward(cfg, gr, W, R, True, dev, 11)
    want = _abi_src_backward(cfg, gr, W, R, False, dev, 11)
    assert got is not None
    for a, b in zip(got, want):
        assert (a is None) == (b is None)
        if a is not None:
            assert torch.isfinite(b).all()
            assert torch.equal(a, b)


@pytest.mark.parametrize("cfg", [(80, 20, 6, 70, 10, 4), (8, 4, 0, 70, 4, 0), (8, 20, 0, 8, 20, 0)],
                         ids=["type2", "Os70", "Ov20"])
def test_fused_source_backward_declines_uncovered_layers(dev, cfg):
    """Type-2 paths, more than 64 scalar or 16 vector output channels: GEO_ERR_UNSUPPORTED and
    nothing written (the layer then takes geo_se3_bwd_src and the GEMMs)."""
    gr = _graph(300, 2, 0.22, 24, sum(cfg), False)
    _, _, _, W, R, _, _ = _inputs(cfg, gr, 6, dev)
    W = {k: (w.to(dev) if w is not None else None) for k, w in W.items()}
    assert _abi_src_backward(cfg, gr, W, R.to(dev), True, dev, 12) is None


def _abi_edge_backward(cfg, gr, s, v, W, R, fused, dev, seed):
    """Per-edge gradients (dR, ddir, dY; NaN-initialised, then zero-filled like the module) from
    prepared output gradients (random rows, zero padding) through the C ABI:
    geo_se3_bwd_edge_fused, or gX by geo_se3_gemm + geo_se3_bwd_edge.  None when the fused entry
    point declines the layer."""
    from gdl_amd import _native as nat
    from gdl_amd.se3_conv import PATH_NAMES, _Plan, _cg_on, _gemm, _pack, _pad64, path_columns
    Cs, Cv, Ct, Os, Ov, Ot = cfg
    N, E = gr.N, gr.E
    pc = path_columns(W, Ct > 0, True, Ot)
    p = _Plan(Cs, Cv, Ct, Os, Ov, Ot, pc, R.shape[1], gr.Y.shape[1], Ot > 0)
    g = torch.Generator().manual_seed(seed)
    f32 = dict(dtype=torch.float32, device=dev)
    Gs = torch.zeros(N, p.OsP)
    Gs[:, :Os] = torch.randn(N, Os, generator=g)
    Gv = torch.zeros(N, 3, p.OvP)
    Gv[:, :, :Ov] = torch.randn(N, 3, Ov, generator=g)
    Gs, Gv = (Gs.to(dev) if Os > 0 else None), (Gv.to(dev) if Ov > 0 else None)
    Wl = [W[k] for k in PATH_NAMES]
    WsT, WvT = _pack(p, Wl, [(3, _pad64(p.Ks), p.OsP if Gs is not None else 0),
                             (4, _pad64(p.Kv), p.OvP if Gv is not None else 0)], dev)
    dR = torch.zeros(E, p.P, **f32)
    ddir = torch.zeros(E, 3, **f32)
    dY = torch.zeros(E, p.ysh, **f32)
    perm = None if getattr(gr, "_perm_identity", False) else gr.perm
    cg = _cg_on(dev) if pc[7] >= 0 else None
    L, st = nat.lib(), nat.stream_of(dev)
    graph = (nat.ptr(gr.row), nat.ptr(perm), nat.ptr(gr.node_start), nat.ptr(gr.node_end), E,
             nat.ptr(gr.direction), nat.ptr(gr.Y), gr.Y.shape[1], nat.ptr(R), R.shape[1], p.pc_c,
             nat.ptr(cg))
    if fused:
        rc = L.geo_se3_bwd_edge_fused(nat.ptr(s), nat.ptr(v), N, Cs, Cv, *graph, nat.ptr(Gs), p.OsP,
                                      nat.ptr(Gv), p.OvP, nat.ptr(WsT), WsT.shape[0], nat.ptr(WvT),
                                      WvT.shape[0], p.Ks, p.Kv, nat.ptr(dR), nat.ptr(ddir),
                                      nat.ptr(dY), st)
        torch.cuda.synchronize()
        if rc == nat.GEO_ERR_UNSUPPORTED:
            for o in (dR, ddir, dY):  # declined: nothing written
                assert not o.any()
            return None
        nat.check(rc, "geo_se3_bwd_edge_fused")
    else:
        gXs = torch.empty(N, p.Ks, **f32) if Gs is not None else None
        gXv = torch.empty(N, 3, p.Kv, **f32) if Gv is not None else None
        if Gs is not None:
            _gemm(Gs, N, p.OsP, WsT, p.Ks, 1, gXs, p.Ks)
        if Gv is not None:
            _gemm(Gv, 3 * N, p.OvP, WvT, p.Kv, 1, gXv, p.Kv)
        nat.check(L.geo_se3_bwd_edge(nat.ptr(s), nat.ptr(v), None, N, Cs, Cv, 0, *graph,
                                     nat.ptr(gXs), p.Ks, nat.ptr(gXv), p.Kv, None, 0, nat.ptr(dR),
                                     nat.ptr(ddir), nat.ptr(dY), st), "geo_se3_bwd_edge")
        torch.cuda.synchronize()
    return dR, ddir, dY


EDGE_FUSED_CONFIGS = [
    # Cs, Cv, Ct, Os, Ov, Ot (the edge path's limits are on the inputs: Cs <= 64, Cv <= 16)
    (64, 16, 0, 64, 16, 0),    # the C2 layer
    (8, 4, 0, 8, 4, 0),
    (40, 8, 0, 96, 8, 0),      # 96 output channels: a 96-wide gradient tile
    (0, 4, 0, 3, 2, 0),        # no scalar input
    (20, 0, 0, 6, 0, 0),       # no vector channels
]


@pytest.mark.parametrize("cfg", EDGE_FUSED_CONFIGS, ids=[str(c) for c in EDGE_FUSED_CONFIGS])
@pytest.mark.parametrize("graph", ["sorted", "shuffled", "dense"])
def test_fused_edge_backward_bitwise_vs_two_step_path(dev, cfg, graph):
    """geo_se3_bwd_edge_fused (gX formed per tile of 16 targets in LDS) equals the gX GEMMs +
    geo_se3_bwd_edge bit for bit: partial tiles, targets without edges, dense targets with more
    than 64 edges (several staging rounds), a shuffled edge order."""
    if graph == "dense":
        gr = _graph(250, 1, 0.45, 100, 7, False)
    else:
        gr = _graph(300, 2, 0.22, 24, sum(cfg) + 1, graph == "shuffled")
    s, v, _, W, R, _, _ = _inputs(cfg, gr, 8, dev)
    s, v, R = s.to(dev), v.to(dev), R.to(dev)
    W = {k: (w.to(dev) if w is not None else None) for k, w in W.items()}
    print(f"[se3 edge fused] cfg={cfg} graph={graph} N={gr.N} E={gr.E}", flush=True)
    got = _abi_edge_backward(cfg, gr, s, v, W, R, True, dev, 13)
    want = _abi_edge_backward(cfg, gr, s, v, W, R, False, dev, 13)
    assert got is not None
    for a, b in zip(got, want):
        assert torch.isfinite(b).all()
        assert torch.equal(a, b)
    assert want[0].abs().sum() > 0


@pytest.mark.parametrize("cfg", [(80, 20, 6, 70, 10, 4), (96, 4, 0, 8, 4, 0), (8, 20, 0, 8, 20, 0)],
                         ids=["type2", "Cs96", "Cv20"])
def test_fused_edge_backward_declines_uncovered_layers(dev, cfg):
    """Type-2 paths, more than 64 scalar or 16 vector input channels: GEO_ERR_UNSUPPORTED and
    nothing written (the layer then takes the gX GEMMs and geo_se3_bwd_edge)."""
    gr = _graph(300, 2, 0.22, 24, sum(cfg), False)
    s, v, _, W, R, _, _ = _inputs(cfg, gr, 9, dev)
    W = {k: (w.to(dev) if w is not None else None) for k, w in W.items()}
    assert _abi_edge_backward(cfg, gr, s.to(dev), v.to(dev), W, R.to(dev), True, dev, 14) is None


@pytest.mark.parametrize("cfg", FUSED_CONFIGS + [CONFIGS[2]], ids=[str(c) for c in FUSED_CONFIGS + [CONFIGS[2]]])
def test_forward_without_grad_vs_oracle(dev, cfg):
    """Under no_grad nothing keeps the aggregates: the fused forward writes only the outputs."""
    from gdl_amd.se3_conv import se3_message_aggregate
    Cs, Cv, Ct, Os, Ov, Ot = cfg
    gr = _graph(300, 2, 0.22, 24, sum(cfg) + 3, True)
    s, v, t, W, R, bias, mask = _inputs(cfg, gr, 4, dev)
    Wg = {k: (w.to(dev).requires_grad_(True) if w is not None else None) for k, w in W.items()}
    with torch.no_grad():
        outs = se3_message_aggregate(s.to(dev), v.to(dev), gr, R.to(dev), Wg, Os, Ov, Ot,
                                     type2=t.to(dev) if t is not None else None,
                                     bias=bias.to(dev) if bias is not None else None,
                                     mask=mask.to(dev), return_type2=True)
    Wc = {k: (w.double() if w is not None else None) for k, w in W.items()}
    want = ose3.se3_conv(s.double(), v.double(), t.double() if t is not None else None,
                         gr.row.cpu(), gr.col.cpu(), gr.direction.cpu().double(),
                         gr.Y.cpu().double(), R.double(), Wc, ose3.cg_11_2_cartesian(), Os, Ov, Ot,
                         gr.avg_degree.cpu(), bias=bias.double() if bias is not None else None,
                         mask=mask)
    for o, w in zip(outs, want):
        if w is None:
            assert o is None or o.numel() == 0
            continue
        _close(o, w, 2e-4, 2e-5)
