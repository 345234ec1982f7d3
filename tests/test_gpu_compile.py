"""torch.compile transparency of the custom ops, restating the reference's
tests/test_torch_compile.py:83-197 for this build:

* ``torch._dynamo.explain`` reports 0 graph breaks through ``segment_reduce`` (sum, mean, max)
  and through a two-layer SE3Conv network (the reference's MiniSE3Net, :34-76), and through one
  C2-sized SE3Conv layer (64 scalar + 16 vector channels on one 4096-point cloud, r = 0.1);
* compiled and eager results agree: forward within 1e-5, backward (inputs and parameters)
  within 1e-4 (the reference's atol values, :136-197).

Graphs are built outside the compiled region, as in the reference (:100-104).
"""

import pytest
import torch
import torch.nn as nn

pytestmark = pytest.mark.gpu

BACKENDS = ["aot_eager", "inductor"]


def _csr(dev, E=600, N=90, C=24, seed=0):
    import geoembodied  # noqa: F401
    from geoembodied.functional.segment_reduce import sort_and_build_csr
    g = torch.Generator().manual_seed(seed)
    col = torch.randint(0, N, (E,), generator=g).to(dev)
    msg = torch.randn(E, C, generator=g).to(dev)
    return msg, sort_and_build_csr(col, N), N


class _Seg(nn.Module):
    def __init__(self, reduce):
        super().__init__()
        self.reduce = reduce

    def forward(self, msg, cs, pm, ns, ne, N: int):
        from geoembodied.functional.segment_reduce import segment_reduce
        out = segment_reduce(msg * 2.0, cs, pm, ns, ne, N, reduce=self.reduce)
        return out.relu() + 1.0


@pytest.mark.parametrize("reduce", ["sum", "mean", "max"])
def test_segment_reduce_zero_graph_breaks(dev, reduce):
    torch._dynamo.reset()
    msg, (cs, pm, ns, ne), N = _csr(dev)
    ex = torch._dynamo.explain(_Seg(reduce))(msg, cs, pm, ns, ne, N)
    assert ex.graph_break_count == 0, ex.break_reasons
    assert ex.graph_count == 1


@pytest.mark.parametrize("backend", BACKENDS)
@pytest.mark.parametrize("reduce", ["sum", "mean", "max"])
def test_segment_reduce_compiled_matches_eager(dev, reduce, backend):
    torch._dynamo.reset()
    msg, (cs, pm, ns, ne), N = _csr(dev, seed=1)
    model = _Seg(reduce)
    x1 = msg.clone().requires_grad_(True)
    x2 = msg.clone().requires_grad_(True)
    gout = torch.randn(N, msg.shape[1], device=dev)
    eager = model(x1, cs, pm, ns, ne, N)
    (eager * gout).sum().backward()
    comp = torch.compile(model, backend=backend, dynamic=True)
    out = comp(x2, cs, pm, ns, ne, N)
    (out * gout).sum().backward()
    assert torch.allclose(eager, out, atol=1e-5, rtol=0)
    assert torch.allclose(x1.grad, x2.grad, atol=1e-4, rtol=0)


class MiniSE3Net(nn.Module):
    """The reference's two-layer test backbone (tests/test_torch_compile.py:34-76)."""

    def __init__(self):
        super().__init__()
        from gdl_amd.se3_conv import SE3Conv
        self.conv1 = SE3Conv(8, 4, 8, 4, radius=3.0, max_num_neighbors=16)
        self.conv2 = SE3Conv(8, 4, 4, 2, radius=3.0, max_num_neighbors=16)

    def forward(self, scalars, vectors, graph):
        s, v = self.conv1(scalars, vectors, graph)
        return self.conv2(s, v, graph)


def _mini_graph(dev):
    from gdl_amd.graph import SpatialGraph
    torch.manual_seed(42)
    pos = torch.randn(15, 3, device=dev) * 0.5
    s = torch.randn(15, 8, device=dev)
    v = torch.randn(15, 4, 3, device=dev)
    return pos, s, v, SpatialGraph.build(pos, radius=3.0, max_num_neighbors=16)


def test_se3net_zero_graph_breaks(dev):
    torch._dynamo.reset()
    model = MiniSE3Net().to(dev).eval()
    _, s, v, graph = _mini_graph(dev)
    ex = torch._dynamo.explain(model)(s, v, graph)
    assert ex.graph_break_count == 0, ex.break_reasons
    assert ex.graph_count == 1


def test_se3conv_c2_layer_zero_graph_breaks(dev):
    """One C2-sized layer: 64 scalar + 16 vector channels on a 4096-point unit-sphere cloud,
    r = 0.1, K = 32 (~41k edges), forward and backward under explain."""
    import bench
    from gdl_amd.graph import SpatialGraph
    from gdl_amd.se3_conv import SE3Conv
    torch._dynamo.reset()
    c = bench.make_c2(B=1)
    pos = c["pos"].to(dev)
    graph = SpatialGraph.build(pos, c["r"], max_num_neighbors=c["K"])
    assert graph.E > 30000
    torch.manual_seed(0)
    conv = SE3Conv(64, 16, 64, 16, radius=c["r"]).to(dev)
    s = torch.randn(graph.N, 64, device=dev, requires_grad=True)
    v = torch.randn(graph.N, 16, 3, device=dev, requires_grad=True)

    def step(s, v, graph):
        so, vo = conv(s, v, graph)
        return so.square().sum() + vo.square().sum()

    ex = torch._dynamo.explain(step)(s, v, graph)
    print(f"[compile] SE3Conv C2 layer (E={graph.E}): {ex.graph_break_count} graph breaks, "
          f"{ex.graph_count} graph(s)", flush=True)
    assert ex.graph_break_count == 0, ex.break_reasons


@pytest.mark.parametrize("backend", BACKENDS)
def test_se3net_forward_parity(dev, backend):
    torch._dynamo.reset()
    model = MiniSE3Net().to(dev).eval()
    _, s, v, graph = _mini_graph(dev)
    with torch.no_grad():
        s_e, v_e = model(s, v, graph)
        comp = torch.compile(model, backend=backend, dynamic=True)
        s_c, v_c = comp(s, v, graph)
    assert torch.allclose(s_e, s_c, atol=1e-5, rtol=0), (s_e - s_c).abs().max()
    assert torch.allclose(v_e, v_c, atol=1e-5, rtol=0), (v_e - v_c).abs().max()


@pytest.mark.parametrize("backend", BACKENDS)
def test_se3net_backward_parity(dev, backend):
    torch._dynamo.reset()
    m_e = MiniSE3Net().to(dev)
    m_c = MiniSE3Net().to(dev)
    m_c.load_state_dict(m_e.state_dict())
    _, s, v, graph = _mini_graph(dev)
    s1, v1 = s.clone().requires_grad_(True), v.clone().requires_grad_(True)
    s_e, v_e = m_e(s1, v1, graph)
    (s_e.sum() + v_e.sum()).backward()
    comp = torch.compile(m_c, backend=backend, dynamic=True)
    s2, v2 = s.clone().requires_grad_(True), v.clone().requires_grad_(True)
    s_c, v_c = comp(s2, v2, graph)
    (s_c.sum() + v_c.sum()).backward()
    assert torch.allclose(s1.grad, s2.grad, atol=1e-4, rtol=0)
    assert torch.allclose(v1.grad, v2.grad, atol=1e-4, rtol=0)
    n = 0
    for (n1, p1), (n2, p2) in zip(m_e.named_parameters(), m_c.named_parameters()):
        assert n1 == n2
        assert (p1.grad is None) == (p2.grad is None), n1
        if p1.grad is not None:
            assert torch.allclose(p1.grad, p2.grad, atol=1e-4, rtol=0), n1
            n += 1
    assert n >= 10   # path weights, radial MLP and biases of both layers


def test_se3conv_forward_does_not_sync(dev):
    """The forward issues no device-to-host copy: the CG table and every size stay where they
    are (a type-2 layer reads its CG buffer on the device)."""
    from gdl_amd.se3_conv import SE3Conv
    _, s, v, graph = _mini_graph(dev)
    conv = SE3Conv(8, 4, 8, 4, in_type2_channels=2, out_type2_channels=3, radius=3.0).to(dev)
    t = torch.randn(15, 2, 5, device=dev)
    conv(s, v, graph, type2=t)      # warm-up (first-call allocations)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        so, vo, to = conv(s, v, graph, type2=t)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    assert to.shape == (15, 3, 5) and torch.isfinite(to).all()
