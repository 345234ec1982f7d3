"""GPU: the fused radial basis MLP (forward and backward) against the float64 oracle
(oracle/se3.py radial_basis, pinned by closed forms in test_oracle_se3.py).

Bars: R within 1e-5 |R| + 1e-5 max|R|; gradients within 1e-4 relative + 1e-5 of the tensor's
max (fp32 with sums over up to E edges for the weight gradients)."""

import math

import numpy as np
import pytest
import torch

from oracle import se3 as ose3

pytestmark = pytest.mark.gpu


def _close(got, want, rtol, arel):
    got = got.detach().double().cpu().numpy()
    want = want.detach().double().cpu().numpy()
    scale = max(float(np.abs(want).max()) if want.size else 0.0, 1e-30)
    np.testing.assert_allclose(got, want, rtol=rtol, atol=arel * scale)


@pytest.mark.parametrize("E,NB,H,P", [(1000, 16, 64, 5), (70001, 16, 64, 9), (333, 8, 32, 1),
                                      (16, 16, 64, 16), (5, 3, 7, 2),
                                      # beyond the matrix-core kernels: the LDS-tiled kernels
                                      (3000, 32, 64, 5), (2001, 16, 128, 9), (777, 16, 64, 20),
                                      (40000, 48, 200, 33), (3, 17, 65, 17)])
def test_radial_mlp_vs_oracle(dev, E, NB, H, P):
    from gdl_amd.se3_conv import radial_mlp
    g = torch.Generator().manual_seed(E + P)
    cutoff = 0.3
    dist = torch.rand(E, generator=g) * cutoff * 1.1
    dist[0] = 0.0
    freqs = torch.arange(1, NB + 1, dtype=torch.float32) * math.pi / cutoff
    W1 = torch.randn(H, NB, generator=g) / NB ** 0.5
    b1 = torch.randn(H, generator=g) * 0.1
    W2 = torch.randn(P, H, generator=g) / H ** 0.5
    b2 = torch.randn(P, generator=g) * 0.1
    leaves = {"d": dist, "W1": W1, "b1": b1, "W2": W2, "b2": b2}
    gp = {k: v.to(dev).requires_grad_(True) for k, v in leaves.items()}
    cp = {k: v.double().requires_grad_(True) for k, v in leaves.items()}
    R = radial_mlp(gp["d"], freqs.to(dev), cutoff, gp["W1"], gp["b1"], gp["W2"], gp["b2"])
    Rw = ose3.radial_basis(cp["d"], freqs, cutoff, cp["W1"], cp["b1"], cp["W2"], cp["b2"])
    assert R.shape == (E, P)
    _close(R, Rw, 1e-5, 1e-5)
    c = torch.randn(E, P, generator=g, dtype=torch.float64)
    (R * c.to(dev).float()).sum().backward()
    (Rw * c).sum().backward()
    for k in leaves:
        _close(gp[k].grad, cp[k].grad, 1e-4, 1e-5)


def test_radial_basis_module_matches_reference_formula(dev):
    from gdl_amd.se3_conv import RadialBasis
    torch.manual_seed(0)
    rb = RadialBasis(num_basis=16, cutoff=0.5, num_hidden=64, num_output=5).to(dev)
    d = torch.rand(4000, device=dev) * 0.6
    R = rb(d)
    l1, l2 = rb.mlp[0], rb.mlp[2]
    want = ose3.radial_basis(d.cpu(), rb.freqs.cpu(), 0.5, l1.weight.cpu(), l1.bias.cpu(),
                             l2.weight.cpu(), l2.bias.cpu())
    _close(R, want, 1e-5, 1e-5)
    assert rb(torch.empty(0, device=dev)).shape == (0, 5)


def test_se3conv_with_32_radial_basis_functions(dev):
    """SE3Conv(num_radial_basis=32) -- the radial MLP beyond 16 basis functions -- runs forward and
    backward, and its radial weights match the float64 oracle."""
    from gdl_amd.graph import SpatialGraph
    from gdl_amd.se3_conv import SE3Conv
    torch.manual_seed(3)
    pos = torch.rand(2000, 3, device=dev)
    gr = SpatialGraph.build(pos, 0.12, max_num_neighbors=16)
    conv = SE3Conv(8, 4, 8, 4, radius=0.12, num_radial_basis=32).to(dev)
    fs = torch.randn(gr.N, 8, device=dev, requires_grad=True)
    fv = torch.randn(gr.N, 4, 3, device=dev, requires_grad=True)
    s, v = conv(fs, fv, gr)
    (s.square().sum() + v.square().sum()).backward()
    assert torch.isfinite(fs.grad).all() and torch.isfinite(fv.grad).all()
    rb = conv.radial_basis
    l1, l2 = rb.mlp[0], rb.mlp[2]
    want = ose3.radial_basis(gr.dist.detach().cpu(), rb.freqs.cpu(), rb.cutoff, l1.weight.cpu(),
                             l1.bias.cpu(), l2.weight.cpu(), l2.bias.cpu())
    _close(rb(gr.dist.detach()), want, 1e-5, 1e-5)


def _radial_ref_fp32_args(d, freqs, cutoff, W1, b1, W2, b2):
    """The radial MLP in float64 with the sine and cosine arguments rounded to float32 as an fp32
    evaluation rounds them (f * d and (pi / cutoff) * d, each one fp32 product; pi / cutoff in
    fp32): for arguments of thousands of radians that rounding, not the sine, sets the value.
    Gradients flow through the exact products."""
    f64, f32 = torch.float64, torch.float32

    def rounded(exact, value32):  # value of the fp32 product, derivative of the exact one
        return exact + (value32.to(f64) - exact).detach()

    d32 = d.detach().to(f32)
    a = rounded(freqs.to(f64)[None, :] * d[:, None], freqs.to(f32)[None, :] * d32[:, None])
    pic32 = torch.tensor(math.pi, dtype=f32) / torch.tensor(cutoff, dtype=f32)
    t = rounded(pic32.to(f64) * d, pic32 * d32)
    env = (0.5 * (1.0 + torch.cos(t))).clamp(min=0.0)[:, None]
    x = torch.sin(a) / d.clamp(min=1e-8)[:, None] * env
    h = torch.nn.functional.silu(torch.nn.functional.linear(x, W1, b1))
    return torch.nn.functional.linear(h, W2, b2)


@pytest.mark.parametrize("P", [3, 5, 9, 16])
def test_radial_mlp_tiles_outside_the_fast_range(dev, P):
    """A 16-edge tile takes the hardware sine / cosine without range checks only when every
    argument is below 1000 rad; a tile holding one large distance (or only large ones) takes the
    range-checked functions for all its edges.  Mixed tiles, d = 0 and a ragged end, forward and
    backward (P = 3, 5, 9, 16: every backward variant), against float64 with the arguments rounded
    to fp32 as an fp32 evaluation rounds them.  Bars as above."""
    from gdl_amd.se3_conv import radial_mlp
    g = torch.Generator().manual_seed(100 + P)
    E, NB, H, cutoff = 16 * 40 + 7, 16, 64, 0.3
    dist = torch.rand(E, generator=g) * cutoff * 1.1
    dist[0] = 0.0
    dist[16 * 3 + 5] = 60.0                    # one large edge: the whole tile checked
    dist[16 * 7: 16 * 8] = 50.0 + torch.rand(16, generator=g) * 50.0   # a tile of large edges
    dist[16 * 11 + 15] = 1e4                   # the pi d / cutoff argument alone is large too
    dist[-1] = 75.0                            # in the ragged last tile
    freqs = torch.arange(1, NB + 1, dtype=torch.float32) * math.pi / cutoff
    assert float(freqs.max() * 60.0) > 1000.0 and float(freqs.max() * cutoff * 1.1) < 1000.0
    W1 = torch.randn(H, NB, generator=g) / NB ** 0.5
    b1 = torch.randn(H, generator=g) * 0.1
    W2 = torch.randn(P, H, generator=g) / H ** 0.5
    b2 = torch.randn(P, generator=g) * 0.1
    leaves = {"d": dist, "W1": W1, "b1": b1, "W2": W2, "b2": b2}
    gp = {k: v.to(dev).requires_grad_(True) for k, v in leaves.items()}
    cp = {k: v.double().requires_grad_(True) for k, v in leaves.items()}
    R = radial_mlp(gp["d"], freqs.to(dev), cutoff, gp["W1"], gp["b1"], gp["W2"], gp["b2"])
    Rw = _radial_ref_fp32_args(cp["d"], freqs, cutoff, cp["W1"], cp["b1"], cp["W2"], cp["b2"])
    _close(R, Rw, 1e-5, 1e-5)
    c = torch.randn(E, P, generator=g, dtype=torch.float64)
    (R * c.to(dev).float()).sum().backward()
    (Rw * c).sum().backward()
    for k in leaves:
        _close(gp[k].grad, cp[k].grad, 1e-4, 1e-5)
