"""Pins of the SE3Conv message-passing oracle (oracle/se3.py), independent of its formulas:
hand-computed single-edge values of every path, the CG table's structure and its identity with
the spherical harmonics, and rotation equivariance of all three output types."""

import math

import numpy as np
import pytest
import torch

import oracle
from oracle import se3 as ose3


def _one_edge(path: int, s0, v0, t0):
    """Graph 0 -> 1 along +x, R one-hot on `path`'s column, all 1x1 weights = 1."""
    d = np.array([[1.0, 0.0, 0.0]])
    Y = torch.from_numpy(oracle.spherical_harmonics(d, 2, False))
    W = {k: torch.ones(1, 1, dtype=torch.float64) for k in ose3.PATH_NAMES}
    pc = ose3.path_columns(W, True, True, 1)
    R = torch.zeros(1, 9, dtype=torch.float64)
    R[0, pc[path]] = 1.0
    s = torch.tensor([[s0], [0.0]], dtype=torch.float64)
    v = torch.tensor([v0, [0.0, 0.0, 0.0]], dtype=torch.float64).view(2, 1, 3)
    t = torch.tensor([t0, [0.0] * 5], dtype=torch.float64).view(2, 1, 5)
    out = ose3.se3_conv(s, v, t, torch.tensor([0]), torch.tensor([1]), torch.from_numpy(d), Y, R, W,
                        ose3.cg_11_2_cartesian(), 1, 1, 1, torch.ones(2))
    return [o[1].numpy().reshape(-1) for o in out], Y[0].numpy()


def test_single_edge_closed_forms():
    s0, v0, t0 = 2.0, [0.0, 3.0, 0.0], [1.0, -2.0, 0.5, 0.0, 4.0]
    y0 = 0.5 / math.sqrt(math.pi)
    h = math.sqrt(0.5)
    (s, v, t), Y = _one_edge(0, s0, v0, t0)
    np.testing.assert_allclose(s, [y0 * s0]); np.testing.assert_allclose(v, 0); np.testing.assert_allclose(t, 0)
    (s, v, t), _ = _one_edge(1, s0, v0, t0)
    np.testing.assert_allclose(v, [s0, 0, 0])                     # d * s along +x
    (s, v, t), _ = _one_edge(2, s0, v0, t0)
    np.testing.assert_allclose(v, [0, y0 * 3.0, 0])
    (s, v, t), _ = _one_edge(3, s0, [5.0, 3.0, 0.0], t0)
    np.testing.assert_allclose(s, [5.0])                          # x . (5, 3, 0)
    (s, v, t), _ = _one_edge(4, s0, v0, t0)
    np.testing.assert_allclose(v, [0, 0, 3.0])                    # x cross 3y = 3z
    (s, v, t), Y = _one_edge(5, s0, v0, t0)
    np.testing.assert_allclose(t, s0 * Y[4:9])
    (s, v, t), _ = _one_edge(6, s0, v0, t0)
    np.testing.assert_allclose(t, y0 * np.array(t0))
    (s, v, t), _ = _one_edge(7, s0, v0, t0)
    np.testing.assert_allclose(t, [3.0 * h, 0, 0, 0, 0], atol=1e-15)  # xy component only
    (s, v, t), _ = _one_edge(7, s0, [4.0, 0.0, 0.0], t0)
    np.testing.assert_allclose(t, [0, 0, -4.0 / math.sqrt(6.0), 0, 4.0 / math.sqrt(2.0)], atol=1e-15)
    (s, v, t), _ = _one_edge(8, s0, v0, t0)
    np.testing.assert_allclose(s, [sum(x * x for x in t0)])


def test_cg_table_structure_and_sh_identity():
    cg = ose3.cg_11_2_cartesian().numpy()
    np.testing.assert_allclose(cg, cg.transpose(1, 0, 2))                       # symmetric
    np.testing.assert_allclose(np.einsum("iim->m", cg), 0, atol=1e-15)         # traceless
    np.testing.assert_allclose(np.einsum("ijm,ijn->mn", cg, cg), np.eye(5), atol=1e-14)  # orthonormal
    u = np.random.default_rng(0).normal(size=(200, 3))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    tp = np.einsum("ni,nj,ijm->nm", u, u, cg)
    Y2 = oracle.spherical_harmonics(u, 2, False)[:, 4:9]
    np.testing.assert_allclose(tp, Y2 / math.sqrt(15.0 / (8.0 * math.pi)), atol=1e-13)


def _rotation(seed):
    q, _ = np.linalg.qr(np.random.default_rng(seed).normal(size=(3, 3)))
    return q * np.sign(np.linalg.det(q))


def _wigner_d2(Q):
    u = np.random.default_rng(7).normal(size=(64, 3))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    A = oracle.spherical_harmonics(u, 2, False)[:, 4:9]
    B = oracle.spherical_harmonics(u @ Q.T, 2, False)[:, 4:9]
    D, *_ = np.linalg.lstsq(A, B, rcond=None)       # B = A D  ->  Y2(Q u) = D^T Y2(u)
    return D.T


@pytest.mark.parametrize("seed", [0, 1])
def test_rotation_equivariance(seed):
    g = torch.Generator().manual_seed(seed)
    N, Cs, Cv, Ct, Os, Ov, Ot = 40, 5, 4, 3, 6, 5, 2
    pos = torch.rand(N, 3, generator=g, dtype=torch.float64) * 2
    row, col = oracle.radius_graph(pos.float().numpy(), 0.9, 16)
    row, col = torch.from_numpy(row), torch.from_numpy(col)
    s = torch.randn(N, Cs, generator=g, dtype=torch.float64)
    v = torch.randn(N, Cv, 3, generator=g, dtype=torch.float64)
    t = torch.randn(N, Ct, 5, generator=g, dtype=torch.float64)
    spec = {"w_ss": (Os, Cs), "w_sv": (Ov, Cs), "w_vv_scalar": (Ov, Cv), "w_vs": (Os, Cv),
            "w_vv_cross": (Ov, Cv), "w_st2": (Ot, Cs), "w_t2t2": (Ot, Ct), "w_vt2": (Ot, Cv),
            "w_t2s": (Os, Ct)}
    W = {k: torch.randn(*sh, generator=g, dtype=torch.float64) for k, sh in spec.items()}
    Rw = torch.randn(row.numel(), 9, generator=g, dtype=torch.float64)
    avg = torch.rand(N, generator=g, dtype=torch.float64) + 1
    cg = ose3.cg_11_2_cartesian()

    def run(p, s, v, t):
        d, _, Y = oracle.edge_geometry(p.numpy(), row.numpy(), col.numpy())
        return ose3.se3_conv(s, v, t, row, col, torch.from_numpy(d), torch.from_numpy(Y), Rw, W, cg,
                             Os, Ov, Ot, avg)

    Q = _rotation(seed)
    D2 = _wigner_d2(Q)
    s1, v1, t1 = run(pos, s, v, t)
    Qt, D2t = torch.from_numpy(Q), torch.from_numpy(D2)
    s2, v2, t2 = run(pos @ Qt.T, s, v @ Qt.T, t @ D2t.T)
    np.testing.assert_allclose(s2.numpy(), s1.numpy(), atol=1e-10)
    np.testing.assert_allclose(v2.numpy(), (v1 @ Qt.T).numpy(), atol=1e-10)
    np.testing.assert_allclose(t2.numpy(), (t1 @ D2t.T).numpy(), atol=1e-10)


def test_sh_torch_helper_matches_oracle():
    from sh_torch import sh_torch
    u = np.random.default_rng(3).normal(size=(50, 3))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    np.testing.assert_allclose(sh_torch(torch.from_numpy(u), 2).numpy(),
                               oracle.spherical_harmonics(u, 2, False), atol=1e-14)


def test_radial_basis_closed_forms():
    """sin(f d) / d times the cosine envelope, through Linear -> SiLU -> Linear: identity-like
    weights expose the basis; the envelope is 1 at d = 0+ and 0 at the cutoff."""
    freqs = torch.arange(1, 5, dtype=torch.float64) * math.pi / 2.0
    d = torch.tensor([1e-6, 0.5, 1e-9, 2.0], dtype=torch.float64)
    W1 = torch.eye(4, dtype=torch.float64) * 1e-3     # silu(z) ~ z/2 for small z
    b1 = torch.zeros(4, dtype=torch.float64)
    W2 = torch.eye(4, dtype=torch.float64)
    b2 = torch.zeros(4, dtype=torch.float64)
    R = ose3.radial_basis(d, freqs, 2.0, W1, b1, W2, b2)
    z = 1e-3 * torch.sin(freqs * d.unsqueeze(-1)) / d.clamp(min=1e-8).unsqueeze(-1) * \
        (0.5 * (1 + torch.cos(math.pi * d / 2.0))).unsqueeze(-1)
    np.testing.assert_allclose(R.numpy(), (z / (1 + torch.exp(-z))).numpy(), rtol=1e-12, atol=1e-18)
    # d -> 0: sin(f d)/d -> f, envelope -> 1 (silu(z) ~ z/2);  below 1e-8 the divisor is clamped;
    # d = cutoff: envelope 0
    np.testing.assert_allclose(R[0].numpy(), (1e-3 * freqs / 2).numpy(), rtol=5e-3)
    np.testing.assert_allclose(R[2].numpy(), (1e-3 * freqs * 0.1 / 2).numpy(), rtol=5e-3)
    np.testing.assert_allclose(R[3].numpy(), 0.0, atol=1e-20)
