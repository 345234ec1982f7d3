"""GPU parity of the fused neighbourhood gather-sum and the interpolation weights against the
float64 oracle (itself pinned to the reference's op sequence in test_oracle.py).

Bars: fp32 |out - ref| <= 1e-5 * sum_k |w| |feat| (the segment-sum bar), bf16 2e-2 on the same
scale plus the final rounding, fp64 1e-12; IDW weights within 2 ulp-scale (1e-6 relative);
gradients on the same scales.
"""

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float64: 1e-12}


def _f():
    import geoembodied  # noqa: F401
    from geoembodied.functional.gather import gather_weighted_sum, idw_weights, knn_interpolate
    return gather_weighted_sum, idw_weights, knn_interpolate


def _np(t):
    return t.detach().cpu().double().numpy()


def _close(got, ref, scale, dtype):
    bound = TOL[dtype] * scale + 1e-30
    if dtype == torch.bfloat16:
        bound = bound + np.abs(ref) * 2.0 ** -8
    assert np.all(np.abs(got - ref) <= bound), float(np.max(np.abs(got - ref) - bound))


# the last two shapes are large enough for two output rows per lane group (the kernel's choice
# when K <= 4 and at least 16384 waves would run at one row each)
@pytest.mark.parametrize("Ns,No,K,C", [(1, 1, 1, 1), (100, 60, 3, 5), (3000, 5000, 8, 64),
                                       (2000, 3000, 16, 112), (500, 700, 32, 13), (4000, 4000, 3, 300),
                                       (9000, 40001, 3, 112), (3000, 70001, 2, 64)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float64])
def test_gather_weighted_sum_vs_oracle(dev, Ns, No, K, C, dtype):
    gws, _, _ = _f()
    g = torch.Generator().manual_seed(Ns + K + C)
    idx = torch.randint(-1, Ns, (No, K), generator=g)          # -1 = padding
    idx[: max(1, No // 10)] = -1                               # rows with no neighbour
    feat = torch.randn(Ns, C, generator=g, dtype=torch.float64).to(dtype)
    w = torch.rand(No, K, generator=g, dtype=torch.float64).to(dtype)
    fd = feat.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    out = gws(fd, idx.to(dev), wd)
    assert out.shape == (No, C) and out.dtype == dtype
    ref, scale = oracle.gather_weighted_sum(_np(feat), idx.numpy(), _np(w))
    _close(_np(out), ref, scale, dtype)
    go = torch.randn(No, C, generator=g, dtype=torch.float64).to(dtype)
    out.backward(go.to(dev))
    gf, gw = oracle.gather_weighted_sum_bwd(_np(go), _np(feat), idx.numpy(), _np(w))
    # scales: sum of |w| |grad_out| per source row, sum of |grad_out| |feat| per weight
    ok = (idx.numpy() >= 0)
    sf = np.zeros_like(gf)
    n_i, k_i = np.nonzero(ok)
    np.add.at(sf, idx.numpy()[n_i, k_i], np.abs(_np(w))[n_i, k_i][:, None] * np.abs(_np(go))[n_i])
    _close(_np(fd.grad), gf, sf, dtype)
    sw = np.where(ok, np.einsum("nc,nkc->nk", np.abs(_np(go)), np.abs(_np(feat))[np.where(ok, idx.numpy(), 0)]), 0)
    _close(_np(wd.grad), gw, sw, dtype)


def test_vector_features_and_knn_interpolate(dev):
    """Trailing dims are channels; knn_interpolate = IDW weights + gather-sum on KNN output."""
    import geoembodied  # noqa: F401
    from geoembodied.functional.knn import knn
    gws, idw, knn_interp = _f()
    g = torch.Generator().manual_seed(3)
    dense, coarse = torch.randn(4000, 3, generator=g), torch.randn(1000, 3, generator=g)
    pd, pc = torch.tensor([0, 2500, 4000]), torch.tensor([0, 600, 1000])
    idx, dist = knn(dense.to(dev), coarse.to(dev), pd.to(dev), pc.to(dev), 3)
    v = torch.randn(1000, 16, 3, generator=g)
    out = knn_interp(v.to(dev), idx, dist)
    assert out.shape == (4000, 16, 3)
    w_ref = oracle.idw_weights(idx.cpu().numpy(), dist.cpu().numpy())
    w = idw(idx, dist)
    np.testing.assert_allclose(_np(w), w_ref, rtol=1e-6, atol=1e-7)
    ref, scale = oracle.gather_weighted_sum(v.reshape(1000, -1).numpy(), idx.cpu().numpy(), w_ref)
    _close(_np(out).reshape(4000, -1), ref, scale + 1e-6 * np.abs(ref), torch.float32)


def test_idw_padding_and_ties(dev):
    _, idw, _ = _f()
    idx = torch.tensor([[3, -1, -1], [1, 2, 0], [-1, -1, -1], [5, 6, 7]], device=dev)
    dist = torch.tensor([[0.5, 1e30, 1e30], [1.0, 1.0, 1.0], [1e30, 1e30, 1e30], [0.0, 1e-5, 4.0]],
                        device=dev)
    w = idw(idx, dist).cpu().numpy()
    np.testing.assert_allclose(w, oracle.idw_weights(idx.cpu().numpy(), dist.cpu().numpy()),
                               rtol=1e-6)
    assert w[0].tolist() == [1.0, 0.0, 0.0] and w[2].tolist() == [0.0, 0.0, 0.0]


def test_gather_gradcheck_fp64(dev):
    gws, _, _ = _f()
    g = torch.Generator().manual_seed(5)
    idx = torch.randint(-1, 20, (15, 4), generator=g).to(dev)
    f = torch.randn(20, 3, generator=g, dtype=torch.float64).to(dev).requires_grad_(True)
    w = torch.randn(15, 4, generator=g, dtype=torch.float64).to(dev).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b: gws(a, idx, b), (f, w))


@pytest.mark.parametrize("No,K,C", [(1, 1, 1), (777, 3, 112), (40001, 3, 112), (5000, 4, 48),
                                    (3000, 8, 64), (2000, 16, 20), (600, 32, 7), (70001, 2, 64)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float64])
def test_fused_idw_interpolate_bitwise_vs_two_calls(dev, No, K, C, dtype):
    """knn_interpolate without weights runs IDW weights + gather-sum as one kernel: output,
    weights and feature gradient bitwise equal to idw_weights then gather_weighted_sum, with
    padding (-1), indices past the sources (weighted by IDW, skipped by the gather), zero and
    huge distances."""
    from geoembodied.csrc import idw_interpolate_forward_hip
    gws, idw, knn_interp = _f()
    Ns = 3000
    g = torch.Generator().manual_seed(No + K + C)
    idx = torch.randint(-1, Ns + 5, (No, K), generator=g)
    dist = torch.rand(No, K, generator=g) * 0.05
    dist[:, 0] = torch.where(torch.rand(No, generator=g) < 0.05, 0.0, dist[:, 0])
    dist[: max(1, No // 50)] = 1e30
    idx[-max(1, No // 40):] = -1
    feat = torch.randn(Ns, C, generator=g, dtype=torch.float64).to(dtype).to(dev)
    idx, dist = idx.to(dev), dist.to(dev)
    out_f, w_f = idw_interpolate_forward_hip(feat, idx, dist)
    w_2 = idw(idx, dist)
    assert torch.equal(w_f, w_2)
    assert torch.equal(out_f, gws(feat, idx, w_2))
    fa = feat.clone().requires_grad_(True)
    fb = feat.clone().requires_grad_(True)
    out_a = knn_interp(fa, idx, dist)
    out_b = gws(fb, idx, idw(idx, dist))
    assert torch.equal(out_a, out_b)
    go = torch.randn(No, C, generator=g, dtype=torch.float64).to(dtype).to(dev)
    out_a.backward(go)
    out_b.backward(go)
    assert torch.equal(fa.grad, fb.grad)
