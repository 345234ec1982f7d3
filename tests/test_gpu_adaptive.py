"""GPU: device-side adaptive radius (no host round trip) and the radius graph reading its radius
from device memory.  The statistic matches the oracle (mean to float32 rounding, median
exactly); a graph built from the device radius is bit-identical to the graph built from the
same radius passed as a Python float."""

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _f():
    import geoembodied  # noqa: F401
    from geoembodied.functional.adaptive import adaptive_radius, median_cutoff
    from geoembodied.functional.knn import knn, knn_self
    from geoembodied.functional.radius_graph import radius_graph
    return adaptive_radius, median_cutoff, knn, knn_self, radius_graph


@pytest.mark.parametrize("N,B", [(50, 1), (4096, 4), (20001, 3)])
def test_adaptive_radius_and_device_radius_graph(dev, N, B):
    adaptive_radius, median_cutoff, knn, knn_self, radius_graph = _f()
    g = torch.Generator().manual_seed(N)
    pos = torch.randn(N, 3, generator=g)
    cuts = sorted(torch.randint(1, N, (B - 1,), generator=g).tolist())
    ptr = torch.tensor([0] + cuts + [N])
    p, pt = pos.to(dev), ptr.to(dev)
    r = adaptive_radius(p, pt, 4.0)
    assert r.dtype == torch.float64 and r.device.type == "cuda" and r.numel() == 1
    _, d = knn_self(p, pt, 2)
    want = oracle.knn_radius_stat(d.cpu().numpy(), 1, "mean", 4.0)
    assert float(r) == pytest.approx(want, rel=2e-7)
    m = median_cutoff(p, pt, 1.5)
    _, d2 = knn(p, p, pt, pt, 2)
    assert float(m) == oracle.knn_radius_stat(d2.cpu().numpy(), 1, "median", 1.5)
    batch = torch.repeat_interleave(torch.arange(B), torch.diff(ptr)).to(dev)
    for rad in (r, m):
        row_d, col_d = radius_graph(p, rad, batch=batch, num_batch_elements=B, max_num_neighbors=16)
        row_h, col_h = radius_graph(p, float(rad), batch=batch, num_batch_elements=B, max_num_neighbors=16)
        assert torch.equal(row_d, row_h) and torch.equal(col_d, col_h)
        wr, wc = oracle.radius_graph(pos.numpy(), float(rad), 16, batch=batch.cpu().numpy(),
                                     num_batch_elements=B)
        np.testing.assert_array_equal(row_d.cpu().numpy(), wr)
        np.testing.assert_array_equal(col_d.cpu().numpy(), wc)


def test_device_radius_edge_cases(dev):
    *_, radius_graph = _f()
    p = torch.randn(300, 3, device=dev)
    for bad in (0.0, -1.0, float("nan")):
        row, col = radius_graph(p, torch.tensor(bad, dtype=torch.float64, device=dev))
        assert row.numel() == 0 and col.numel() == 0
    row, col = radius_graph(p, torch.tensor([1e30], device=dev), max_num_neighbors=300)
    assert row.numel() == 300 * 299   # every pair, the cloud in one cell
