"""Adaptive graph radii computed on the GPU, without a host round trip.

The reference estimates a radius from nearest-neighbour spacing and reads it back with
``.item()`` before building the graph (geoembodied/nn/modules/multi_scale_se3_net.py:99-124,
equivariant_skip_fusion.py:243-248).  These return the same quantity as a float64 device scalar
that ``radius_graph`` accepts as ``r`` and its kernels read directly:

    r = adaptive_radius(pos, ptr, multiplier=4.0)    # mean NN distance * multiplier
    row, col = radius_graph(pos, r, batch=batch, num_batch_elements=B)

``float(r)`` gives the reference's Python float when a host value is wanted.
"""

from __future__ import annotations

from torch import Tensor

from gdl_amd.csrc import knn_radius_stat_hip
from gdl_amd.functional.knn import knn, knn_self


def adaptive_radius(pos: Tensor, ptr: Tensor, multiplier: float = 4.0) -> Tensor:
    """multiplier * mean over points of the distance to the nearest other point of the same
    cloud (knn_self with k = 2; distances clamped to [1e-4, 1e10] as sqrt of [1e-8, 1e20])."""
    _, dists = knn_self(pos, ptr, 2)
    return knn_radius_stat_hip(dists, 1, "mean", multiplier)


def median_cutoff(pos: Tensor, ptr: Tensor, multiplier: float = 1.0) -> Tensor:
    """multiplier * median (lower median for an even count) of the nearest-neighbour distance
    (KNN of the points against themselves with k = 2, last column, clamped below at 1e-6)."""
    _, dists = knn(pos, pos, ptr, ptr, 2)
    return knn_radius_stat_hip(dists, dists.shape[1] - 1, "median", multiplier)
