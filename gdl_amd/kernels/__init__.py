"""Geometry kernels re-exported under ``geoembodied.kernels``.

The reference package's ``kernels`` module holds its Triton spherical harmonics
(``kernels.triton_sph_harm``, replaced here by ``gdl_amd.kernels.sph_harm`` under the same module
path); this build exposes the point-cloud kernels here as well so that code importing them from
``geoembodied.kernels`` finds the same functions as ``geoembodied.functional``."""

from gdl_amd.functional import (
    compute_edge_vectors,
    farthest_point_sampling,
    knn,
    knn_self,
    radius_graph,
    segment_reduce,
    sort_and_build_csr,
)
from gdl_amd.kernels.sph_harm import get_l_channels, spherical_harmonics

__all__ = [
    "farthest_point_sampling", "knn", "knn_self", "radius_graph", "compute_edge_vectors",
    "segment_reduce", "sort_and_build_csr", "spherical_harmonics", "get_l_channels",
]
