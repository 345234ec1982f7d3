"""Geometry kernels re-exported under ``geoembodied.kernels``.

The reference package's ``kernels`` module holds only its Triton spherical harmonics; this
build exposes the four point-cloud kernels here as well so that code importing them from
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

__all__ = [
    "farthest_point_sampling", "knn", "knn_self", "radius_graph", "compute_edge_vectors",
    "segment_reduce", "sort_and_build_csr",
]
