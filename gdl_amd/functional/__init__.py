"""Public geometry ops with the reference's call signatures (geoembodied.functional)."""

from gdl_amd.functional.adaptive import adaptive_radius, median_cutoff
from gdl_amd.functional.fps import farthest_point_sampling
from gdl_amd.functional.gather import gather_weighted_sum, idw_weights, knn_interpolate
from gdl_amd.functional.knn import knn, knn_self
from gdl_amd.functional.radius_graph import compute_edge_vectors, radius_graph
from gdl_amd.functional.segment_reduce import (
    SegmentReduceFunction,
    segment_reduce,
    sort_and_build_csr,
)
from gdl_amd.functional.segment_softmax import segment_softmax, sparse_softmax

__all__ = [
    "farthest_point_sampling", "knn", "knn_self", "radius_graph", "compute_edge_vectors",
    "segment_reduce", "sort_and_build_csr", "SegmentReduceFunction", "segment_softmax",
    "sparse_softmax", "gather_weighted_sum", "idw_weights", "knn_interpolate",
    "adaptive_radius", "median_cutoff",
]
