"""K-nearest-neighbour search for packed point clouds (drop-in for
geoembodied/functional/knn.py:31-85).

Both functions use ``ptr`` CSR offsets ([B+1]) to delimit clouds and return
``(indices int64 [N_q, k], squared distances float32 [N_q, k])`` sorted ascending by
(distance, source index); missing neighbours are -1 / 1e30.
"""

from __future__ import annotations

from typing import Tuple

from torch import Tensor

from gdl_amd.csrc import knn_cuda as _knn_dispatch


def knn(query: Tensor, source: Tensor, ptr_q: Tensor, ptr_s: Tensor, k: int) -> Tuple[Tensor, Tensor]:
    """k nearest sources of every query, searched inside the query's own cloud."""
    return _knn_dispatch(query, source, ptr_q, ptr_s, k)


def knn_self(pos: Tensor, ptr: Tensor, k: int) -> Tuple[Tensor, Tensor]:
    """Self-KNN: the first neighbour of each point is the point itself (distance 0)."""
    return _knn_dispatch(pos, pos, ptr, ptr, k)
