"""Radius graph construction (drop-in for geoembodied/functional/radius_graph.py:19-105,338-358).

``radius_graph`` returns directed edges ``row[e] -> col[e]`` (source, target) with
``|x[row] - x[col]| < r`` inside each cloud, at most ``max_num_neighbors`` sources per target
(the nearest by (squared distance, source index)).  Edges come sorted by target, then source.
The distance test is ``d < fl32(r*r)`` on the exactly rounded fp32 squared distance.
"""

from __future__ import annotations

from typing import Optional, Tuple

from torch import Tensor

from gdl_amd.csrc import radius_graph_hip


def radius_graph(
    x: Tensor,
    r: float,
    *,
    max_num_neighbors: int = 32,
    batch: Optional[Tensor] = None,
    loop: bool = False,
    mask: Optional[Tensor] = None,
    num_batch_elements: Optional[int] = None,
) -> Tuple[Tensor, Tensor]:
    """Build the radius graph.

    Args:
        x: [N, 3] positions (GPU).
        r: radius (strict: ``|xi - xj| < r``): a number, or a one-element device tensor such
            as ``adaptive_radius(...)`` returns (read by the kernels, no host sync).
        max_num_neighbors: cap on sources per target.
        batch: optional [N] cloud id per point (any order).
        loop: include self edges.
        mask: optional [N] bool, False points take part in no edge.
        num_batch_elements: number of clouds; avoids the ``batch.max()`` host sync.  Without
            ``batch`` it splits the points into that many contiguous equal clouds.

    Returns:
        (row, col) int64 edge indices.
    """
    return radius_graph_hip(
        x, r,
        max_num_neighbors=max_num_neighbors,
        loop=loop,
        mask=mask,
        batch=batch,
        num_batch_elements=num_batch_elements,
    )


def compute_edge_vectors(x: Tensor, row: Tensor, col: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
    """Edge vectors x[col] - x[row], their lengths (clamped below at 1e-8) and unit directions."""
    diff = x[col] - x[row]
    length = diff.norm(dim=-1, keepdim=True).clamp(min=1e-8)
    return diff, length.squeeze(-1), diff / length
