"""Farthest point sampling (drop-in for geoembodied/functional/fps.py:29-162).

The greedy max-min selection runs in the gfx950 kernel ``geo_fps`` (one workgroup per cloud,
no host round trip inside the selection loop).  Selection starts at the first point of each
cloud and each step takes the lowest index attaining the largest squared distance to the
selected set; a cloud asked for at least as many samples as it has returns all its indices in
order.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor


def farthest_point_sampling(
    pos: Tensor,
    num_samples: int,
    batch: Optional[Tensor] = None,
    ptr: Optional[Tensor] = None,
) -> Tensor:
    """Select ``num_samples`` points per cloud by farthest point sampling.

    Args:
        pos: [N, 3] point positions (GPU).
        num_samples: samples per cloud (K).
        batch: optional [N] cloud id per point (legacy API; clouds need not be contiguous).
        ptr: optional [B+1] CSR offsets (preferred API; takes precedence over ``batch``).

    Returns:
        int64 global indices: [min(K, N)] for one cloud, or the per-cloud selections
        concatenated in cloud order.
    """
    if ptr is not None:
        return _fps_batched_ptr(pos, num_samples, ptr)
    if batch is None:
        return _fps_single(pos, num_samples)
    return _fps_batch_vector(pos, num_samples, batch)


def _fps_batched_ptr(pos: Tensor, num_samples: int, ptr: Tensor) -> Tensor:
    """k_per_batch = clamp(sizes, max=num_samples) (reference fps.py:108-109), formed on the
    device by the prepare kernel."""
    from gdl_amd.csrc import fps_uniform_hip

    return fps_uniform_hip(pos, ptr, num_samples)


def _fps_single(pos: Tensor, num_samples: int) -> Tensor:
    from gdl_amd.csrc import fps_cuda

    N = pos.shape[0]
    if num_samples >= N:
        return torch.arange(N, device=pos.device)
    ptr = torch.tensor([0, N], dtype=torch.int64, device=pos.device)
    k = torch.tensor([max(int(num_samples), 0)], dtype=torch.int64, device=pos.device)
    return fps_cuda(pos, ptr, k)


def _fps_batch_vector(pos: Tensor, num_samples: int, batch: Tensor) -> Tensor:
    """Cloud b = the points with batch == b, in index order (reference fps.py:69-81).

    A stable sort by cloud id makes every cloud contiguous without changing its internal
    order, so the ptr kernel applies; indices are mapped back through the sort permutation."""
    from gdl_amd.csrc import fps_cuda

    batch = batch.to(device=pos.device, dtype=torch.int64).reshape(-1)
    num_clouds = int(batch.max().item()) + 1
    order = torch.sort(batch, stable=True).indices
    counts = torch.bincount(batch, minlength=num_clouds)
    ptr = torch.zeros(num_clouds + 1, dtype=torch.int64, device=pos.device)
    ptr[1:] = counts.cumsum(0)
    k_per_batch = counts.clamp(max=int(num_samples))
    local = fps_cuda(pos[order], ptr, k_per_batch)
    return order[local]
