"""Fused neighbourhood gather-sums (the interpolation / pooling / skip-fusion aggregation of the
reference, geoembodied/nn/modules/equivariant_interp.py:95-125, equivariant_pool.py:412-471,
equivariant_skip_fusion.py:304-320).

    out = gather_weighted_sum(feat, idx, w)     # sum_k w[n, k] * feat[idx[n, k]], [N_out, C]
    out = knn_interpolate(feat, idx, dist)      # with the interpolation layer's IDW weights

``feat`` may carry extra trailing dimensions (vector features [N, C_v, 3], type-2 [N, C_t2, 5]):
they are flattened into channels, since the sum is linear per component.  Padding neighbours
(idx = -1, as KNN returns them) contribute nothing and a row without neighbours is 0 — the
reference reaches the same result through ``idx.clamp(min=0)`` and zero weights.  Gradients flow
to ``feat`` (through the CSR of ``idx``, no atomics) and to ``w``.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from gdl_amd.csrc import (
    gather_weighted_sum_backward_hip,
    gather_weighted_sum_forward_hip,
    idw_interpolate_forward_hip,
    idw_weights_hip,
)


class _GatherWeightedSum(torch.autograd.Function):
    @staticmethod
    def forward(ctx, feat, idx, w):
        out = gather_weighted_sum_forward_hip(feat, idx, w)
        ctx.save_for_backward(feat, idx, w)
        return out

    @staticmethod
    def backward(ctx, grad):
        feat, idx, w = ctx.saved_tensors
        gf, gw = gather_weighted_sum_backward_hip(grad, feat, idx, w, ctx.needs_input_grad[0],
                                                  ctx.needs_input_grad[2])
        if gw is not None:
            gw = gw.to(w.dtype)
        return gf, None, gw


class _IdwInterpolate(torch.autograd.Function):
    """IDW weights and gather-sum in one kernel; the weights (functions of the KNN distances
    alone, which carry no gradient here, as in the two-step path) are kept for the backward."""

    @staticmethod
    def forward(ctx, feat, idx, dist):
        out, w = idw_interpolate_forward_hip(feat, idx, dist)
        ctx.save_for_backward(feat, idx, w.to(feat.dtype))
        return out

    @staticmethod
    def backward(ctx, grad):
        feat, idx, w = ctx.saved_tensors
        gf, _ = gather_weighted_sum_backward_hip(grad, feat, idx, w, True, False)
        return gf, None, None


def gather_weighted_sum(feat: Tensor, idx: Tensor, w: Tensor) -> Tensor:
    """``out[n] = sum_k w[n, k] * feat[idx[n, k]]`` for ``feat [N_src, ...]``, ``idx, w
    [N_out, K]``; returns ``[N_out, ...]`` in ``feat``'s dtype."""
    shape = feat.shape
    f2 = feat.reshape(shape[0], -1)
    out = _GatherWeightedSum.apply(f2, idx, w.to(feat.dtype) if not w.requires_grad else w)
    return out.reshape((idx.shape[0],) + tuple(shape[1:]))


def idw_weights(idx: Tensor, dist: Tensor) -> Tensor:
    """Inverse-distance weights from KNN output (equivariant_interp.py:95-99), float32."""
    return idw_weights_hip(idx, dist)


def knn_interpolate(feat: Tensor, idx: Tensor, dist: Tensor, weights: Optional[Tensor] = None) -> Tensor:
    """IDW interpolation of ``feat`` at the query points of a KNN result (idx, squared dist).
    Without ``weights`` the inverse-distance weights and the gather-sum run as one kernel."""
    if weights is not None:
        return gather_weighted_sum(feat, idx, weights)
    shape = feat.shape
    out = _IdwInterpolate.apply(feat.reshape(shape[0], -1), idx, dist.detach())
    return out.reshape((idx.shape[0],) + tuple(shape[1:]))
