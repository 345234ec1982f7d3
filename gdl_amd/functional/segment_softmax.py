"""Softmax over the edges of each target node (drop-in for ``_sparse_softmax``,
geoembodied/nn/modules/invariant_attention.py:202-230).

    w = sparse_softmax(scores, index, num_nodes)        # scores [E, H], index [E] -> [E, H]

computes, per target n and head h, ``exp(scores - max) / max(sum exp(scores - max), 1e-8)`` over
the edges with ``index == n`` — the reference's scatter 'amax' / exp / scatter_add / divide
sequence — in one gfx950 kernel over the CSR of ``index`` (built with the stable radix sort of
``sort_and_build_csr``).  Callers that already hold the CSR use ``segment_softmax``.  The
backward is ``w * (g - segment sum of g * w)``, the gradient autograd forms for the reference's
op sequence (its max-shift term cancels).  Scores are computed in float32 (bfloat16 / float16
inputs are promoted, as the reference's float32 max buffer promotes them) or float64.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from gdl_amd.csrc import (
    segment_softmax_backward_hip,
    segment_softmax_forward_hip,
    sort_and_build_csr_cuda,
    target_bounds,
)


class _SegmentSoftmax(torch.autograd.Function):
    @staticmethod
    def forward(ctx, scores, perm, node_start, node_end, num_nodes, contiguous_csr):
        out = segment_softmax_forward_hip(scores, perm, node_start, node_end, num_nodes,
                                          contiguous_csr)
        ctx.save_for_backward(out, perm, node_start, node_end)
        ctx.num_nodes, ctx.contiguous_csr = num_nodes, contiguous_csr
        return out

    @staticmethod
    def backward(ctx, grad):
        out, perm, node_start, node_end = ctx.saved_tensors
        g = segment_softmax_backward_hip(grad, out, perm, node_start, node_end, ctx.num_nodes,
                                         ctx.contiguous_csr)
        return g, None, None, None, None, None


def _compute_dtype(scores: Tensor) -> Tensor:
    return scores if scores.dtype in (torch.float32, torch.float64) else scores.float()


def segment_softmax(
    scores: Tensor,
    perm: Optional[Tensor],
    node_start: Tensor,
    node_end: Tensor,
    num_nodes: int,
    *,
    contiguous_csr: bool = False,
) -> Tensor:
    """Softmax of ``scores [E, H]`` (or ``[E]``) over each CSR segment: rows ``perm[e]`` for
    ``e`` in ``[node_start[n], node_end[n])`` form target ``n``; ``perm`` may be None.  Rows in
    no segment are 0.  ``contiguous_csr=True`` states that the node ranges are ascending and
    contiguous from 0, as ``sort_and_build_csr`` and ``SpatialGraph`` produce them; the kernel
    then writes those zeros itself instead of the output being zero-filled first."""
    squeeze = scores.dim() == 1
    x = _compute_dtype(scores.unsqueeze(-1) if squeeze else scores)
    if torch.is_grad_enabled() and x.requires_grad:
        out = _SegmentSoftmax.apply(x, perm, node_start, node_end, int(num_nodes),
                                    bool(contiguous_csr))
    else:  # nothing to differentiate: the kernel call without the autograd node
        out = segment_softmax_forward_hip(x, perm, node_start, node_end, int(num_nodes),
                                          bool(contiguous_csr))
    return out.squeeze(-1) if squeeze else out


def sparse_softmax(scores: Tensor, index: Tensor, num_nodes: int) -> Tensor:
    """Softmax over sparse edges grouped by target node (reference argument order)."""
    bounds = target_bounds(index, int(num_nodes)) if isinstance(index, Tensor) else None
    if bounds is not None:  # a radius graph's targets: its row pointer is the CSR, perm identity
        return segment_softmax(scores, None, bounds[0], bounds[1], num_nodes, contiguous_csr=True)
    _, perm, node_start, node_end = sort_and_build_csr_cuda(index, int(num_nodes))
    return segment_softmax(scores, perm, node_start, node_end, num_nodes, contiguous_csr=True)


_sparse_softmax = sparse_softmax
