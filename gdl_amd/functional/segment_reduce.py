"""Deterministic segment reduce for message aggregation (drop-in for
geoembodied/functional/segment_reduce.py:41-313).

    col_sorted, perm, node_start, node_end = sort_and_build_csr(col, N)   # once per graph
    out = segment_reduce(msg, col_sorted, perm, node_start, node_end, N)  # per layer

``reduce`` selects sum (default, the reference's only reduction), mean (sum / max(count, 1),
empty segment -> 0, as global_mean_pool in nn/modules/se3_net.py:226-270) or max (empty
segment -> 0, gradient split evenly over tied maxima, as scatter_reduce 'amax' with
include_self=False in nn/modules/invariant_attention.py:212-219; ``max_ties="first"`` routes it
to the first maximum instead).

The forward and backward are ``torch.library`` custom ops in the ``geoembodied`` namespace
(``segment_reduce_sum`` keeps the reference's name and signature) with fake implementations,
so ``torch.compile`` traces through them without graph breaks.  Every reduction runs in the
gfx950 kernels; CPU tensors raise.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from gdl_amd.csrc import (
    segment_reduce_available,
    segment_reduce_backward_hip,
    segment_reduce_forward_hip,
    sort_and_build_csr_cuda,
)

_REDUCE_NAMES = ("sum", "mean", "max")


def sort_and_build_csr(col: Tensor, N: int) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """Stable sort of edges by target plus CSR offsets.

    Returns int32 ``(col_sorted [E], perm [E], node_start [N], node_end [N])`` with
    ``col_sorted[e] = col[perm[e]]``, ``perm`` ascending within each target and
    ``[node_start[n], node_end[n])`` the sorted edge range of target n."""
    if col.shape[0] == 0:
        dev = col.device
        return (
            torch.empty(0, dtype=torch.int32, device=dev),
            torch.empty(0, dtype=torch.int32, device=dev),
            torch.zeros(int(N), dtype=torch.int32, device=dev),
            torch.zeros(int(N), dtype=torch.int32, device=dev),
        )
    return sort_and_build_csr_cuda(col, N)


# ═══════════════════════════════════════════════════════════════════
# Custom ops
# ═══════════════════════════════════════════════════════════════════


@torch.library.custom_op("geoembodied::segment_reduce_sum", mutates_args=())
def _segment_reduce_sum_op(msg: Tensor, col_sorted: Tensor, perm: Tensor, node_start: Tensor,
                           node_end: Tensor, N: int) -> Tensor:
    return segment_reduce_forward_hip(msg, perm, node_start, node_end, N, "sum")[0]


@torch.library.custom_op("geoembodied::segment_reduce_mean", mutates_args=())
def _segment_reduce_mean_op(msg: Tensor, col_sorted: Tensor, perm: Tensor, node_start: Tensor,
                            node_end: Tensor, N: int) -> Tensor:
    return segment_reduce_forward_hip(msg, perm, node_start, node_end, N, "mean")[0]


@torch.library.custom_op("geoembodied::segment_reduce_max", mutates_args=())
def _segment_reduce_max_op(msg: Tensor, col_sorted: Tensor, perm: Tensor, node_start: Tensor,
                           node_end: Tensor, N: int, tie_mode: int) -> Tuple[Tensor, Tensor]:
    out, arg = segment_reduce_forward_hip(msg, perm, node_start, node_end, N, "max", tie_mode)
    return out, arg


@torch.library.custom_op("geoembodied::segment_reduce_backward", mutates_args=())
def _segment_reduce_backward_op(grad_out: Tensor, col_sorted: Tensor, perm: Tensor,
                                node_start: Tensor, node_end: Tensor, msg: Optional[Tensor],
                                out: Optional[Tensor], arg: Optional[Tensor], E: int,
                                reduce: int) -> Tensor:
    return segment_reduce_backward_hip(grad_out, col_sorted, perm, node_start, node_end, E,
                                       _REDUCE_NAMES[reduce], msg=msg, out=out, arg=arg)


def _fake_forward(msg, col_sorted, perm, node_start, node_end, N):
    C = msg.shape[1] if msg.dim() > 1 else 1
    return msg.new_empty(N, C)


_segment_reduce_sum_op.register_fake(_fake_forward)
_segment_reduce_mean_op.register_fake(_fake_forward)


@_segment_reduce_max_op.register_fake
def _fake_max(msg, col_sorted, perm, node_start, node_end, N, tie_mode):
    C = msg.shape[1] if msg.dim() > 1 else 1
    return msg.new_empty(N, C), msg.new_empty(N, C, dtype=torch.int32)


@_segment_reduce_backward_op.register_fake
def _fake_backward(grad_out, col_sorted, perm, node_start, node_end, msg, out, arg, E, reduce):
    return grad_out.new_empty(E, grad_out.shape[1])


def _setup_sum_mean(ctx, inputs, output) -> None:
    msg, col_sorted, perm, node_start, node_end, N = inputs
    ctx.save_for_backward(col_sorted, perm, node_start, node_end)
    ctx.E = msg.shape[0]


def _backward_sum(ctx, grad_out):
    col_sorted, perm, node_start, node_end = ctx.saved_tensors
    g = torch.ops.geoembodied.segment_reduce_backward(
        grad_out, col_sorted, perm, node_start, node_end, None, None, None, ctx.E, 0)
    return g, None, None, None, None, None


def _backward_mean(ctx, grad_out):
    col_sorted, perm, node_start, node_end = ctx.saved_tensors
    g = torch.ops.geoembodied.segment_reduce_backward(
        grad_out, col_sorted, perm, node_start, node_end, None, None, None, ctx.E, 1)
    return g, None, None, None, None, None


def _setup_max(ctx, inputs, output) -> None:
    msg, col_sorted, perm, node_start, node_end, N, tie_mode = inputs
    out, arg = output
    ctx.save_for_backward(msg, out, arg, col_sorted, perm, node_start, node_end)
    ctx.E = msg.shape[0]


def _backward_max(ctx, grad_out, grad_arg):
    msg, out, arg, col_sorted, perm, node_start, node_end = ctx.saved_tensors
    g = torch.ops.geoembodied.segment_reduce_backward(
        grad_out, col_sorted, perm, node_start, node_end, msg, out, arg, ctx.E, 2)
    return g, None, None, None, None, None, None


_segment_reduce_sum_op.register_autograd(_backward_sum, setup_context=_setup_sum_mean)
_segment_reduce_mean_op.register_autograd(_backward_mean, setup_context=_setup_sum_mean)
_segment_reduce_max_op.register_autograd(_backward_max, setup_context=_setup_max)


class SegmentReduceFunction(torch.autograd.Function):
    """Segment sum as an autograd.Function (reference name; functional/segment_reduce.py:112-158).

    Forward: out[n] = sum of msg[perm[e]] over e in [node_start[n], node_end[n]).
    Backward: grad_msg[perm[e]] = grad_out[col_sorted[e]]."""

    @staticmethod
    def forward(ctx, msg, col_sorted, perm, node_start, node_end, N):
        ctx.save_for_backward(col_sorted, perm)
        ctx.E = msg.shape[0]
        return segment_reduce_forward_hip(msg, perm, node_start, node_end, N, "sum")[0]

    @staticmethod
    def backward(ctx, grad_out):
        col_sorted, perm = ctx.saved_tensors
        g = segment_reduce_backward_hip(grad_out, col_sorted, perm, None, None, ctx.E, "sum")
        return g, None, None, None, None, None


def segment_reduce(
    msg: Tensor,
    col_sorted: Tensor,
    perm: Tensor,
    node_start: Tensor,
    node_end: Tensor,
    N: int,
    *,
    reduce: str = "sum",
    max_ties: str = "split",
) -> Tensor:
    """Aggregate edge messages per target node without atomics.

    Args:
        msg: [E, C] float32 / bfloat16 / float64 messages in original edge order.
        col_sorted, perm, node_start, node_end: output of ``sort_and_build_csr``.
        N: number of target nodes.
        reduce: "sum" | "mean" | "max".
        max_ties: for "max", "split" (gradient shared evenly by tied maxima) or "first".

    Returns:
        [N, C] aggregated features in msg's dtype.
    """
    if reduce == "sum":
        return torch.ops.geoembodied.segment_reduce_sum(msg, col_sorted, perm, node_start,
                                                        node_end, N)
    if reduce == "mean":
        return torch.ops.geoembodied.segment_reduce_mean(msg, col_sorted, perm, node_start,
                                                         node_end, N)
    if reduce == "max":
        if max_ties not in ("split", "first"):
            raise ValueError(f"max_ties must be 'split' or 'first', got {max_ties!r}")
        out, _ = torch.ops.geoembodied.segment_reduce_max(
            msg, col_sorted, perm, node_start, node_end, N, 0 if max_ties == "split" else 1)
        return out
    raise ValueError(f"reduce must be 'sum', 'mean' or 'max', got {reduce!r}")


__all__ = ["sort_and_build_csr", "segment_reduce", "SegmentReduceFunction",
           "segment_reduce_available"]
