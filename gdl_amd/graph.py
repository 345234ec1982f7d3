"""SpatialGraph — the immutable spatial topology shared by message-passing layers (drop-in for
geoembodied/nn/modules/spatial_graph.py), built with one fused edge epilogue.

``SpatialGraph.build`` runs the radius graph, whose output is already in CSR order (targets
ascending, sources ascending), so the CSR of the targets comes from the graph's own row
pointer — ``col_sorted = col``, ``perm = arange(E)``, no sort — and one kernel writes each
edge's unit direction, length and spherical harmonics (l <= 2).  The per-cloud average degree
comes from the same row pointer.  The reference runs compute_edge_vectors (five PyTorch ops),
the spherical harmonics kernel, a radix sort for the CSR and five ops for the degree.

``direction``, ``dist`` and ``Y`` are differentiable with respect to ``pos``: the backward turns
their gradients into per-edge gradients of ``pos[col] - pos[row]`` and adds them to the two
endpoints with segment sums (the targets' CSR, and a CSR of the sources built on first use).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch
from torch import Tensor

from gdl_amd import _native as _nat
from gdl_amd.csrc import (
    _positions,
    edge_geometry_backward_hip,
    edge_geometry_hip,
    graph_avg_degree_hip,
    radius_graph_csr_hip,
    segment_reduce_forward_hip,
    sort_and_build_csr_cuda,
    source_csr,
)

# SpatialGraph.build computes the edge geometry, CSR arrays and degrees on the device right behind
# the radius graph's emit pass, before the host knows E, into buffers of N * max_num_neighbors
# rows (the graph's fields are views of their first E rows), when those buffers stay below this
# size; larger graphs get exact-sized fields after the host has read E.
_FUSED_EPILOGUE_MAX_BYTES = 256 << 20


class _EdgeGeometry(torch.autograd.Function):
    @staticmethod
    def forward(ctx, pos, row, col, max_l, col_csr):
        direction, dist, Y = edge_geometry_hip(pos, row, col, max_l)
        ctx.save_for_backward(direction, dist, row, col)
        ctx.max_l, ctx.N, ctx.col_csr = max_l, pos.shape[0], col_csr
        return direction, dist, Y

    @staticmethod
    def backward(ctx, g_dir, g_dist, g_Y):
        direction, dist, row, col = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None, None, None, None
        g_diff = edge_geometry_backward_hip(direction, dist, g_dir, g_dist, g_Y, ctx.max_l)
        N = ctx.N
        perm_c, ns_c, ne_c = ctx.col_csr if ctx.col_csr is not None else \
            sort_and_build_csr_cuda(col, N)[1:]
        perm_r, ns_r, ne_r = source_csr(row, N)
        into_col = segment_reduce_forward_hip(g_diff, perm_c, ns_c, ne_c, N, "sum")[0]
        from_row = segment_reduce_forward_hip(g_diff, perm_r, ns_r, ne_r, N, "sum")[0]
        return into_col - from_row, None, None, None, None


def edge_geometry(pos: Tensor, row: Tensor, col: Tensor, max_l: int = 2,
                  col_csr: Optional[Tuple[Tensor, Tensor, Tensor]] = None):
    """(direction [E, 3], dist [E], Y [E, (max_l+1)^2]) of the edges row -> col, differentiable
    with respect to ``pos``; ``col_csr`` = (perm, node_start, node_end) of ``col`` if known."""
    return _EdgeGeometry.apply(pos, row, col, max_l, col_csr)


@dataclass(frozen=True)
class SpatialGraph:
    """Spatial topology + cached edge geometry (field meanings as in the reference)."""

    row: Tensor          # [E] int64 source indices
    col: Tensor          # [E] int64 target indices
    direction: Tensor    # [E, 3] float32 unit vectors pos[col] - pos[row], normalised
    dist: Tensor         # [E] float32 edge lengths (clamped below at 1e-8)
    col_sorted: Tensor   # [E] int32 targets in CSR order
    perm: Tensor         # [E] int32 CSR position -> edge index
    node_start: Tensor   # [N] int32
    node_end: Tensor     # [N] int32
    Y: Tensor            # [E, (max_l+1)^2] float32 spherical harmonics of direction
    N: int
    E: int
    avg_degree: Optional[Tensor] = None  # [N] float32 average degree of each node's cloud

    @staticmethod
    def build(
        pos: Tensor,
        radius,
        max_num_neighbors: int = 32,
        mask: Optional[Tensor] = None,
        batch: Optional[Tensor] = None,
        max_l: int = 2,
        num_batch_elements: Optional[int] = None,
    ) -> "SpatialGraph":
        """Radius graph + edge geometry + CSR + per-cloud average degree
        (geoembodied/nn/modules/spatial_graph.py:85-167).  ``radius`` may be a device tensor."""
        N = pos.shape[0]
        dev = pos.device
        nsh = (max_l + 1) ** 2
        K = int(max_num_neighbors)
        differentiable = torch.is_grad_enabled() and pos.requires_grad
        fused = {}
        after_emit = None
        if (not differentiable and N >= 1 and K >= 1
                and N * K * (4 + nsh + 2) * 4 <= _FUSED_EPILOGUE_MAX_BYTES):
            p32 = _positions("spatial_graph", pos)

            def after_emit(row_s, col_s, row_ptr_d, cap, ppc_used):
                # the epilogue runs on the device behind the emit pass, while the host waits for
                # E; only for contiguous clouds (their average degree comes from row_ptr).  As
                # in the reference (spatial_graph.py:157-158), without a batch vector the whole
                # graph is one cloud for the degree, whatever chunks the radius search used.
                fused.clear()
                if ppc_used <= 0:
                    return False
                deg_ppc = ppc_used if batch is not None else N
                fbuf = torch.empty(cap * (4 + nsh) + N, dtype=torch.float32, device=dev)
                ibuf = torch.empty(2 * cap + 2 * N, dtype=torch.int32, device=dev)
                f = dict(direction=fbuf[:3 * cap].view(cap, 3), dist=fbuf[3 * cap:4 * cap],
                         Y=fbuf[4 * cap:(4 + nsh) * cap].view(cap, nsh),
                         avg=fbuf[(4 + nsh) * cap:], col_sorted=ibuf[:cap],
                         perm=ibuf[cap:2 * cap], node_start=ibuf[2 * cap:2 * cap + N],
                         node_end=ibuf[2 * cap + N:])
                with _nat.on_device(dev):
                    _nat.check(_nat.lib().geo_spatial_graph_epilogue_dev(
                        _nat.ptr(p32), N, _nat.ptr(row_s), _nat.ptr(col_s), _nat.ptr(row_ptr_d),
                        cap, int(max_l), int(deg_ppc), *[_nat.ptr(f[k]) for k in (
                            "direction", "dist", "Y", "col_sorted", "perm", "node_start",
                            "node_end", "avg")], _nat.stream_of(dev)),
                        "geo_spatial_graph_epilogue_dev")
                fused.update(f)
                return True   # the graph keeps views of bound-sized fields: row / col may be too

        row, col, row_ptr, B = radius_graph_csr_hip(
            pos, radius, max_num_neighbors=max_num_neighbors, batch=batch, mask=mask,
            num_batch_elements=num_batch_elements, after_emit=after_emit)
        E = row.shape[0]
        if E == 0:
            return SpatialGraph._empty(N, dev, max_l)
        if fused:
            # views of the first E rows of the bound-sized fields the device epilogue wrote
            graph = SpatialGraph(row=row, col=col, direction=fused["direction"][:E],
                                 dist=fused["dist"][:E], col_sorted=fused["col_sorted"][:E],
                                 perm=fused["perm"][:E], node_start=fused["node_start"],
                                 node_end=fused["node_end"], Y=fused["Y"][:E], N=N, E=E,
                                 avg_degree=fused["avg"])
            object.__setattr__(graph, "_perm_identity", True)
            return graph
        if batch is not None:
            # B comes from the radius graph (its batch.max() sync, or num_batch_elements)
            batch = batch.reshape(-1).to(device=dev, dtype=torch.int64)
            ppc = 0
        else:
            B, ppc = 1, N
        ibuf = torch.empty(2 * E + 2 * N, dtype=torch.int32, device=dev)
        col_sorted, perm = ibuf[:E], ibuf[E:2 * E]
        node_start, node_end = ibuf[2 * E:2 * E + N], ibuf[2 * E + N:]
        L = _nat.lib()
        if differentiable:
            # differentiable geometry (autograd function), CSR arrays and degrees separately
            with _nat.on_device(dev):
                _nat.check(L.geo_csr_from_row_ptr(
                    _nat.ptr(row_ptr), N, _nat.ptr(col), E, _nat.ptr(col_sorted), _nat.ptr(perm),
                    _nat.ptr(node_start), _nat.ptr(node_end), _nat.stream_of(dev)),
                    "geo_csr_from_row_ptr")
            direction, dist, Y = edge_geometry(pos, row, col, max_l, (perm, node_start, node_end))
            avg = graph_avg_degree_hip(row_ptr, N, batch, B)
        else:
            # one call for CSR arrays, geometry and degrees; one float allocation for the fields
            p32 = _positions("spatial_graph", pos)
            fbuf = torch.empty(E * (4 + nsh) + N, dtype=torch.float32, device=dev)
            direction = fbuf[:3 * E].view(E, 3)
            dist = fbuf[3 * E:4 * E]
            Y = fbuf[4 * E:(4 + nsh) * E].view(E, nsh)
            avg = fbuf[(4 + nsh) * E:]
            with _nat.on_device(dev):
                ws_bytes = L.geo_graph_avg_degree_workspace_bytes(B)
                ws = _nat.workspace(ws_bytes, dev)
                _nat.check(L.geo_spatial_graph_epilogue(
                    _nat.ptr(p32), N, _nat.ptr(row), _nat.ptr(col), _nat.ptr(row_ptr), E,
                    int(max_l), _nat.ptr(batch), B, ppc, _nat.ptr(direction), _nat.ptr(dist),
                    _nat.ptr(Y), _nat.ptr(col_sorted), _nat.ptr(perm), _nat.ptr(node_start),
                    _nat.ptr(node_end), _nat.ptr(avg), _nat.ptr(ws), ws_bytes, _nat.stream_of(dev)),
                    "geo_spatial_graph_epilogue")
        graph = SpatialGraph(row=row, col=col, direction=direction, dist=dist,
                             col_sorted=col_sorted, perm=perm, node_start=node_start,
                             node_end=node_end, Y=Y, N=N, E=E, avg_degree=avg)
        object.__setattr__(graph, "_perm_identity", True)  # kernels may skip the perm lookup
        return graph

    @staticmethod
    def _empty(N: int, device: torch.device, max_l: int = 2) -> "SpatialGraph":
        num_sh = (max_l + 1) ** 2
        return SpatialGraph(
            row=torch.empty(0, dtype=torch.long, device=device),
            col=torch.empty(0, dtype=torch.long, device=device),
            direction=torch.empty(0, 3, device=device),
            dist=torch.empty(0, device=device),
            col_sorted=torch.empty(0, dtype=torch.int32, device=device),
            perm=torch.empty(0, dtype=torch.int32, device=device),
            node_start=torch.zeros(N, dtype=torch.int32, device=device),
            node_end=torch.zeros(N, dtype=torch.int32, device=device),
            Y=torch.empty(0, num_sh, device=device),
            N=N, E=0,
            avg_degree=torch.ones(N, device=device),
        )

    @staticmethod
    def from_edge_index(
        row: Tensor,
        col: Tensor,
        pos: Tensor,
        N: int,
        max_l: int = 2,
        batch: Optional[Tensor] = None,
        num_batch_elements: Optional[int] = None,
    ) -> "SpatialGraph":
        """Graph from given edges in any order (spatial_graph.py:185-245): the CSR comes from the
        stable radix sort of ``col``."""
        dev = pos.device
        E = row.shape[0]
        if E == 0:
            return SpatialGraph._empty(N, dev, max_l)
        col_sorted, perm, node_start, node_end = sort_and_build_csr_cuda(col, N)
        direction, dist, Y = edge_geometry(pos, row, col, max_l, (perm, node_start, node_end))
        row_ptr = torch.zeros(N + 1, dtype=torch.int64, device=dev)
        row_ptr[1:] = node_end.to(torch.int64)
        row_ptr[:-1] = node_start.to(torch.int64)
        if batch is not None:
            B = int(num_batch_elements) if num_batch_elements is not None else int(batch.max().item()) + 1
        else:
            B = 1
        avg = graph_avg_degree_hip(row_ptr, N, batch, B)
        return SpatialGraph(row=row, col=col, direction=direction, dist=dist,
                            col_sorted=col_sorted, perm=perm, node_start=node_start,
                            node_end=node_end, Y=Y, N=N, E=E, avg_degree=avg)
