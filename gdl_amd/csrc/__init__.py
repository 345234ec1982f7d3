"""Backend dispatcher — gfx950 HIP kernels for radius graph, segment reduce, KNN and FPS.

Same public names as the reference dispatcher (geoembodied/csrc/__init__.py): the
``*_available`` probes, ``get_radius_graph_backend``, ``radius_graph_cuda``,
``sort_and_build_csr_cuda``, ``segment_reduce_sum_cuda``, ``knn_cuda``, ``knn_self_cuda`` and
``fps_cuda``.  On ROCm PyTorch the GPU device type is ``cuda``, so "cuda" names the HIP path.

Differences from the reference, by design:

* Kernels come from the prebuilt ``libgeoembodied_hip.so`` (no JIT compilation at first call).
* There is no CPU path.  CPU tensors raise ``RuntimeError``; the reference's CPU fallbacks
  ``_fps_iterative_fallback`` and ``_knn_bruteforce`` keep their names so that importing callers
  (nn/modules/equivariant_pool.py:261) still import, and raise when called.
* Each op performs at most one device-to-host synchronisation, to size its output
  (``fps_cuda``: sample count; radius graph: edge count; plus ``batch.max()`` when the caller
  does not give ``num_batch_elements``, as the reference does).
"""

from __future__ import annotations

import ctypes
import logging
from typing import Optional, Tuple

import numpy as np
import torch
from torch import Tensor
from torch.utils.weak import WeakIdKeyDictionary

from gdl_amd import _native as _nat

logger = logging.getLogger(__name__)

_NO_CPU = (
    "{name}: this MI355X build of geoembodied runs its geometry kernels on the GPU only; "
    "got a tensor on {device}. Move the inputs to a 'cuda' (HIP) device."
)


def _require_gpu(name: str, *tensors: Optional[Tensor]) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(_NO_CPU.format(name=name, device=t.device))


def _hip_ready() -> bool:
    return torch.cuda.is_available() and _nat.loaded()


def _i64(t: Tensor, device: torch.device) -> Tensor:
    return t.to(device=device, dtype=torch.int64).contiguous()


def _positions(name: str, x: Tensor) -> Tensor:
    if x.dim() != 2 or x.shape[1] != 3:
        raise ValueError(f"{name}: positions must have shape [N, 3], got {tuple(x.shape)}")
    return x.contiguous().float()


def fp32_radius_sq(r: float) -> float:
    """fl32(fl64(r) * fl64(r)): the threshold the reference's CPU path compares against."""
    return float(np.float32(float(r) * float(r)))


# ═══════════════════════════════════════════════════════════════════
# Radius graph
# ═══════════════════════════════════════════════════════════════════


def get_radius_graph_backend() -> str:
    """'cuda' when the HIP library is loaded and a GPU is visible, else 'unavailable'."""
    return "cuda" if _hip_ready() else "unavailable"


# Largest N * max_num_neighbors whose bound-sized emit scratch (16 bytes per entry) is allocated
# to overlap the edge-count sync with the emit pass (2^26 entries = 1 GiB); larger graphs wait.
_RADIUS_ASYNC_MAX_EDGES = 1 << 26
# Bound-sized scratch is returned as the outputs themselves (row / col are views of the first E
# entries of its two rows, sharing one storage) only when the graph fills at least half of it
# and it is at most this large; otherwise the edges are copied into exact-sized tensors (one
# kernel, ~4 us for C2's 657k edges) so a kept graph never holds more than twice its size.
_RADIUS_VIEW_MAX_BYTES = 256 << 20
# batch tensors (by identity, with their version counter) whose clouds proved not to be the
# contiguous equal-chunk layout: later calls with the same unchanged tensor skip that attempt
_BATCH_NOT_CHUNKED: "WeakIdKeyDictionary" = WeakIdKeyDictionary()
# radius-graph target tensors (by identity, with their version counter) -> the graph's row
# pointer.  The graph's edges are already grouped by target in CSR order, so the CSR build of
# those unchanged targets over the same node count is the row pointer itself: one pass, no sort.
_TARGETS_ROW_PTR: "WeakIdKeyDictionary" = WeakIdKeyDictionary()
# the same target tensors -> (version, int32 copy of the row pointer), made on first use by a
# consumer that needs only the CSR bounds (node_start / node_end are its two shifted views)
_TARGETS_BOUNDS32: "WeakIdKeyDictionary" = WeakIdKeyDictionary()


def target_bounds(col: Tensor, N: int) -> Optional[Tuple[Tensor, Tensor]]:
    """(node_start, node_end) int32 [N] of a radius graph's unchanged target tensor ``col`` over N
    nodes: its CSR permutation is the identity, so these and perm = None are the whole CSR.  None
    for any other index tensor (callers then build the CSR)."""
    known = _TARGETS_ROW_PTR.get(col)
    if known is None or known[0] != col._version or known[1].numel() != N + 1:
        return None
    b = _TARGETS_BOUNDS32.get(col)
    if b is None or b[0] != col._version or b[1].numel() != N + 1:
        b = (col._version, known[1].to(torch.int32))  # E < 2^31: the CSR arrays are int32
        _TARGETS_BOUNDS32[col] = b
    return b[1][:-1], b[1][1:]


def radius_graph_hip(
    x: Tensor,
    r,
    *,
    max_num_neighbors: int = 32,
    loop: bool = False,
    mask: Optional[Tensor] = None,
    batch: Optional[Tensor] = None,
    num_batch_elements: Optional[int] = None,
) -> Tuple[Tensor, Tensor]:
    row, col, row_ptr, _ = radius_graph_csr_hip(x, r, max_num_neighbors=max_num_neighbors,
                                                loop=loop, mask=mask, batch=batch,
                                                num_batch_elements=num_batch_elements)
    _TARGETS_ROW_PTR[col] = (col._version, row_ptr)
    return row, col


def radius_graph_csr_hip(
    x: Tensor,
    r,
    *,
    max_num_neighbors: int = 32,
    loop: bool = False,
    mask: Optional[Tensor] = None,
    batch: Optional[Tensor] = None,
    num_batch_elements: Optional[int] = None,
    after_emit=None,
) -> Tuple[Tensor, Tensor, Tensor, int]:
    """Radius graph on the GPU; returns (row=source, col=target) int64, sorted by target then
    source, the CSR row pointer (int64 [N+1]) and the number of clouds B.  Cloud membership comes
    from ``batch`` when given, otherwise from ``num_batch_elements`` contiguous equal chunks (one
    cloud when neither is given).  ``r`` is a Python number or a one-element device tensor (e.g.
    an adaptive radius computed on the GPU), which the kernels read directly: no host round trip
    for the radius.  ``after_emit(row_scratch, col_scratch, row_ptr, cap, ppc)``, if given, is
    called after each launch of the emit pass into bound-sized scratch (cap rows, the first E of
    them the graph), before the host waits for E, with the cloud size ppc that pass assumed (0
    for clouds given by a batch vector of any layout); it is not called when the graph is too
    large for bound-sized scratch.  When its last call returns True (the caller keeps views of
    bound-sized buffers of its own), row and col are views of the scratch whatever E is, instead
    of exact-sized copies of a sparse graph."""
    _require_gpu("radius_graph", x, mask, batch)
    x = _positions("radius_graph", x)
    dev = x.device
    N = x.shape[0]
    K = int(max_num_neighbors)
    if K < 0:
        raise ValueError(f"radius_graph: max_num_neighbors must be >= 0, got {K}")
    r_dev = None
    if isinstance(r, Tensor):
        if r.numel() != 1:
            raise ValueError(f"radius_graph: a tensor radius must have one element, got {r.numel()}")
        r_dev = r.reshape(()).to(device=dev, dtype=torch.float64).contiguous()
        r = 1.0
    r = float(r)
    empty = torch.empty(0, dtype=torch.int64, device=dev)
    if N == 0 or K == 0 or not (r > 0.0):
        B0 = int(num_batch_elements) if num_batch_elements is not None else 1
        return empty, empty.clone(), torch.zeros(N + 1, dtype=torch.int64, device=dev), B0
    r2 = fp32_radius_sq(r)
    ppc_try = 0
    batch_key = batch
    if batch is not None:
        if batch.numel() != N:
            raise ValueError(f"radius_graph: batch has {batch.numel()} entries for {N} points")
        batch = _i64(batch.reshape(-1), dev)
        B = int(num_batch_elements) if num_batch_elements is not None else int(batch.max().item()) + 1
        ppc = 0
        # sorted equal-size clouds (what the reference's GPU path assumes) take the per-cloud
        # front end; the device checks that layout and reports a mismatch with the edge count
        ppc_try = N // B if B >= 1 and N % B == 0 else 0
        if ppc_try and _BATCH_NOT_CHUNKED.get(batch_key) == batch_key._version:
            ppc_try = 0
    else:
        B = int(num_batch_elements) if num_batch_elements is not None else 1
        if B < 1:
            raise ValueError(f"radius_graph: num_batch_elements must be >= 1, got {B}")
        if N % B != 0:
            raise ValueError(f"radius_graph: {N} points do not split into {B} equal clouds")
        ppc = N // B
    if B < 1:
        return empty, empty.clone(), torch.zeros(N + 1, dtype=torch.int64, device=dev), B
    mask_u8 = None
    if mask is not None:
        if mask.numel() != N:
            raise ValueError(f"radius_graph: mask has {mask.numel()} entries for {N} points")
        mask_u8 = mask.to(device=dev, dtype=torch.bool).reshape(-1).contiguous().view(torch.uint8)
    L = _nat.lib()
    with _nat.on_device(dev):
        s = _nat.stream_of(dev)
        ws_bytes = L.geo_radius_workspace_bytes(N, B, K)
        ws = _nat.workspace(ws_bytes, dev)
        row_ptr = torch.empty(N + 1, dtype=torch.int64, device=dev)
        emit = L.geo_radius_emit if r_dev is None else L.geo_radius_emit_dev
        if N * K <= _RADIUS_ASYNC_MAX_EDGES:
            # emit into bound-sized scratch right behind the count; the host waits only for the
            # count (an event) to learn E, and the first E entries are the graph
            edges_h, counted = _nat.sync_slot(dev)
            caller_views = False
            for p_arg in ((ppc_try, 0) if ppc_try else (ppc,)):
                if r_dev is None:
                    args = (_nat.ptr(x), N, _nat.ptr(batch), B, p_arg, _nat.ptr(mask_u8), r2, r, K,
                            int(bool(loop)))
                else:
                    args = (_nat.ptr(x), N, _nat.ptr(batch), B, p_arg, _nat.ptr(mask_u8),
                            _nat.ptr(r_dev), K, int(bool(loop)))
                _nat.check(L.geo_radius_count_async(
                    _nat.ptr(x), N, _nat.ptr(batch), B, p_arg, _nat.ptr(mask_u8), r2, r,
                    _nat.ptr(r_dev), K, int(bool(loop)), _nat.ptr(row_ptr), edges_h.data_ptr(),
                    _nat.ptr(ws), ws_bytes, s), "geo_radius_count_async")
                counted.record(torch.cuda.current_stream(dev))
                scratch = torch.empty(2, N * K, dtype=torch.int64, device=dev)
                _nat.check(emit(*args, _nat.ptr(row_ptr), _nat.ptr(scratch[0]), _nat.ptr(scratch[1]),
                                _nat.ptr(ws), ws_bytes, s), "geo_radius_emit")
                if after_emit is not None:
                    caller_views = bool(after_emit(scratch[0], scratch[1], row_ptr, N * K, p_arg))
                counted.synchronize()
                E, bad = edges_h[:2].tolist()
                if bad == 0:
                    break   # else: batch is not the chunk layout; the general path follows
                _BATCH_NOT_CHUNKED[batch_key] = batch_key._version
            if 16 * N * K <= _RADIUS_VIEW_MAX_BYTES and (2 * E >= N * K or caller_views):
                row, col = scratch[0, :E], scratch[1, :E]
            else:
                row = torch.empty(E, dtype=torch.int64, device=dev)
                col = torch.empty(E, dtype=torch.int64, device=dev)
                _nat.check(L.geo_radius_copy_edges(_nat.ptr(scratch[0]), _nat.ptr(scratch[1]), E,
                                                   _nat.ptr(row), _nat.ptr(col), s),
                           "geo_radius_copy_edges")
        else:
            if r_dev is None:
                args = (_nat.ptr(x), N, _nat.ptr(batch), B, ppc, _nat.ptr(mask_u8), r2, r, K,
                        int(bool(loop)))
            else:
                args = (_nat.ptr(x), N, _nat.ptr(batch), B, ppc, _nat.ptr(mask_u8), _nat.ptr(r_dev),
                        K, int(bool(loop)))
            count = L.geo_radius_count if r_dev is None else L.geo_radius_count_dev
            _nat.check(count(*args, _nat.ptr(row_ptr), _nat.ptr(ws), ws_bytes, s), "geo_radius_count")
            E = int(row_ptr[N].item())
            row = torch.empty(E, dtype=torch.int64, device=dev)
            col = torch.empty(E, dtype=torch.int64, device=dev)
            if E > 0:
                _nat.check(emit(*args, _nat.ptr(row_ptr), _nat.ptr(row), _nat.ptr(col), _nat.ptr(ws),
                                ws_bytes, s), "geo_radius_emit")
    return row, col, row_ptr, B


def radius_graph_cuda(
    x: Tensor,
    r: float,
    *,
    max_num_neighbors: int = 32,
    loop: bool = False,
    mask: Optional[Tensor] = None,
    batch_size: Optional[int] = None,
    points_per_batch: Optional[int] = None,
) -> Tuple[Tensor, Tensor]:
    """Reference-compatible entry (geoembodied/csrc/__init__.py:130-186): one cloud, or
    ``batch_size`` contiguous clouds of ``points_per_batch`` points."""
    if batch_size is not None and batch_size > 1:
        if points_per_batch is None:
            raise ValueError("points_per_batch required when batch_size > 1")
        if int(batch_size) * int(points_per_batch) != x.shape[0]:
            raise ValueError("radius_graph_cuda: batch_size * points_per_batch != N")
        nb = int(batch_size)
    else:
        nb = None
    return radius_graph_hip(x, r, max_num_neighbors=max_num_neighbors, loop=loop, mask=mask,
                            num_batch_elements=nb)


# ═══════════════════════════════════════════════════════════════════
# Segment reduce + CSR build
# ═══════════════════════════════════════════════════════════════════


def segment_reduce_available() -> bool:
    return _hip_ready()


def sort_and_build_csr_cuda(col: Tensor, N: int) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """Stable sort of targets + CSR offsets: (col_sorted, perm, node_start, node_end), int32."""
    _require_gpu("sort_and_build_csr", col)
    if col.dim() != 1:
        raise ValueError(f"sort_and_build_csr: col must be 1-D, got {tuple(col.shape)}")
    N = int(N)
    if N < 0:
        raise ValueError(f"sort_and_build_csr: N must be >= 0, got {N}")
    dev = col.device
    known = _TARGETS_ROW_PTR.get(col)
    col = _i64(col, dev)
    E = col.shape[0]
    i32 = dict(dtype=torch.int32, device=dev)
    col_sorted = torch.empty(E, **i32)
    perm = torch.empty(E, **i32)
    node_start = torch.empty(N, **i32)
    node_end = torch.empty(N, **i32)
    L = _nat.lib()
    if known is not None and known[0] == col._version and known[1].numel() == N + 1:
        with _nat.on_device(dev):  # a radius graph's unchanged targets: its row pointer
            _nat.check(L.geo_csr_from_row_ptr(_nat.ptr(known[1]), N, _nat.ptr(col), E,
                                              _nat.ptr(col_sorted), _nat.ptr(perm),
                                              _nat.ptr(node_start), _nat.ptr(node_end),
                                              _nat.stream_of(dev)), "geo_csr_from_row_ptr")
        return col_sorted, perm, node_start, node_end
    with _nat.on_device(dev):
        ws_bytes = L.geo_csr_workspace_bytes(E, N)
        ws = _nat.workspace(ws_bytes, dev)
        _nat.check(L.geo_csr_build(_nat.ptr(col), E, N, _nat.ptr(col_sorted), _nat.ptr(perm),
                                   _nat.ptr(node_start), _nat.ptr(node_end), _nat.ptr(ws),
                                   ws_bytes, _nat.stream_of(dev)), "geo_csr_build")
    return col_sorted, perm, node_start, node_end


_SOURCE_CSR = WeakIdKeyDictionary()


def source_csr(row: Tensor, N: int) -> Tuple[Tensor, Tensor, Tensor]:
    """(perm, node_start, node_end) of the edges grouped by source: the stable CSR of ``row``
    (the backward passes of message passing and edge geometry scatter onto the sources with it).
    Built once per ``row`` tensor and kept while that tensor lives, so the layers of a network
    sharing one graph sort its sources once; an in-place change of ``row`` (its version counter)
    or another N rebuilds it."""
    key = (row._version, int(N), row.numel())
    hit = _SOURCE_CSR.get(row)
    if hit is not None and hit[0] == key:
        return hit[1]
    _, perm_r, ns_r, ne_r = sort_and_build_csr_cuda(row, N)
    _SOURCE_CSR[row] = (key, (perm_r, ns_r, ne_r))
    return perm_r, ns_r, ne_r


def _dtype_code(name: str, t: Tensor) -> int:
    code = _nat.DTYPE_CODES.get(t.dtype)
    if code is None:
        raise TypeError(f"{name}: unsupported dtype {t.dtype} (float32, bfloat16, float64)")
    return code


def _i32(t: Optional[Tensor], device: torch.device) -> Optional[Tensor]:
    if t is None:
        return None
    if t.dtype == torch.int32 and t.device == device and t.is_contiguous():
        return t
    return t.to(device=device, dtype=torch.int32).contiguous()


def segment_reduce_forward_hip(
    msg: Tensor,
    perm: Optional[Tensor],
    node_start: Tensor,
    node_end: Tensor,
    N: int,
    reduce: str = "sum",
    tie_mode: int = 0,
) -> Tuple[Tensor, Optional[Tensor]]:
    """out[N, C] (and the int32 argmax record for 'max')."""
    _require_gpu("segment_reduce", msg, perm, node_start, node_end)
    if reduce not in _nat.REDUCE_CODES:
        raise ValueError(f"segment_reduce: reduce must be sum, mean or max, got {reduce!r}")
    if msg.dim() != 2:
        raise ValueError(f"segment_reduce: msg must be [E, C], got {tuple(msg.shape)}")
    N = int(N)
    if node_start.numel() < N or node_end.numel() < N:
        raise ValueError("segment_reduce: node_start/node_end shorter than N")
    code = _dtype_code("segment_reduce", msg)
    dev = msg.device
    msg = msg.contiguous()
    E, C = msg.shape
    perm = _i32(perm, dev)
    if perm is not None and perm.numel() != E:
        raise ValueError(f"segment_reduce: perm has {perm.numel()} entries for E={E}")
    ns, ne = _i32(node_start, dev), _i32(node_end, dev)
    out = torch.empty(N, C, dtype=msg.dtype, device=dev)
    arg = torch.empty(N, C, dtype=torch.int32, device=dev) if reduce == "max" else None
    with _nat.on_device(dev):
        _nat.check(_nat.lib().geo_segment_reduce_fwd(
            _nat.REDUCE_CODES[reduce], code, _nat.ptr(msg), _nat.ptr(perm), _nat.ptr(ns),
            _nat.ptr(ne), E, N, C, _nat.ptr(out), _nat.ptr(arg), int(tie_mode),
            _nat.stream_of(dev)), "geo_segment_reduce_fwd")
    return out, arg


def segment_reduce_backward_hip(
    grad_out: Tensor,
    col_sorted: Tensor,
    perm: Optional[Tensor],
    node_start: Optional[Tensor],
    node_end: Optional[Tensor],
    E: int,
    reduce: str = "sum",
    msg: Optional[Tensor] = None,
    out: Optional[Tensor] = None,
    arg: Optional[Tensor] = None,
) -> Tensor:
    """grad_msg[E, C] for the given reduction."""
    _require_gpu("segment_reduce backward", grad_out, col_sorted, perm, msg, out, arg)
    code = _dtype_code("segment_reduce backward", grad_out)
    dev = grad_out.device
    grad_out = grad_out.contiguous()
    S, C = grad_out.shape
    grad_msg = torch.empty(int(E), C, dtype=grad_out.dtype, device=dev)
    cs = _i32(col_sorted, dev)
    pm = _i32(perm, dev)
    ns, ne = _i32(node_start, dev), _i32(node_end, dev)
    if msg is not None:
        msg = msg.to(grad_out.dtype).contiguous()
    if out is not None:
        out = out.to(grad_out.dtype).contiguous()
    if arg is not None:
        arg = arg.contiguous()
    with _nat.on_device(dev):
        _nat.check(_nat.lib().geo_segment_reduce_bwd(
            _nat.REDUCE_CODES[reduce], code, _nat.ptr(grad_out), _nat.ptr(msg), _nat.ptr(out),
            _nat.ptr(arg), _nat.ptr(cs), _nat.ptr(pm), _nat.ptr(ns), _nat.ptr(ne), int(E), S, C,
            _nat.ptr(grad_msg), _nat.stream_of(dev)), "geo_segment_reduce_bwd")
    return grad_msg


def segment_reduce_sum_cuda(
    msg: Tensor,
    perm: Tensor,
    node_start: Tensor,
    node_end: Tensor,
    N: int,
) -> Tensor:
    """Deterministic segment sum (reference name; geoembodied/csrc/__init__.py:280-302)."""
    return segment_reduce_forward_hip(msg, perm, node_start, node_end, N, "sum")[0]


def segment_softmax_forward_hip(
    scores: Tensor,
    perm: Optional[Tensor],
    node_start: Tensor,
    node_end: Tensor,
    N: int,
    contiguous_csr: bool = False,
) -> Tensor:
    """Softmax of scores[E, H] over each target segment of the CSR (rows in no segment -> 0).

    ``contiguous_csr`` states that the node ranges are ascending and contiguous from 0 (the CSR
    of ``sort_and_build_csr`` or of a radius graph): the kernel then also writes the zeros of
    the rows after the last segment and the output needs no separate fill."""
    _require_gpu("segment_softmax", scores, perm, node_start, node_end)
    if scores.dim() != 2:
        raise ValueError(f"segment_softmax: scores must be [E, H], got {tuple(scores.shape)}")
    if scores.dtype not in (torch.float32, torch.float64):
        raise TypeError(f"segment_softmax: scores must be float32 or float64, got {scores.dtype}")
    N = int(N)
    if node_start.numel() < N or node_end.numel() < N:
        raise ValueError("segment_softmax: node_start/node_end shorter than N")
    dev = scores.device
    scores = scores.contiguous()
    E, H = scores.shape
    pm = _i32(perm, dev)
    if pm is not None and pm.numel() != E:
        raise ValueError(f"segment_softmax: perm has {pm.numel()} entries for E={E}")
    ns, ne = _i32(node_start, dev), _i32(node_end, dev)
    out = torch.empty_like(scores) if contiguous_csr else torch.zeros_like(scores)
    with _nat.on_device(dev):
        _nat.check(_nat.lib().geo_segment_softmax_fwd(
            _nat.DTYPE_CODES[scores.dtype], _nat.ptr(scores), _nat.ptr(pm), _nat.ptr(ns),
            _nat.ptr(ne), E, N, H, int(bool(contiguous_csr)), _nat.ptr(out), _nat.stream_of(dev)),
            "geo_segment_softmax_fwd")
    return out


def segment_softmax_backward_hip(
    grad_out: Tensor,
    out: Tensor,
    perm: Optional[Tensor],
    node_start: Tensor,
    node_end: Tensor,
    N: int,
    contiguous_csr: bool = False,
) -> Tensor:
    """grad_scores = out * (grad_out - segment sum of grad_out * out) (rows in no segment -> 0;
    ``contiguous_csr`` as in the forward)."""
    _require_gpu("segment_softmax backward", grad_out, out, perm, node_start, node_end)
    dev = out.device
    grad_out = grad_out.to(out.dtype).contiguous()
    out = out.contiguous()
    E, H = out.shape
    pm = _i32(perm, dev)
    ns, ne = _i32(node_start, dev), _i32(node_end, dev)
    grad = torch.empty_like(out) if contiguous_csr else torch.zeros_like(out)
    with _nat.on_device(dev):
        _nat.check(_nat.lib().geo_segment_softmax_bwd(
            _nat.DTYPE_CODES[out.dtype], _nat.ptr(grad_out), _nat.ptr(out), _nat.ptr(pm),
            _nat.ptr(ns), _nat.ptr(ne), E, int(N), H, int(bool(contiguous_csr)), _nat.ptr(grad),
            _nat.stream_of(dev)), "geo_segment_softmax_bwd")
    return grad


def gather_weighted_sum_forward_hip(feat: Tensor, idx: Tensor, w: Tensor) -> Tensor:
    """out[n] = sum_k w[n, k] * feat[idx[n, k]] (idx < 0 or >= N_src contributes nothing)."""
    _require_gpu("gather_weighted_sum", feat, idx, w)
    if feat.dim() != 2 or idx.dim() != 2 or w.shape != idx.shape:
        raise ValueError(f"gather_weighted_sum: feat [N_src, C], idx and w [N_out, K]; got "
                         f"{tuple(feat.shape)}, {tuple(idx.shape)}, {tuple(w.shape)}")
    code = _dtype_code("gather_weighted_sum", feat)
    dev = feat.device
    feat = feat.contiguous()
    idx = idx.to(device=dev, dtype=torch.int64).contiguous()
    w = w.to(device=dev, dtype=feat.dtype).contiguous()
    (N_src, C), (N_out, K) = feat.shape, idx.shape
    out = torch.empty(N_out, C, dtype=feat.dtype, device=dev)
    with _nat.on_device(dev):
        _nat.check(_nat.lib().geo_gather_weighted_sum(
            code, _nat.ptr(feat), N_src, C, _nat.ptr(idx), _nat.ptr(w), N_out, K, _nat.ptr(out),
            _nat.stream_of(dev)), "geo_gather_weighted_sum")
    return out


def gather_weighted_sum_backward_hip(
    grad_out: Tensor,
    feat: Tensor,
    idx: Tensor,
    w: Tensor,
    need_feat: bool = True,
    need_w: bool = True,
    csr: Optional[Tuple[Tensor, Tensor, Tensor, Tensor]] = None,
) -> Tuple[Optional[Tensor], Optional[Tensor]]:
    """(grad_feat [N_src, C], grad_w [N_out, K]) of gather_weighted_sum; ``csr`` is the CSR of
    the flattened idx over the sources (built here when not given)."""
    _require_gpu("gather_weighted_sum backward", grad_out, feat, idx, w)
    code = _dtype_code("gather_weighted_sum backward", feat)
    dev = feat.device
    grad_out = grad_out.to(feat.dtype).contiguous()
    feat = feat.contiguous()
    idx = idx.to(device=dev, dtype=torch.int64).contiguous()
    w = w.to(device=dev, dtype=feat.dtype).contiguous()
    (N_src, C), (N_out, K) = feat.shape, idx.shape
    grad_feat = torch.empty(N_src, C, dtype=feat.dtype, device=dev) if need_feat else None
    grad_w = torch.empty(N_out, K, dtype=feat.dtype, device=dev) if need_w else None
    pm = ns = ne = None
    if need_feat:
        if csr is None:
            csr = sort_and_build_csr_cuda(idx.reshape(-1), N_src)
        _, pm, ns, ne = csr
    with _nat.on_device(dev):
        _nat.check(_nat.lib().geo_gather_weighted_sum_bwd(
            code, _nat.ptr(grad_out), _nat.ptr(feat), _nat.ptr(w), _nat.ptr(idx), N_src, C,
            N_out, K, _nat.ptr(pm), _nat.ptr(ns), _nat.ptr(ne), _nat.ptr(grad_feat),
            _nat.ptr(grad_w), _nat.stream_of(dev)), "geo_gather_weighted_sum_bwd")
    return grad_feat, grad_w


def idw_weights_hip(idx: Tensor, dist: Tensor) -> Tensor:
    """Inverse-distance weights of the interpolation layer (equivariant_interp.py:95-99)."""
    _require_gpu("idw_weights", idx, dist)
    dev = dist.device
    idx = idx.to(device=dev, dtype=torch.int64).contiguous()
    dist = dist.to(torch.float32).contiguous()
    if idx.shape != dist.shape or idx.dim() != 2:
        raise ValueError("idw_weights: idx and dist must both be [N_out, K]")
    N_out, K = idx.shape
    w = torch.empty(N_out, K, dtype=torch.float32, device=dev)
    with _nat.on_device(dev):
        _nat.check(_nat.lib().geo_idw_weights(_nat.ptr(idx), _nat.ptr(dist), N_out, K, _nat.ptr(w),
                                              _nat.stream_of(dev)), "geo_idw_weights")
    return w


def idw_interpolate_forward_hip(feat: Tensor, idx: Tensor, dist: Tensor) -> Tuple[Tensor, Tensor]:
    """(out, w): the IDW weights of ``idw_weights_hip`` (float32) and the gather-sum of ``feat``
    with them (rounded to feat's dtype), in one kernel; bitwise equal to the two calls."""
    _require_gpu("idw_interpolate", feat, idx, dist)
    if feat.dim() != 2 or idx.dim() != 2 or dist.shape != idx.shape:
        raise ValueError(f"idw_interpolate: feat [N_src, C], idx and dist [N_out, K]; got "
                         f"{tuple(feat.shape)}, {tuple(idx.shape)}, {tuple(dist.shape)}")
    code = _dtype_code("idw_interpolate", feat)
    dev = feat.device
    feat = feat.contiguous()
    idx = idx.to(device=dev, dtype=torch.int64).contiguous()
    dist = dist.to(device=dev, dtype=torch.float32).contiguous()
    (N_src, C), (N_out, K) = feat.shape, idx.shape
    out = torch.empty(N_out, C, dtype=feat.dtype, device=dev)
    w = torch.empty(N_out, K, dtype=torch.float32, device=dev)
    with _nat.on_device(dev):
        _nat.check(_nat.lib().geo_idw_interpolate(
            code, _nat.ptr(feat), N_src, C, _nat.ptr(idx), _nat.ptr(dist), N_out, K, _nat.ptr(out),
            _nat.ptr(w), _nat.stream_of(dev)), "geo_idw_interpolate")
    return out, w


def knn_radius_stat_hip(dist: Tensor, col: int, mode: str, multiplier: float) -> Tensor:
    """multiplier * (mean of sqrt(clamp(d, 1e-8, 1e20)) | lower median of sqrt(max(d, 1e-12)))
    over column ``col`` of a KNN distance matrix, as a float64 device scalar (no host sync)."""
    _require_gpu("knn_radius_stat", dist)
    if dist.dim() != 2 or dist.shape[0] == 0:
        raise ValueError(f"knn_radius_stat: dist must be a non-empty [N, k], got {tuple(dist.shape)}")
    codes = {"mean": 0, "median": 1}
    if mode not in codes:
        raise ValueError(f"knn_radius_stat: mode must be 'mean' or 'median', got {mode!r}")
    dev = dist.device
    d = dist.to(torch.float32).contiguous()
    N, k = d.shape
    out = torch.empty((), dtype=torch.float64, device=dev)
    L = _nat.lib()
    with _nat.on_device(dev):
        ws_bytes = L.geo_knn_radius_stat_workspace_bytes(N)
        ws = _nat.workspace(ws_bytes, dev)
        _nat.check(L.geo_knn_radius_stat(_nat.ptr(d), N, k, int(col) % k, codes[mode],
                                         float(multiplier), _nat.ptr(out), _nat.ptr(ws), ws_bytes,
                                         _nat.stream_of(dev)), "geo_knn_radius_stat")
    return out


def edge_geometry_hip(pos: Tensor, row: Tensor, col: Tensor, max_l: int = 2,
                      with_sh: bool = True) -> Tuple[Tensor, Tensor, Optional[Tensor]]:
    """(direction [E, 3], dist [E], Y [E, (max_l+1)^2] or None) of the edges row -> col."""
    _require_gpu("edge_geometry", pos, row, col)
    pos = _positions("edge_geometry", pos)
    dev = pos.device
    row, col = _i64(row.reshape(-1), dev), _i64(col.reshape(-1), dev)
    E = row.numel()
    direction = torch.empty(E, 3, dtype=torch.float32, device=dev)
    dist = torch.empty(E, dtype=torch.float32, device=dev)
    Y = torch.empty(E, (max_l + 1) ** 2, dtype=torch.float32, device=dev) if with_sh else None
    with _nat.on_device(dev):
        _nat.check(_nat.lib().geo_edge_geometry(
            _nat.ptr(pos), pos.shape[0], _nat.ptr(row), _nat.ptr(col), E, int(max_l),
            _nat.ptr(direction), _nat.ptr(dist), _nat.ptr(Y), _nat.stream_of(dev)), "geo_edge_geometry")
    return direction, dist, Y


def edge_geometry_backward_hip(direction: Tensor, dist: Tensor, grad_direction: Optional[Tensor],
                               grad_dist: Optional[Tensor], grad_Y: Optional[Tensor],
                               max_l: int = 2) -> Tensor:
    """d loss / d diff [E, 3] from the gradients of direction, dist and Y."""
    dev = direction.device
    E = direction.shape[0]
    out = torch.empty(E, 3, dtype=torch.float32, device=dev)

    def f32(t):
        return None if t is None else t.to(torch.float32).contiguous()

    gd, gl, gy = f32(grad_direction), f32(grad_dist), f32(grad_Y)
    with _nat.on_device(dev):
        _nat.check(_nat.lib().geo_edge_geometry_bwd(
            _nat.ptr(direction), _nat.ptr(dist), _nat.ptr(gd), _nat.ptr(gl), _nat.ptr(gy), E,
            int(max_l), _nat.ptr(out), _nat.stream_of(dev)), "geo_edge_geometry_bwd")
    return out


def spherical_harmonics_hip(xyz: Tensor, max_l: int, normalize: bool):
    """(Y [N, (max_l+1)^2], unit [N, 3] or None, norm [N] or None) of xyz [N, 3] (fp32)."""
    _require_gpu("spherical_harmonics", xyz)
    dev = xyz.device
    xyz = xyz.to(torch.float32).contiguous()
    N = xyz.shape[0]
    Y = torch.empty(N, (max_l + 1) ** 2, dtype=torch.float32, device=dev)
    unit = torch.empty(N, 3, dtype=torch.float32, device=dev) if normalize else None
    norm = torch.empty(N, dtype=torch.float32, device=dev) if normalize else None
    with _nat.on_device(dev):
        _nat.check(_nat.lib().geo_spherical_harmonics(
            _nat.ptr(xyz), N, int(max_l), int(bool(normalize)), _nat.ptr(Y), _nat.ptr(unit),
            _nat.ptr(norm), _nat.stream_of(dev)), "geo_spherical_harmonics")
    return Y, unit, norm


def spherical_harmonics_backward_hip(xyz: Tensor, grad_Y: Tensor, max_l: int) -> Tensor:
    dev = xyz.device
    N = xyz.shape[0]
    out = torch.empty(N, 3, dtype=torch.float32, device=dev)
    gY = grad_Y.to(torch.float32).contiguous()
    with _nat.on_device(dev):
        _nat.check(_nat.lib().geo_spherical_harmonics_bwd(
            _nat.ptr(xyz), _nat.ptr(gY), N, int(max_l), _nat.ptr(out), _nat.stream_of(dev)),
            "geo_spherical_harmonics_bwd")
    return out


def graph_avg_degree_hip(row_ptr: Tensor, N: int, batch: Optional[Tensor], B: int) -> Tensor:
    """Per-node average degree of its cloud from the CSR row pointer, clamped below at 1."""
    dev = row_ptr.device
    out = torch.empty(N, dtype=torch.float32, device=dev)
    if N == 0:
        return out
    ppc = 0 if batch is not None else N // max(B, 1)
    b = None if batch is None else _i64(batch.reshape(-1), dev)
    L = _nat.lib()
    with _nat.on_device(dev):
        ws_bytes = L.geo_graph_avg_degree_workspace_bytes(B)
        ws = _nat.workspace(ws_bytes, dev)
        _nat.check(L.geo_graph_avg_degree(_nat.ptr(row_ptr.contiguous()), N, _nat.ptr(b), B, ppc,
                                          _nat.ptr(out), _nat.ptr(ws), ws_bytes, _nat.stream_of(dev)),
                   "geo_graph_avg_degree")
    return out


# ═══════════════════════════════════════════════════════════════════
# KNN
# ═══════════════════════════════════════════════════════════════════


def knn_available() -> bool:
    return _hip_ready()


def knn_cuda(
    query: Tensor,
    source: Tensor,
    ptr_q: Tensor,
    ptr_s: Tensor,
    k: int,
) -> Tuple[Tensor, Tensor]:
    """k nearest sources of each query within its cloud: (indices int64 [N_q, k] global source
    indices or -1, squared distances float32 [N_q, k] or 1e30), ascending by (distance, index)."""
    _require_gpu("knn", query, source)
    q = _positions("knn", query)
    s = _positions("knn", source)
    dev = q.device
    if ptr_q.numel() != ptr_s.numel():
        raise ValueError("ptr_q and ptr_s must have same length (B+1)")
    k = int(k)
    if k < 0:
        raise ValueError(f"knn: k must be >= 0, got {k}")
    pq, ps = _i64(ptr_q, dev), _i64(ptr_s, dev)
    B = pq.numel() - 1
    Nq, Ns = q.shape[0], s.shape[0]
    out_idx = torch.empty(Nq, k, dtype=torch.int64, device=dev)
    out_d = torch.empty(Nq, k, dtype=torch.float32, device=dev)
    if Nq == 0 or k == 0:
        return out_idx, out_d
    L = _nat.lib()
    with _nat.on_device(dev):
        ws_bytes = L.geo_knn_workspace_bytes(Nq, Ns, max(B, 0), k)
        ws = _nat.workspace(ws_bytes, dev)
        _nat.check(L.geo_knn(_nat.ptr(q), Nq, _nat.ptr(s), Ns, _nat.ptr(pq), _nat.ptr(ps),
                             max(B, 0), k, _nat.ptr(out_idx), _nat.ptr(out_d), _nat.ptr(ws),
                             ws_bytes, _nat.stream_of(dev)), "geo_knn")
    return out_idx, out_d


def knn_self_cuda(points: Tensor, ptr: Tensor, k: int) -> Tuple[Tensor, Tensor]:
    """Self-KNN within each cloud; self (distance 0) is included."""
    return knn_cuda(points, points, ptr, ptr, k)


def _knn_bruteforce(query, source, ptr_q, ptr_s, k):
    """Name kept from the reference CPU fallback; this build has no CPU path."""
    raise RuntimeError(_NO_CPU.format(name="_knn_bruteforce", device=query.device))


# ═══════════════════════════════════════════════════════════════════
# FPS
# ═══════════════════════════════════════════════════════════════════


def fps_available() -> bool:
    return _hip_ready()


def fps_cuda(pos: Tensor, ptr: Tensor, k_per_batch: Tensor) -> Tensor:
    """Farthest point sampling per cloud; int64 global indices concatenated by cloud.

    k is clamped to [0, cloud size]; a cloud sampled completely returns its indices in order.
    One host sync (the output size)."""
    _require_gpu("fps", pos)
    pos = _positions("fps", pos)
    dev = pos.device
    p = _i64(ptr, dev)
    kk = _i64(k_per_batch, dev)
    B = p.numel() - 1
    if B < 0:
        raise ValueError("fps: ptr must have at least one entry")
    if kk.numel() != B:
        raise ValueError(f"fps: k_per_batch has {kk.numel()} entries for {B} clouds")
    return _fps_run(pos, p, B, lambda L, out_ptr, info, s: L.geo_fps_prepare(
        _nat.ptr(p), _nat.ptr(kk), B, pos.shape[0], _nat.ptr(out_ptr), _nat.ptr(info), s))


def fps_uniform_hip(pos: Tensor, ptr: Tensor, num_samples: int) -> Tensor:
    """``fps_cuda(pos, ptr, (ptr[1:] - ptr[:-1]).clamp(max=num_samples))``, the ptr path of
    ``farthest_point_sampling``, with the host sync taken off the GPU's critical path.

    The prepare kernel forms the per-cloud k and writes its summary (total, largest cloud,
    validity) to device memory and to a pinned host buffer.  The sampling kernel for clouds of
    the average size is launched right behind it, before the host has read anything; it reads
    the device summary itself and does nothing if ptr is invalid or a cloud is larger than it
    holds.  The host waits only for the prepare kernel (an event), and launches the right kernel
    itself in that case.  The output is allocated at its bound min(N, B * num_samples) and
    returned as the prefix of length total."""
    _require_gpu("fps", pos)
    pos = _positions("fps", pos)
    dev = pos.device
    p = _i64(ptr, dev)
    B = p.numel() - 1
    if B < 0:
        raise ValueError("fps: ptr must have at least one entry")
    N = pos.shape[0]
    k = max(int(num_samples), 0)
    L = _nat.lib()
    with _nat.on_device(dev):
        s = _nat.stream_of(dev)
        out_ptr = torch.empty(B + 1, dtype=torch.int64, device=dev)
        info = torch.empty(3, dtype=torch.int64, device=dev)
        info_h, prepared = _nat.sync_slot(dev)
        out = torch.empty(min(N, B * k), dtype=torch.int64, device=dev)
        _nat.check(L.geo_fps_prepare_uniform(_nat.ptr(p), k, B, N, _nat.ptr(out_ptr),
                                             _nat.ptr(info), info_h.data_ptr(), s),
                   "geo_fps_prepare_uniform")
        prepared.record(torch.cuda.current_stream(dev))
        cap = ctypes.c_int64(0)
        guess = -(-N // B) if B > 0 and out.numel() > 0 else 0
        _nat.check(L.geo_fps_guarded(_nat.ptr(pos), N, _nat.ptr(p), _nat.ptr(out_ptr), B, guess,
                                     _nat.ptr(out), _nat.ptr(info), ctypes.byref(cap), s),
                   "geo_fps_guarded")
        prepared.synchronize()
        total, max_n, bad = info_h[:3].tolist()
        if bad:
            raise ValueError(f"fps: ptr is not a non-decreasing offset array within [0, {N}] "
                             f"(first bad entry: ptr[{bad - 1}])")
        if total < out.numel():
            out = out[:total]
        if total == 0 or 0 < max_n <= cap.value:
            return out
        ws_bytes = L.geo_fps_workspace_bytes(B, N, max_n)
        ws = _nat.workspace(ws_bytes, dev)
        _nat.check(L.geo_fps(_nat.ptr(pos), N, _nat.ptr(p), _nat.ptr(out_ptr), B, max_n,
                             _nat.ptr(out), _nat.ptr(ws), ws_bytes, s), "geo_fps")
    return out


def _fps_run(pos: Tensor, p: Tensor, B: int, prepare) -> Tensor:
    """prepare (offsets, total, largest cloud, validity) -> one host sync -> geo_fps."""
    dev = pos.device
    N = pos.shape[0]
    L = _nat.lib()
    with _nat.on_device(dev):
        s = _nat.stream_of(dev)
        out_ptr = torch.empty(B + 1, dtype=torch.int64, device=dev)
        info = torch.empty(3, dtype=torch.int64, device=dev)
        _nat.check(prepare(L, out_ptr, info, s), "geo_fps_prepare")
        total, max_n, bad = info.tolist()
        if bad:
            raise ValueError(f"fps: ptr is not a non-decreasing offset array within [0, {N}] "
                             f"(first bad entry: ptr[{bad - 1}])")
        out = torch.empty(total, dtype=torch.int64, device=dev)
        if total == 0:
            return out
        ws_bytes = L.geo_fps_workspace_bytes(B, N, max_n)
        ws = _nat.workspace(ws_bytes, dev)
        _nat.check(L.geo_fps(_nat.ptr(pos), N, _nat.ptr(p), _nat.ptr(out_ptr), B, max_n,
                             _nat.ptr(out), _nat.ptr(ws), ws_bytes, s), "geo_fps")
    return out


def _fps_iterative_fallback(pos, ptr, k_per_batch):
    """Name kept from the reference CPU fallback; this build has no CPU path."""
    raise RuntimeError(_NO_CPU.format(name="_fps_iterative_fallback", device=pos.device))


__all__ = [
    "get_radius_graph_backend", "radius_graph_cuda", "radius_graph_hip", "fp32_radius_sq",
    "segment_reduce_available", "sort_and_build_csr_cuda", "source_csr", "segment_reduce_sum_cuda",
    "segment_softmax_forward_hip", "segment_softmax_backward_hip",
    "gather_weighted_sum_forward_hip", "gather_weighted_sum_backward_hip", "idw_weights_hip",
    "idw_interpolate_forward_hip",
    "knn_radius_stat_hip", "radius_graph_csr_hip", "edge_geometry_hip",
    "edge_geometry_backward_hip", "spherical_harmonics_hip", "spherical_harmonics_backward_hip",
    "graph_avg_degree_hip",
    "segment_reduce_forward_hip", "segment_reduce_backward_hip",
    "knn_available", "knn_cuda", "knn_self_cuda",
    "fps_available", "fps_cuda", "fps_uniform_hip",
]
