"""CPU oracle for the geometry kernels — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker (or the timed CPU baseline), never as the thing measured
or shipped.  The product (``gdl_amd`` / ``geoembodied``) never imports it.

Contents:

* FPS, KNN, radius graph and the CSR build: ``geo_oracle.c`` (exact fp32 arithmetic in the
  reference's operation order) through ctypes.  Reference files followed are cited per function.
* Segment sum / mean / max, forward and backward: numpy below.  Sum and mean are accumulated in
  float64 and returned with the per-element scale ``sum |msg|`` that the tolerance of the
  comparison multiplies; max, argmax and every backward value are exact.
* Segment softmax (``sparse_softmax``) and its backward: numpy float64 below.
* Neighbourhood gather-sum (``gather_weighted_sum``, ``idw_weights``) and its backward: numpy
  float64 below.

Pinning (what checks each function independently of this restatement) is listed in
``tests/test_oracle.py``: reference KATs, closed forms on integer lattices where fp32 arithmetic
is exact, scipy / numpy library routines and brute force on tiny inputs.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
# GEO_ORACLE_LIB selects another build of geo_oracle.c (e.g. the sanitizer build of
# oracle/build.py, which the sanitizer tests load)
_LIB_PATH = Path(os.environ.get("GEO_ORACLE_LIB", str(_HERE / "lib" / "libgeo_oracle.so")))
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int64


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            from oracle.build import build
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        lib.oracle_fps.argtypes = [_P, _P, _P, _I, _P, _P]
        lib.oracle_knn.argtypes = [_P, _P, _P, _P, _I, _I, _I, _P, _P]
        lib.oracle_radius.argtypes = [_P, _I, _P, ctypes.c_float, _I, ctypes.c_int, _P, _P, _P, _P]
        lib.oracle_csr.argtypes = [_P, _I, _I, _P, _P, _P, _P]
        for f in (lib.oracle_fps, lib.oracle_knn, lib.oracle_radius, lib.oracle_csr):
            f.restype = None
        _lib = lib
    return _lib


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def fp32_radius_sq(r: float) -> float:
    """fl32(fl64(r) * fl64(r)) — geoembodied/functional/radius_graph.py:232 computes r*r in
    Python floats and the fp32 tensor comparison at :248 rounds it to fp32."""
    return float(np.float32(float(r) * float(r)))


# ---------------------------------------------------------------------------------- FPS ---

def fps(pos, ptr, k_per_batch) -> np.ndarray:
    """Farthest point sampling; geoembodied/csrc/__init__.py:600-654 (see geo_oracle.c)."""
    pos = _c(pos, np.float32).reshape(-1, 3)
    ptr = _c(ptr, np.int64)
    B = ptr.shape[0] - 1
    kk = _c(k_per_batch, np.int64)
    n = ptr[1:] - ptr[:-1]
    kc = np.clip(kk, 0, n)
    out_ptr = np.zeros(B + 1, dtype=np.int64)
    out_ptr[1:] = np.cumsum(kc)
    out = np.empty(int(out_ptr[-1]), dtype=np.int64)
    _load().oracle_fps(_p(pos), _p(ptr), _p(kc), B, _p(out_ptr), _p(out))
    return out


# ---------------------------------------------------------------------------------- KNN ---

def knn(query, source, ptr_q, ptr_s, k: int):
    """(indices int64 [Nq, k], squared distances float32 [Nq, k]);
    geoembodied/csrc/__init__.py:435-492 with ties toward the lower source index."""
    q = _c(query, np.float32).reshape(-1, 3)
    s = _c(source, np.float32).reshape(-1, 3)
    pq, ps = _c(ptr_q, np.int64), _c(ptr_s, np.int64)
    Nq = q.shape[0]
    idx = np.empty((Nq, k), dtype=np.int64)
    dist = np.empty((Nq, k), dtype=np.float32)
    _load().oracle_knn(_p(q), _p(s), _p(pq), _p(ps), pq.shape[0] - 1, int(k), Nq, _p(idx),
                       _p(dist))
    return idx, dist


# ------------------------------------------------------------------------- radius graph ---

def cloud_ids(N: int, batch=None, num_batch_elements=None, mask=None) -> np.ndarray:
    """Cloud id per point (-1: excluded).  With ``batch`` the ids are its values (those outside
    [0, B) excluded); without it, ``num_batch_elements`` contiguous equal chunks
    (geoembodied/functional/radius_graph.py:151-163)."""
    if batch is not None:
        c = _c(batch, np.int64).copy()
        B = int(num_batch_elements) if num_batch_elements is not None else (int(c.max()) + 1 if N else 0)
        c[(c < 0) | (c >= B)] = -1
    else:
        B = int(num_batch_elements) if num_batch_elements is not None else 1
        c = np.arange(N, dtype=np.int64) // max(N // max(B, 1), 1)
    if mask is not None:
        c = np.where(_c(mask, bool), c, -1)
    return c


def radius_graph(x, r: float, max_num_neighbors: int = 32, loop: bool = False, mask=None,
                 batch=None, num_batch_elements=None):
    """(row=source, col=target) int64 sorted by (target, source);
    geoembodied/functional/radius_graph.py:204-335 with the exact squared distance."""
    x = _c(x, np.float32).reshape(-1, 3)
    N = x.shape[0]
    K = int(max_num_neighbors)
    empty = np.zeros(0, dtype=np.int64)
    if N == 0 or K <= 0 or not (float(r) > 0):
        return empty, empty.copy()
    cloud = cloud_ids(N, batch, num_batch_elements, mask)
    r2 = fp32_radius_sq(r)
    deg = np.zeros(N, dtype=np.int64)
    lib = _load()
    lib.oracle_radius(_p(x), N, _p(cloud), r2, K, int(bool(loop)), _p(deg), None, None, None)
    row_ptr = np.zeros(N + 1, dtype=np.int64)
    row_ptr[1:] = np.cumsum(deg)
    E = int(row_ptr[-1])
    row = np.empty(E, dtype=np.int64)
    col = np.empty(E, dtype=np.int64)
    lib.oracle_radius(_p(x), N, _p(cloud), r2, K, int(bool(loop)), None, _p(row_ptr), _p(row),
                      _p(col))
    return row, col


# ---------------------------------------------------------------------------- CSR build ---

def sort_and_build_csr(col, N: int):
    """(col_sorted, perm, node_start, node_end) int32; stable sort by target
    (geoembodied/csrc/segment_reduce_kernel.cu:118-152 ordering, offsets as
    geoembodied/functional/segment_reduce.py:96-102)."""
    col = _c(col, np.int64)
    E = col.shape[0]
    cs = np.empty(E, dtype=np.int32)
    pm = np.empty(E, dtype=np.int32)
    ns = np.empty(int(N), dtype=np.int32)
    ne = np.empty(int(N), dtype=np.int32)
    _load().oracle_csr(_p(col), E, int(N), _p(cs), _p(pm), _p(ns), _p(ne))
    return cs, pm, ns, ne


# ------------------------------------------------------------------------ segment reduce ---

def bf16_round(x) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even, NaN -> 0x7fc0), returned as float32 values."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    r = np.where(nan, 0x7FC00000, r & 0xFFFFFFFF).astype(np.uint32)
    return r.view(np.float32)


def _ranges(node_start, node_end, N, E):
    a = np.clip(_c(node_start, np.int64)[:N], 0, E)
    b = np.clip(_c(node_end, np.int64)[:N], 0, E)
    return a, np.maximum(a, b)


def _rows(perm, E):
    return np.arange(E, dtype=np.int64) if perm is None else _c(perm, np.int64)


def _max_eq(a, b):
    return (a == b) | (np.isnan(a) & np.isnan(b))


def segment_reduce_fwd(msg, perm, node_start, node_end, N: int, reduce: str = "sum",
                       tie_mode: int = 0, segments=None):
    """Forward oracle.  ``msg`` holds the exact input values (bf16 inputs as float32).

    sum:  out[s] = sum of msg[perm[e]] over the segment (float64; the sum of the reference's
          segment_reduce_sum, geoembodied/csrc/segment_reduce_kernel.cu:66-93 and
          geoembodied/functional/segment_reduce.py:161-199), scale[s] = sum |msg|.
    mean: out = sum / max(count, 1) (geoembodied/nn/modules/se3_net.py:264-268), scale / count.
    max:  out = value of the first maximum (NaN above numbers, +-0 equal), empty -> 0
          (geoembodied/nn/modules/invariant_attention.py:212-219); arg = sorted position of the
          first maximum, -1 if empty, -(tie count) when tied and tie_mode == 0.
    Returns (out float64 [S', C], scale or arg [S', C]) for the requested ``segments``.
    """
    m = np.asarray(msg)
    E, C = m.shape
    rows = _rows(perm, E)
    a, b = _ranges(node_start, node_end, N, E)
    segs = np.arange(N) if segments is None else np.asarray(segments)
    out = np.zeros((len(segs), C), dtype=np.float64)
    aux = np.zeros((len(segs), C), dtype=np.float64 if reduce != "max" else np.int64)
    for o, s in enumerate(segs):
        lo, hi = int(a[s]), int(b[s])
        r = rows[lo:hi]
        r = r[(r >= 0) & (r < E)]
        pos = np.arange(lo, hi)[(rows[lo:hi] >= 0) & (rows[lo:hi] < E)]
        vals = m[r].astype(np.float64)
        if reduce in ("sum", "mean"):
            tot = vals.sum(axis=0) if len(r) else np.zeros(C)
            sc = np.abs(vals).sum(axis=0) if len(r) else np.zeros(C)
            if reduce == "mean":
                d = max(hi - lo, 1)
                tot, sc = tot / d, sc / d
            out[o], aux[o] = tot, sc
        else:
            if len(r) == 0:
                out[o], aux[o] = 0.0, -1
                continue
            isn = np.isnan(vals)
            has_nan = isn.any(axis=0)
            mx = np.where(has_nan, np.nan, np.nanmax(np.where(isn, -np.inf, vals), axis=0))
            eq = _max_eq(vals, mx[None, :])
            first = eq.argmax(axis=0)
            cnt = eq.sum(axis=0)
            out[o] = vals[first, np.arange(C)]
            arg = pos[first]
            aux[o] = np.where((cnt == 1) | (tie_mode == 1), arg, -cnt)
    return out, aux


def _div_in_dtype(g: np.ndarray, d: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "float64":
        return g.astype(np.float64) / d
    q = (g.astype(np.float32) / np.asarray(d, dtype=np.float32)).astype(np.float32)
    return bf16_round(q) if dtype == "bfloat16" else q


def segment_reduce_bwd(grad_out, col_sorted, perm, node_start, node_end, E: int,
                       reduce: str = "sum", msg=None, out=None, arg=None,
                       dtype: str = "float32"):
    """Backward oracle, exact in the input dtype.

    sum:  grad_msg[perm[e]] = grad_out[col_sorted[e]] (geoembodied/functional/segment_reduce.py:
          259-270); mean divides by max(count, 1); max routes grad to the recorded argmax or,
          for -(count) ties, grad / count to every position equal to out.
    Rows whose target is out of range get zeros."""
    g = np.asarray(grad_out)
    S, C = g.shape
    cs = _c(col_sorted, np.int64)
    rows = _rows(perm, E)
    res = np.zeros((E, C), dtype=np.float64)
    ok = (cs >= 0) & (cs < S) & (rows >= 0) & (rows < E)
    e_idx = np.nonzero(ok)[0]
    s_idx = cs[e_idx]
    p_idx = rows[e_idx]
    if reduce == "sum":
        res[p_idx] = g[s_idx]
    elif reduce == "mean":
        cnt = (_c(node_end, np.int64) - _c(node_start, np.int64))[s_idx]
        res[p_idx] = _div_in_dtype(g[s_idx], np.maximum(cnt, 1)[:, None], dtype)
    else:
        A = np.asarray(arg)[s_idx]
        gv = g[s_idx]
        first = A == e_idx[:, None]
        tie = A <= -2
        eqv = _max_eq(np.asarray(msg)[p_idx].astype(np.float64), np.asarray(out)[s_idx].astype(np.float64))
        split = _div_in_dtype(gv, np.where(tie, -A, 1), dtype)
        res[p_idx] = np.where(first, gv, np.where(tie & eqv, split, 0.0))
    return res


# ------------------------------------------------------------------------ segment softmax ---

def sparse_softmax(scores, index, N: int) -> np.ndarray:
    """Softmax of scores [E, H] over the edges of each target (float64), following
    _sparse_softmax, geoembodied/nn/modules/invariant_attention.py:202-230: per-target max of the
    edges' scores (NaN propagates), exp(score - max), per-target sum, divide by the sum clamped
    at 1e-8."""
    x = np.asarray(scores, dtype=np.float64)
    squeeze = x.ndim == 1
    if squeeze:
        x = x[:, None]
    idx = np.asarray(index, dtype=np.int64)
    H = x.shape[1]
    m = np.full((N, H), -np.inf)
    np.maximum.at(m, idx, x)
    with np.errstate(invalid="ignore", over="ignore"):
        ex = np.exp(x - m[idx])
    z = np.zeros((N, H))
    np.add.at(z, idx, ex)
    with np.errstate(invalid="ignore"):
        w = ex / np.maximum(z[idx], 1e-8)
    return w[:, 0] if squeeze else w


def sparse_softmax_bwd(grad, w, index, N: int) -> np.ndarray:
    """Gradient of sparse_softmax with respect to the scores: w * (g - per-target sum of g * w)."""
    g = np.asarray(grad, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    idx = np.asarray(index, dtype=np.int64)
    dot = np.zeros((N,) + w.shape[1:])
    np.add.at(dot, idx, g * w)
    return w * (g - dot[idx])


# ------------------------------------------------------------- neighbourhood gather-sum ---

def idw_weights(idx, dist) -> np.ndarray:
    """Inverse-distance weights, float64: v = 1/sqrt(max(d, 1e-4)) for idx >= 0 else 0, divided
    by max(sum v, 1e-8) (geoembodied/nn/modules/equivariant_interp.py:95-99)."""
    i = np.asarray(idx, dtype=np.int64)
    d = np.asarray(dist, dtype=np.float64)
    v = np.where(i >= 0, 1.0 / np.sqrt(np.maximum(d, 1e-4)), 0.0)
    return v / np.maximum(v.sum(-1, keepdims=True), 1e-8)


def gather_weighted_sum(feat, idx, w):
    """(out [N_out, C] float64, scale = sum_k |w| |feat| per element) of out[n] = sum_k w[n, k] *
    feat[idx[n, k]], padding (idx outside [0, N_src)) skipped — the reference's
    (w.unsqueeze(-1) * feat[idx.clamp(min=0)]).sum(1) with zero weights on padding
    (equivariant_interp.py:104-125)."""
    f = np.asarray(feat, dtype=np.float64)
    i = np.asarray(idx, dtype=np.int64)
    wt = np.asarray(w, dtype=np.float64)
    ok = (i >= 0) & (i < f.shape[0])
    g = f[np.where(ok, i, 0)] * ok[..., None]
    return (wt[..., None] * g).sum(1), (np.abs(wt)[..., None] * np.abs(g)).sum(1)


def gather_weighted_sum_bwd(grad_out, feat, idx, w):
    """(grad_feat, grad_w) of gather_weighted_sum, float64."""
    go = np.asarray(grad_out, dtype=np.float64)
    f = np.asarray(feat, dtype=np.float64)
    i = np.asarray(idx, dtype=np.int64)
    wt = np.asarray(w, dtype=np.float64)
    ok = (i >= 0) & (i < f.shape[0])
    gf = np.zeros_like(f)
    n_idx, k_idx = np.nonzero(ok)
    np.add.at(gf, i[n_idx, k_idx], wt[n_idx, k_idx][:, None] * go[n_idx])
    gw = np.where(ok, np.einsum("nc,nkc->nk", go, f[np.where(ok, i, 0)]), 0.0)
    return gf, gw


# ------------------------------------------------------------- adaptive radius statistic ---

def knn_radius_stat(dist, col: int, mode: str, multiplier: float) -> float:
    """mode "mean": multiplier * float32 mean of sqrt(clamp(d, 1e-8, 1e20)) (values in float32,
    summed in float64, rounded once) — geoembodied/nn/modules/multi_scale_se3_net.py:118-123;
    mode "median": multiplier * sqrt(lower median of max(d, 1e-12)), NaN if any d is NaN —
    equivariant_skip_fusion.py:243-248."""
    d = np.asarray(dist, dtype=np.float32)[:, col]
    if mode == "mean":
        v = np.sqrt(np.maximum(np.minimum(d, np.float32(1e20)), np.float32(1e-8)))
        return float(np.float32(v.astype(np.float64).sum() / d.size)) * multiplier
    c = np.maximum(d, np.float32(1e-12))
    if np.isnan(c).any():
        return float("nan")
    return float(np.sqrt(np.sort(c)[(c.size - 1) // 2])) * multiplier


# ---------------------------------------------------- spatial-graph edge geometry + SH ---

def spherical_harmonics(xyz, max_l: int = 2, normalize: bool = False) -> np.ndarray:
    """Real spherical harmonics, float64, order Y_0^0 | Y_1^{-1,0,1} | Y_2^{-2..2}
    (geoembodied/kernels/triton_sph_harm.py:177-220 formulas; normalisation xyz / max(|xyz|,
    1e-8) when asked, triton_sph_harm.py:361-362)."""
    v = np.asarray(xyz, dtype=np.float64).reshape(-1, 3)
    if normalize:
        v = v / np.maximum(np.linalg.norm(v, axis=1, keepdims=True), 1e-8)
    x, y, z = v[:, 0], v[:, 1], v[:, 2]
    cols = [np.full_like(x, np.sqrt(1.0 / (4.0 * np.pi)))]
    if max_l >= 1:
        c1 = np.sqrt(3.0 / (4.0 * np.pi))
        cols += [c1 * y, c1 * z, c1 * x]
    if max_l >= 2:
        c20, c21, c22 = np.sqrt(5.0 / (16.0 * np.pi)), np.sqrt(15.0 / (4.0 * np.pi)), np.sqrt(15.0 / (16.0 * np.pi))
        cols += [c21 * x * y, c21 * y * z, c20 * (3.0 * z * z - 1.0), c21 * x * z, c22 * (x * x - y * y)]
    return np.stack(cols, axis=1)


def edge_geometry(pos, row, col, max_l: int = 2):
    """(direction, dist, Y) float64 of the edges row -> col: diff = pos[col] - pos[row],
    dist = max(|diff|, 1e-8), direction = diff / dist, Y of direction
    (geoembodied/functional/radius_graph.py:336-358, nn/modules/spatial_graph.py:125-129)."""
    p = np.asarray(pos, dtype=np.float64)
    diff = p[np.asarray(col)] - p[np.asarray(row)]
    dist = np.maximum(np.linalg.norm(diff, axis=1), 1e-8)
    direction = diff / dist[:, None]
    return direction, dist, spherical_harmonics(direction, max_l)


def graph_avg_degree(node_start, node_end, batch=None, B: int = 1) -> np.ndarray:
    """Per-node average degree of its cloud, clamped below at 1 (spatial_graph.py:137-152)."""
    deg = np.asarray(node_end, np.float64) - np.asarray(node_start, np.float64)
    N = deg.size
    if batch is None:
        avg = np.full(N, deg.mean() if N else 0.0)
    else:
        b = np.asarray(batch, np.int64)
        s = np.bincount(b, weights=deg, minlength=B)
        c = np.bincount(b, minlength=B)
        avg = (s / np.maximum(c, 1))[b]
    return np.maximum(avg, 1.0)
