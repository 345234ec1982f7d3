"""SE(3)-equivariant convolution with fused message passing (drop-in for
geoembodied/nn/modules/se3_conv.py: ``SE3Conv``, ``RadialBasis``).

The reference forms one message per edge for up to nine tensor-product paths, concatenates them
into an ``[E, Cs + 3 Cv + 5 Ct]`` tensor and segment-sums it over targets (se3_conv.py:61-235,
:516-545).  Every path is ``r_p(e) * W_p * x_p(e)`` with ``W_p`` shared by all edges, so here the
r-weighted source features are summed per target node first (one kernel pass over the target
CSR, no per-edge tensor) and the weights applied once per node by an fp32 MFMA GEMM whose
epilogue divides by the average degree, adds the scalar bias and applies the mask.  The
backward is the transposed structure: per-edge gradients of R, the direction and Y from
per-node gradient rows, and source-side sums over the CSR of the sources followed by GEMMs
with the transposed weights.  Weight gradients are long reductions over nodes on the matrix
cores (geo_se3_gemm_tn).

Arithmetic is fp32 (inputs of lower precision are computed in fp32, as the reference does;
float64 inputs are computed in fp32 and returned as float64).  Results equal the reference's
up to the order of the sums.
"""

from __future__ import annotations

import ctypes
import math
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn as nn
from torch import Tensor

from gdl_amd import _native as _nat
from gdl_amd.csrc import _require_gpu, source_csr

PATH_NAMES = ("w_ss", "w_sv", "w_vv_scalar", "w_vs", "w_vv_cross", "w_st2", "w_t2t2", "w_vt2", "w_t2s")


def _pad16(x: int) -> int:
    return (int(x) + 15) // 16 * 16


def _pad64(x: int) -> int:
    return max((int(x) + 63) // 64 * 64, 64)


def cg_11_2_cartesian(dtype=torch.float32, device=None) -> Tensor:
    """CG(1, 1 -> 2) as [3, 3, 5] in Cartesian (x, y, z) order: the symmetric traceless products
    (xy, yz, (2zz - xx - yy)/sqrt3, xz, xx - yy) / sqrt2 in the basis order of Y_2
    (the reference's table, functional/tensor_product.py:104-126, permuted from the (y, z, x)
    order as se3_conv.py:384-390 does)."""
    c = torch.zeros(3, 3, 5, dtype=torch.float64)
    h = math.sqrt(0.5)
    c[0, 1, 0] = c[1, 0, 0] = h
    c[1, 2, 1] = c[2, 1, 1] = h
    c[2, 2, 2] = 2.0 / math.sqrt(6.0)
    c[0, 0, 2] = c[1, 1, 2] = -1.0 / math.sqrt(6.0)
    c[0, 2, 3] = c[2, 0, 3] = h
    c[0, 0, 4] = 1.0 / math.sqrt(2.0)
    c[1, 1, 4] = -1.0 / math.sqrt(2.0)
    return c.to(dtype=dtype, device=device)


def path_columns(weights: Dict[str, Optional[Tensor]], has_t2_src: bool, has_y2: bool,
                 Ct2_out: int) -> list:
    """Column of R of each path, -1 where it does not run.  A path runs when its weight exists
    and, for the type-2 paths, its inputs do; columns are numbered in the order the paths run
    (se3_conv.py:149-233)."""
    run = [
        weights.get("w_ss") is not None,
        weights.get("w_sv") is not None,
        weights.get("w_vv_scalar") is not None,
        weights.get("w_vs") is not None,
        weights.get("w_vv_cross") is not None,
        weights.get("w_st2") is not None and has_y2 and Ct2_out > 0,
        weights.get("w_t2t2") is not None and has_t2_src and Ct2_out > 0,
        weights.get("w_vt2") is not None and Ct2_out > 0,
        weights.get("w_t2s") is not None and has_t2_src,
    ]
    cols, k = [], 0
    for r in run:
        cols.append(k if r else -1)
        k += int(r)
    return cols


class _Plan:
    """Sizes, padded row widths and the path table of one call."""

    def __init__(self, Cs, Cv, Ct, Os, Ov, Ot, pc, P, ysh, t_out):
        self.Cs, self.Cv, self.Ct = Cs, Cv, Ct
        self.Os, self.Ov, self.Ot = Os, Ov, (Ot if t_out else 0)
        self.pc, self.P, self.ysh = pc, P, ysh
        self.Ks = _pad16(Cs + Cv + Ct)
        self.Kv = _pad16(Cs + 2 * Cv)
        self.Kt = _pad16(Cs + Ct + Cv)
        self.OsP, self.OvP, self.OtP = _pad16(self.Os), _pad16(self.Ov), _pad16(self.Ot)
        self.KZs = _pad16(self.Os + self.Ov + self.Ot)
        self.KZv = _pad16(2 * self.Ov + self.Os + self.Ot)
        self.KZt = _pad16(self.Ot)
        self.KZ8 = _pad16(self.Os)
        self.pc_c = (ctypes.c_int32 * 9)(*pc)


def _pack(p: "_Plan", W, specs, device) -> list:
    """Zero-padded weight blocks [(kind, rows, cols), ...] built by one kernel launch."""
    specs = [sp for sp in specs]
    outs = [torch.empty(r, c, dtype=torch.float32, device=device) for _, r, c in specs]
    live = [(o, sp) for o, sp in zip(outs, specs) if o.numel() > 0]
    if live:
        n = len(live)
        wp = (ctypes.c_void_p * 9)(*[(W[i].data_ptr() if p.pc[i] >= 0 else None) for i in range(9)])
        op = (ctypes.c_void_p * n)(*[o.data_ptr() for o, _ in live])
        rows = (ctypes.c_int32 * n)(*[sp[1] for _, sp in live])
        cols = (ctypes.c_int32 * n)(*[sp[2] for _, sp in live])
        kinds = (ctypes.c_int32 * n)(*[sp[0] for _, sp in live])
        _nat.check(_nat.lib().geo_se3_pack_weights(wp, p.Cs, p.Cv, p.Ct, p.Os, p.Ov, p.Ot, n, op, rows,
                                                   cols, kinds, _nat.stream_of(device)),
                   "geo_se3_pack_weights")
    return outs


def _gemm(A: Tensor, M: int, K: int, B: Tensor, O: int, G: int, out: Tensor, ostride: int,
          avg=None, bias=None, mask=None) -> None:
    if M == 0 or O == 0:
        return
    _nat.check(_nat.lib().geo_se3_gemm(
        _nat.ptr(A), M, K, _nat.ptr(B), B.shape[0], O, G, _nat.ptr(out), ostride, _nat.ptr(avg),
        _nat.ptr(bias), _nat.ptr(mask), _nat.stream_of(A.device)), "geo_se3_gemm")


def _plan_of(s: Tensor, v: Tensor, t: Optional[Tensor], Y: Tensor, R: Tensor, dims) -> _Plan:
    """The plan of one call from the feature shapes and ``dims`` = [Os, Ov, Ot, pc_0 .. pc_8]
    (Ot = 0 when no type-2 output is wanted)."""
    Ct = t.shape[1] if t is not None else 0
    Os, Ov, Ot = int(dims[0]), int(dims[1]), int(dims[2])
    return _Plan(s.shape[1], v.shape[1], Ct, Os, Ov, Ot, [int(x) for x in dims[3:12]], R.shape[1],
                 Y.shape[1], Ot > 0)


def _fused(p: _Plan) -> bool:
    """True when the forward runs as one fused launch (its aggregate tile fits in LDS)."""
    return _nat.lib().geo_se3_fwd_fused_lds_bytes(p.Os, p.Ov, p.Ot, p.Ks, p.Kv, p.Kt) > 0


def _u8(mask: Optional[Tensor]) -> Optional[Tensor]:
    return None if mask is None else mask.view(torch.uint8)


_EMPTY = (0,)


# The fused forward and backward are torch.library custom ops with fake implementations, so
# torch.compile traces SE3Conv through them (the reference checks the same transparency for its
# segment-sum op, tests/test_torch_compile.py:83-197).  The nine path weights are separate
# optional arguments; gradients that are not needed come back as empty tensors.
def _se3_fwd_impl(s: Tensor, v: Tensor, t: Optional[Tensor], row: Tensor, col: Tensor,
                perm: Optional[Tensor], node_start: Tensor, node_end: Tensor, direction: Tensor,
                Y: Tensor, R: Tensor, avg: Tensor, mask: Optional[Tensor], bias: Optional[Tensor],
                cg: Optional[Tensor], dims: List[int], w0: Optional[Tensor], w1: Optional[Tensor],
                w2: Optional[Tensor], w3: Optional[Tensor], w4: Optional[Tensor],
                w5: Optional[Tensor], w6: Optional[Tensor], w7: Optional[Tensor],
                w8: Optional[Tensor]) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(s_out, v_out, t_out, Xs, Xv, Xt): outputs and the per-node aggregates (kept for the
    weight gradients when ``dims[12]`` is 1; empty when not kept or their output is not
    computed)."""
    W = (w0, w1, w2, w3, w4, w5, w6, w7, w8)
    p = _plan_of(s, v, t, Y, R, dims)
    keep = len(dims) <= 12 or int(dims[12]) != 0
    dev = s.device
    N, E = s.shape[0], row.shape[0]
    f32 = dict(dtype=torch.float32, device=dev)
    mask_u8 = _u8(mask)
    with _nat.on_device(dev):
        L = _nat.lib()
        st = _nat.stream_of(dev)
        fused = _fused(p)
        keep = keep or not fused
        Xs = torch.empty(N, p.Ks, **f32) if p.Os > 0 and keep else None
        Xv = torch.empty(N, 3, p.Kv, **f32) if p.Ov > 0 and keep else None
        Xt = torch.empty(N, 5, p.Kt, **f32) if p.Ot > 0 and keep else None
        Ws, Wv, Wt = _pack(p, W, [(0, _pad64(p.Os), p.Ks), (1, _pad64(p.Ov), p.Kv),
                                  (2, _pad64(p.Ot), p.Kt)], dev)
        s_out = torch.empty(N, p.Os, **f32)
        v_out = torch.empty(N, p.Ov, 3, **f32)
        t_out = torch.empty(N, p.Ot, 5, **f32)
        if fused:
            # one launch: aggregates in LDS, weights applied there (aggregates to HBM only if kept)
            _nat.check(L.geo_se3_fwd_fused(
                _nat.ptr(s), _nat.ptr(v), _nat.ptr(t), N, p.Cs, p.Cv, p.Ct, _nat.ptr(row),
                _nat.ptr(perm), _nat.ptr(node_start), _nat.ptr(node_end), E, _nat.ptr(direction),
                _nat.ptr(Y), p.ysh, _nat.ptr(R), p.P, p.pc_c, _nat.ptr(cg), _nat.ptr(Ws),
                Ws.shape[0], _nat.ptr(Wv), Wv.shape[0], _nat.ptr(Wt), Wt.shape[0], p.Os, p.Ov, p.Ot,
                p.Ks, p.Kv, p.Kt, _nat.ptr(avg), _nat.ptr(bias), _nat.ptr(mask_u8), _nat.ptr(s_out),
                _nat.ptr(v_out), _nat.ptr(t_out), _nat.ptr(Xs), _nat.ptr(Xv), _nat.ptr(Xt), st),
                "geo_se3_fwd_fused")
        else:
            _nat.check(L.geo_se3_aggregate_fwd(
                _nat.ptr(s), _nat.ptr(v), _nat.ptr(t), N, p.Cs, p.Cv, p.Ct, _nat.ptr(row),
                _nat.ptr(perm), _nat.ptr(node_start), _nat.ptr(node_end), E, _nat.ptr(direction),
                _nat.ptr(Y), p.ysh, _nat.ptr(R), p.P, p.pc_c, _nat.ptr(cg), _nat.ptr(Xs), p.Ks,
                _nat.ptr(Xv), p.Kv, _nat.ptr(Xt), p.Kt, st), "geo_se3_aggregate_fwd")
            _gemm(Xs, N, p.Ks, Ws, p.Os, 1, s_out, p.Os, avg, bias, mask_u8)
            _gemm(Xv, 3 * N, p.Kv, Wv, p.Ov, 3, v_out, 3 * p.Ov, avg, None, mask_u8)
            _gemm(Xt, 5 * N, p.Kt, Wt, p.Ot, 5, t_out, 5 * p.Ot, avg, None, mask_u8)
    empty = s.new_empty(_EMPTY, dtype=torch.float32)
    return (s_out, v_out, t_out, Xs if Xs is not None else empty,
            Xv if Xv is not None else empty.clone(), Xt if Xt is not None else empty.clone())


_se3_fwd_op = torch.library.custom_op("geoembodied::se3_conv_fwd", mutates_args=())(_se3_fwd_impl)


@_se3_fwd_op.register_fake
def _se3_fwd_fake(s, v, t, row, col, perm, node_start, node_end, direction, Y, R, avg, mask, bias,
                  cg, dims, w0, w1, w2, w3, w4, w5, w6, w7, w8):
    p = _plan_of(s, v, t, Y, R, dims)
    keep = len(dims) <= 12 or int(dims[12]) != 0 or not _fused(p)
    N = s.shape[0]
    f = dict(dtype=torch.float32)
    return (s.new_empty(N, p.Os, **f), s.new_empty(N, p.Ov, 3, **f), s.new_empty(N, p.Ot, 5, **f),
            s.new_empty(N, p.Ks, **f) if p.Os > 0 and keep else s.new_empty(_EMPTY, **f),
            s.new_empty(N, 3, p.Kv, **f) if p.Ov > 0 and keep else s.new_empty(_EMPTY, **f),
            s.new_empty(N, 5, p.Kt, **f) if p.Ot > 0 and keep else s.new_empty(_EMPTY, **f))


# gradient slots of the backward op: ds, dv, dt, ddir, dY, dR, dbias, dW0 .. dW8
_NEED_INPUTS = (0, 1, 2, 8, 9, 10, 13, 16, 17, 18, 19, 20, 21, 22, 23, 24)


def _se3_bwd_impl(g_s: Optional[Tensor], g_v: Optional[Tensor], g_t: Optional[Tensor], s: Tensor,
                v: Tensor, t: Optional[Tensor], row: Tensor, col: Tensor, perm: Optional[Tensor],
                node_start: Tensor, node_end: Tensor, direction: Tensor, Y: Tensor, R: Tensor,
                avg: Tensor, mask: Optional[Tensor], cg: Optional[Tensor], Xs: Tensor, Xv: Tensor,
                Xt: Tensor, dims: List[int], need: List[bool], w0: Optional[Tensor],
                w1: Optional[Tensor], w2: Optional[Tensor], w3: Optional[Tensor],
                w4: Optional[Tensor], w5: Optional[Tensor], w6: Optional[Tensor],
                w7: Optional[Tensor], w8: Optional[Tensor]) -> List[Tensor]:
    """[ds, dv, dt, ddir, dY, dR, dbias, dW0 .. dW8]; an entry not in ``need`` is empty."""
    W = (w0, w1, w2, w3, w4, w5, w6, w7, w8)
    p = _plan_of(s, v, t, Y, R, dims)
    dev = s.device
    N, E = s.shape[0], row.shape[0]
    f32 = dict(dtype=torch.float32, device=dev)
    mask_u8 = _u8(mask)
    Xs = Xs if p.Os > 0 else None
    Xv = Xv if p.Ov > 0 else None
    Xt = Xt if p.Ot > 0 else None
    need_s, need_v, need_t, need_dir, need_Y, need_R, need_bias = need[:7]
    need_W = need[7:16]
    if any(need_W[i] and p.pc[i] >= 0 for i in range(9)) and any(
            X is not None and X.dim() == 1 for X in (Xs, Xv, Xt)):
        raise RuntimeError("se3_conv_bwd: weight gradients need the per-node aggregates, which the "
                           "forward kept only if a weight required gradients under grad mode")
    with _nat.on_device(dev):
        L = _nat.lib()
        st = _nat.stream_of(dev)

        def prep(g, O, G, OP):
            if O == 0:
                return None
            out = torch.empty(N, G, OP, **f32)
            gc = (g if g is not None else torch.zeros(N, O, G, **f32)).to(torch.float32).contiguous()
            _nat.check(L.geo_se3_grad_prep(_nat.ptr(gc), N, O, G, OP, _nat.ptr(avg),
                                           _nat.ptr(mask_u8), _nat.ptr(out), st), "geo_se3_grad_prep")
            return out

        Gs = prep(g_s, p.Os, 1, p.OsP)
        Gv = prep(g_v, p.Ov, 3, p.OvP)
        Gt = prep(g_t, p.Ot, 5, p.OtP)
        Cs, Cv, Ct, Os, Ov, Ot = p.Cs, p.Cv, p.Ct, p.Os, p.Ov, p.Ot

        # per-edge gradients of R, direction and Y from gX = G W (per target node)
        dR = ddir = dY = None
        gXs = gXv = gXt = None
        fused_edge = False
        if (need_dir or need_Y or need_R) and E > 0:
            WsT, WvT, WtT = _pack(p, W, [(3, _pad64(p.Ks), p.OsP if Gs is not None else 0),
                                         (4, _pad64(p.Kv), p.OvP if Gv is not None else 0),
                                         (5, _pad64(p.Kt), p.OtP if Gt is not None else 0)], dev)
            dR = torch.zeros(E, p.P, **f32) if need_R else None
            ddir = torch.zeros(E, 3, **f32) if need_dir else None
            dY = torch.zeros(E, p.ysh, **f32) if need_Y else None
            fused_edge = False
            if Gt is None and Ct == 0 and all(p.pc[i] < 0 for i in (5, 6, 7, 8)):
                # gX formed per tile of targets on the chip and used there (never in HBM);
                # layers the tile kernel does not cover fall back to the GEMMs below
                rc = L.geo_se3_bwd_edge_fused(
                    _nat.ptr(s), _nat.ptr(v), N, Cs, Cv, _nat.ptr(row), _nat.ptr(perm),
                    _nat.ptr(node_start), _nat.ptr(node_end), E, _nat.ptr(direction), _nat.ptr(Y),
                    p.ysh, _nat.ptr(R), p.P, p.pc_c, _nat.ptr(cg), _nat.ptr(Gs), p.OsP,
                    _nat.ptr(Gv), p.OvP, _nat.ptr(WsT), WsT.shape[0], _nat.ptr(WvT), WvT.shape[0],
                    p.Ks, p.Kv, _nat.ptr(dR), _nat.ptr(ddir), _nat.ptr(dY), st)
                if rc == 0:
                    fused_edge = True
                elif rc != _nat.GEO_ERR_UNSUPPORTED:
                    _nat.check(rc, "geo_se3_bwd_edge_fused")
        if (need_dir or need_Y or need_R) and E > 0 and not fused_edge:
            if Gs is not None:
                gXs = torch.empty(N, p.Ks, **f32)
                _gemm(Gs, N, p.OsP, WsT, p.Ks, 1, gXs, p.Ks)
            if Gv is not None:
                gXv = torch.empty(N, 3, p.Kv, **f32)
                _gemm(Gv, 3 * N, p.OvP, WvT, p.Kv, 1, gXv, p.Kv)
            if Gt is not None:
                gXt = torch.empty(N, 5, p.Kt, **f32)
                _gemm(Gt, 5 * N, p.OtP, WtT, p.Kt, 1, gXt, p.Kt)
            _nat.check(L.geo_se3_bwd_edge(
                _nat.ptr(s), _nat.ptr(v), _nat.ptr(t), N, Cs, Cv, Ct, _nat.ptr(row), _nat.ptr(perm),
                _nat.ptr(node_start), _nat.ptr(node_end), E, _nat.ptr(direction), _nat.ptr(Y), p.ysh,
                _nat.ptr(R), p.P, p.pc_c, _nat.ptr(cg), _nat.ptr(gXs), p.Ks, _nat.ptr(gXv), p.Kv,
                _nat.ptr(gXt), p.Kt, _nat.ptr(dR), _nat.ptr(ddir), _nat.ptr(dY), st),
                "geo_se3_bwd_edge")

        # feature gradients: source-side sums over the CSR of the sources, then GEMMs with W^T
        ds = dv = dt = None
        want_s, want_v, want_t = need_s and Cs > 0, need_v and Cv > 0, need_t and Ct > 0
        fused_src = False
        if (want_s or want_v) and not want_t and all(p.pc[i] < 0 for i in (5, 6, 7, 8)):
            # no type-2 paths: the source-side sums and the GEMMs with the transposed weights in
            # one launch (the sums stay in LDS); layers the row kernel does not cover fall back
            perm_r, ns_r, ne_r = source_csr(row, N)
            Bs, Bv = _pack(p, W, [(6, _pad64(Cs), p.KZs if want_s else 0),
                                  (7, _pad64(Cv), p.KZv if want_v else 0)], dev)
            ds = torch.empty(N, Cs, **f32) if want_s else None
            dv = torch.empty(N, Cv, 3, **f32) if want_v else None
            rc = L.geo_se3_bwd_src_fused(
                _nat.ptr(Gs), Os, p.OsP, _nat.ptr(Gv), Ov, p.OvP, N, _nat.ptr(col),
                _nat.ptr(perm_r), _nat.ptr(ns_r), _nat.ptr(ne_r), E, _nat.ptr(direction),
                _nat.ptr(Y), p.ysh, _nat.ptr(R), p.P, p.pc_c, _nat.ptr(cg), p.KZs, p.KZv,
                _nat.ptr(Bs), Bs.shape[0], Cs, _nat.ptr(ds), _nat.ptr(Bv), Bv.shape[0], Cv,
                _nat.ptr(dv), st)
            if rc == 0:
                fused_src = True
            elif rc == _nat.GEO_ERR_UNSUPPORTED:
                ds = dv = None
            else:
                _nat.check(rc, "geo_se3_bwd_src_fused")
        if (want_s or want_v or want_t) and not fused_src:
            perm_r, ns_r, ne_r = source_csr(row, N)
            Zs = torch.empty(N, p.KZs, **f32) if want_s else None
            Zv = torch.empty(N, 3, p.KZv, **f32) if want_v else None
            Zt = torch.empty(N, 5, p.KZt, **f32) if want_t and Ot > 0 else None
            Z8 = torch.empty(N, p.KZ8, **f32) if want_t and p.pc[8] >= 0 else None
            _nat.check(L.geo_se3_bwd_src(
                _nat.ptr(Gs), Os, p.OsP, _nat.ptr(Gv), Ov, p.OvP, _nat.ptr(Gt), Ot, p.OtP, N,
                _nat.ptr(col), _nat.ptr(perm_r), _nat.ptr(ns_r), _nat.ptr(ne_r), E,
                _nat.ptr(direction), _nat.ptr(Y), p.ysh, _nat.ptr(R), p.P, p.pc_c, _nat.ptr(cg),
                _nat.ptr(Zs), p.KZs, _nat.ptr(Zv), p.KZv, _nat.ptr(Zt), p.KZt, _nat.ptr(Z8), p.KZ8,
                st), "geo_se3_bwd_src")

            t6 = want_t and Zt is not None and p.pc[6] >= 0
            Bs, Bv, Bt, B8 = _pack(p, W, [(6, _pad64(Cs), p.KZs if want_s else 0),
                                          (7, _pad64(Cv), p.KZv if want_v else 0),
                                          (8, _pad64(Ct), p.KZt if t6 else 0),
                                          (9, _pad64(Ct), p.KZ8 if Z8 is not None else 0)], dev)
            if want_s:
                ds = torch.empty(N, Cs, **f32)
                _gemm(Zs, N, p.KZs, Bs, Cs, 1, ds, Cs)
            if want_v:
                dv = torch.empty(N, Cv, 3, **f32)
                _gemm(Zv, 3 * N, p.KZv, Bv, Cv, 3, dv, 3 * Cv)
            if want_t:
                dt = torch.zeros(N, Ct, 5, **f32)
                if t6:
                    _gemm(Zt, 5 * N, p.KZt, Bt, Ct, 5, dt, 5 * Ct)
                if Z8 is not None:
                    u = torch.empty(N, Ct, **f32)
                    _gemm(Z8, N, p.KZ8, B8, Ct, 1, u, Ct)
                    dt = dt + 2.0 * t * u.unsqueeze(-1)

        # weight gradients: sums over nodes of (prepared output gradient) x (per-node aggregate)
        dW = [None] * 9
        for Gm, Xm, rows, OP, O_, KX, width, parts in (
                (Gs, Xs, N, p.OsP, Os, p.Ks, Cs + Cv + Ct,
                 ((0, 0, Cs), (3, Cs, Cs + Cv), (8, Cs + Cv, Cs + Cv + Ct))),
                (Gv, Xv, 3 * N, p.OvP, Ov, p.Kv, Cs + 2 * Cv,
                 ((1, 0, Cs), (2, Cs, Cs + Cv), (4, Cs + Cv, Cs + 2 * Cv))),
                (Gt, Xt, 5 * N, p.OtP, Ot, p.Kt, Cs + Ct + Cv,
                 ((5, 0, Cs), (6, Cs, Cs + Ct), (7, Cs + Ct, Cs + Ct + Cv)))):
            if Gm is None or not any(need_W[i] and p.pc[i] >= 0 for i, _, _ in parts) or width == 0:
                continue
            # each path's block of the product straight into its own gradient tensor (outputs
            # of a custom op may not alias each other, so no views of one shared result)
            for i, a, b in parts:
                if p.pc[i] >= 0 and need_W[i]:
                    dW[i] = torch.empty(O_, b - a, **f32)
            cols = (ctypes.c_int32 * 4)(*[a for _, a, _ in parts], parts[-1][2])
            outs = (ctypes.c_void_p * 3)(*[dW[i].data_ptr() if dW[i] is not None else None
                                           for i, _, _ in parts])
            nbytes = L.geo_se3_gemm_tn_workspace_bytes(rows, O_, width)
            ws = _nat.workspace(nbytes, dev)
            _nat.check(L.geo_se3_gemm_tn_split(_nat.ptr(Gm), rows, OP, O_, _nat.ptr(Xm), KX, width,
                                               len(parts), cols, outs, _nat.ptr(ws), nbytes, st),
                       "geo_se3_gemm_tn_split")
        dbias = None
        if need_bias and g_s is not None:
            # sum over the (unmasked) nodes of the scalar output gradient, in a fixed order
            dbias = torch.empty(Os, **f32)
            gc = g_s.to(torch.float32).contiguous()
            nbytes = L.geo_se3_colsum_workspace_bytes(N, Os)
            ws = _nat.workspace(nbytes, dev)
            _nat.check(L.geo_se3_colsum(_nat.ptr(gc), N, Os, _nat.ptr(mask_u8), _nat.ptr(dbias),
                                        _nat.ptr(ws), nbytes, st), "geo_se3_colsum")
        elif need_bias:
            dbias = torch.zeros(Os, **f32)
    # a requested gradient has its input's shape (zeros where nothing contributes: no channels,
    # no edges, a path that does not run); one not requested is an empty placeholder
    shapes = _bwd_shapes(s, v, t, row, Y, R, dims, need, W)
    outs = [ds, dv, dt, ddir, dY, dR, dbias, *dW]
    return [o if o is not None else torch.zeros(sh, **f32) for o, sh in zip(outs, shapes)]


def _bwd_shapes(s, v, t, row, Y, R, dims, need, W):
    """Shapes of the backward op's outputs: the input's shape where ``need``, else (0,)."""
    N, E = s.shape[0], row.shape[0]
    Ct = t.shape[1] if t is not None else 0
    full = [(N, s.shape[1]), (N, v.shape[1], 3), (N, Ct, 5), (E, 3), (E, Y.shape[1]),
            (E, R.shape[1]), (int(dims[0]),)]
    full += [tuple(w.shape) if w is not None else _EMPTY for w in W]
    return [sh if n else _EMPTY for sh, n in zip(full, need)]


_se3_bwd_op = torch.library.custom_op("geoembodied::se3_conv_bwd", mutates_args=())(_se3_bwd_impl)


@_se3_bwd_op.register_fake
def _se3_bwd_fake(g_s, g_v, g_t, s, v, t, row, col, perm, node_start, node_end, direction, Y, R,
                  avg, mask, cg, Xs, Xv, Xt, dims, need, w0, w1, w2, w3, w4, w5, w6, w7, w8):
    shapes = _bwd_shapes(s, v, t, row, Y, R, dims, need, (w0, w1, w2, w3, w4, w5, w6, w7, w8))
    return [s.new_empty(sh, dtype=torch.float32) for sh in shapes]


def _se3_setup(ctx, inputs, output) -> None:
    (s, v, t, row, col, perm, ns, ne, direction, Y, R, avg, mask, bias, cg, dims, *W) = inputs
    s_out, v_out, t_out, Xs, Xv, Xt = output
    ctx.dims = list(dims)
    ctx.set_materialize_grads(False)
    ctx.mark_non_differentiable(Xs, Xv, Xt)
    ctx.save_for_backward(s, v, t, row, col, perm, ns, ne, direction, Y, R, avg, mask, cg, Xs, Xv,
                          Xt, *W)


def _se3_grads(ctx, g_s, g_v, g_t, bwd):
    """Gradients of the forward's inputs, in its argument order, from the backward ``bwd``."""
    (s, v, t, row, col, perm, ns, ne, direction, Y, R, avg, mask, cg, Xs, Xv, Xt,
     *W) = ctx.saved_tensors
    ni = ctx.needs_input_grad
    need = [bool(ni[i]) for i in _NEED_INPUTS]
    grads = bwd(g_s, g_v, g_t, s, v, t, row, col, perm, ns, ne, direction, Y, R, avg, mask, cg,
                Xs, Xv, Xt, ctx.dims, need, *W)
    g = [x if n else None for x, n in zip(grads, need)]
    ds, dv, dt, ddir, dY, dR, dbias, *dW = g
    return (ds, dv, dt, None, None, None, None, None, ddir, dY, dR, None, None, dbias, None, None,
            *dW)


def _se3_backward(ctx, g_s, g_v, g_t, _gXs, _gXv, _gXt):
    return _se3_grads(ctx, g_s, g_v, g_t, torch.ops.geoembodied.se3_conv_bwd)


_se3_fwd_op.register_autograd(_se3_backward, setup_context=_se3_setup)


def _plain_eager(x: Tensor) -> bool:
    """True for a plain tensor outside tracing: the eager path may call the implementations
    directly.  Fake or other subclassed tensors, and torch.compile, take the custom ops."""
    return type(x) is torch.Tensor and not torch.compiler.is_compiling()


class _SE3ConvEager(torch.autograd.Function):
    """Eager mode: the custom ops' forward and backward implementations called directly.  The
    custom-op layers (schema defaults, dispatch, the registered autograd) cost more host time per
    call than a C2 layer's kernels take; under torch.compile the custom ops are used, so the
    compiled graph still traces through them."""

    @staticmethod
    def forward(ctx, *args):
        out = _se3_fwd_impl(*args)
        _se3_setup(ctx, args, out)
        return tuple(out)

    @staticmethod
    def backward(ctx, g_s, g_v, g_t, _gXs, _gXv, _gXt):
        return _se3_grads(ctx, g_s, g_v, g_t, _se3_bwd_impl)

_DEFAULT_CG: Dict[torch.device, Tensor] = {}


def _cg_on(device: torch.device) -> Tensor:
    """The CG(1,1->2) table on `device` (built once per device)."""
    t = _DEFAULT_CG.get(device)
    if t is None:
        t = _DEFAULT_CG[device] = cg_11_2_cartesian(device=device).contiguous()
    return t


def se3_message_aggregate(
    scalars: Tensor,
    vectors: Tensor,
    graph,
    R: Tensor,
    weights: Dict[str, Optional[Tensor]],
    Cs_out: int,
    Cv_out: int,
    Ct2_out: int = 0,
    type2: Optional[Tensor] = None,
    cg_11_2: Optional[Tensor] = None,
    bias: Optional[Tensor] = None,
    mask: Optional[Tensor] = None,
    return_type2: bool = False,
):
    """Messages of the nine tensor-product paths summed over each target's edges, divided by the
    per-node average degree, plus the scalar bias, masked (se3_conv.py:61-235 and :482-579 from
    the radial weights R on).  ``graph`` provides row, col, perm, node_start, node_end (CSR of the
    targets), direction, Y, avg_degree and N.  Returns (s [N, Cs_out], v [N, Cv_out, 3]) or with
    ``return_type2`` also t [N, Ct2_out, 5]; differentiable with respect to the features, the
    graph's direction and Y, R, the weights and the bias.  No host synchronisation."""
    _require_gpu("se3_message_aggregate", scalars, vectors, R)
    dev = scalars.device
    N = int(graph.N)
    f32 = torch.float32
    s = scalars.to(f32).contiguous()
    v = vectors.to(f32).contiguous()
    Cv = v.shape[1]
    if s.shape[0] != N or v.shape[0] != N or v.shape[2] != 3:
        raise ValueError(f"se3_message_aggregate: features {tuple(s.shape)}, {tuple(v.shape)} for N={N}")
    t = type2.to(f32).contiguous() if type2 is not None else None
    Ct = t.shape[1] if t is not None else 0
    Y = graph.Y.to(f32).contiguous()
    ysh = Y.shape[1]
    pc = path_columns(weights, t is not None and Ct > 0, ysh >= 9, Ct2_out)
    if t is not None and Ct == 0:
        t = None
    R = R.to(f32).contiguous()
    P = R.shape[1]
    if max(pc) >= P:
        raise ValueError(f"se3_message_aggregate: {max(pc) + 1} paths run but R has {P} columns")
    Ot = Ct2_out if (return_type2 and Ct2_out > 0) else 0
    # the per-node aggregates go to HBM only when a weight gradient will need them
    keep = torch.is_grad_enabled() and any(w is not None and w.requires_grad
                                           for w in weights.values())
    dims = [int(Cs_out), int(Cv_out), int(Ot), *pc, int(keep)]
    cg = None
    if pc[7] >= 0:
        cg = (cg_11_2.to(device=dev, dtype=f32).contiguous() if cg_11_2 is not None
              else _cg_on(dev))
    row = graph.row.to(device=dev, dtype=torch.int64).contiguous()
    col = graph.col.to(device=dev, dtype=torch.int64).contiguous()
    perm = None if getattr(graph, "_perm_identity", False) else \
        graph.perm.to(device=dev, dtype=torch.int32).contiguous()
    ns = graph.node_start.to(device=dev, dtype=torch.int32).contiguous()
    ne = graph.node_end.to(device=dev, dtype=torch.int32).contiguous()
    avg = graph.avg_degree
    avg = (avg.to(device=dev, dtype=f32).contiguous() if avg is not None
           else torch.ones(N, dtype=f32, device=dev))
    m = None
    if mask is not None:
        m = mask.to(device=dev, dtype=torch.bool).reshape(-1).contiguous()
    b = bias.to(f32).contiguous() if bias is not None and Cs_out > 0 else None
    Wl = [(weights.get(k).to(f32).contiguous() if weights.get(k) is not None else None)
          for k in PATH_NAMES]
    direction = graph.direction.to(f32).contiguous()
    args = (s, v, t, row, col, perm, ns, ne, direction, Y, R, avg, m, b, cg, dims, *Wl)
    if _plain_eager(s):
        s_out, v_out, t_out, _, _, _ = _SE3ConvEager.apply(*args)
    else:
        s_out, v_out, t_out, _, _, _ = torch.ops.geoembodied.se3_conv_fwd(*args)
    if return_type2:
        return s_out, v_out, (t_out if Ct2_out > 0 else None)
    return s_out, v_out


def _radial_impl(dist: Tensor, freqs: Tensor, cutoff: float, W1: Tensor, b1: Tensor, W2: Tensor,
               b2: Tensor) -> Tensor:
    """R = W2 silu(W1 (basis(dist) * envelope(dist)) + b1) + b2 in one kernel (fp32 inputs)."""
    dev = dist.device
    E = dist.shape[0]
    H, NB = W1.shape
    P = W2.shape[0]
    R = torch.empty(E, P, dtype=torch.float32, device=dev)
    with _nat.on_device(dev):
        _nat.check(_nat.lib().geo_radial_mlp_fwd(
            _nat.ptr(dist), E, _nat.ptr(freqs), NB, float(cutoff), _nat.ptr(W1), _nat.ptr(b1), H,
            _nat.ptr(W2), _nat.ptr(b2), P, _nat.ptr(R), _nat.stream_of(dev)), "geo_radial_mlp_fwd")
    return R


_radial_op = torch.library.custom_op("geoembodied::radial_mlp", mutates_args=())(_radial_impl)


@_radial_op.register_fake
def _radial_fake(dist, freqs, cutoff, W1, b1, W2, b2):
    return dist.new_empty(dist.shape[0], W2.shape[0], dtype=torch.float32)


def _radial_bwd_impl(dR: Tensor, dist: Tensor, freqs: Tensor, cutoff: float, W1: Tensor, b1: Tensor,
                   W2: Tensor, b2: Tensor, need: List[bool]) -> List[Tensor]:
    """[d dist, dW1, db1, dW2, db2]; an entry not in ``need`` is empty."""
    dev = dist.device
    E = dist.shape[0]
    H, NB = W1.shape
    P = W2.shape[0]
    f32 = dict(dtype=torch.float32, device=dev)
    shapes = ((E,), (H, NB), (H,), (P, H), (P,))
    outs = [torch.empty(sh, **f32) if n else None for sh, n in zip(shapes, need)]
    g = dR.to(torch.float32).contiguous()
    L = _nat.lib()
    with _nat.on_device(dev):
        nbytes = L.geo_radial_mlp_bwd_workspace_bytes(E, NB, H, P)
        ws = _nat.workspace(nbytes, dev)
        _nat.check(L.geo_radial_mlp_bwd(
            _nat.ptr(dist), E, _nat.ptr(freqs), NB, float(cutoff), _nat.ptr(W1), _nat.ptr(b1), H,
            _nat.ptr(W2), _nat.ptr(b2), P, _nat.ptr(g), *[_nat.ptr(o) for o in outs], _nat.ptr(ws),
            nbytes, _nat.stream_of(dev)), "geo_radial_mlp_bwd")
    return [o if o is not None else dist.new_empty(_EMPTY, dtype=torch.float32) for o in outs]


_radial_bwd_op = torch.library.custom_op("geoembodied::radial_mlp_bwd",
                                         mutates_args=())(_radial_bwd_impl)


@_radial_bwd_op.register_fake
def _radial_bwd_fake(dR, dist, freqs, cutoff, W1, b1, W2, b2, need):
    E = dist.shape[0]
    H, NB = W1.shape
    P = W2.shape[0]
    shapes = ((E,), (H, NB), (H,), (P, H), (P,))
    return [dist.new_empty(sh if n else _EMPTY, dtype=torch.float32) for sh, n in zip(shapes, need)]


def _radial_setup(ctx, inputs, output) -> None:
    dist, freqs, cutoff, W1, b1, W2, b2 = inputs
    ctx.cutoff = float(cutoff)
    ctx.save_for_backward(dist, freqs, W1, b1, W2, b2)


def _radial_grads(ctx, dR, bwd):
    dist, freqs, W1, b1, W2, b2 = ctx.saved_tensors
    ni = ctx.needs_input_grad
    need = [bool(ni[i]) for i in (0, 3, 4, 5, 6)]
    grads = bwd(dR, dist, freqs, ctx.cutoff, W1, b1, W2, b2, need)
    dd, dW1, db1, dW2, db2 = [x if n else None for x, n in zip(grads, need)]
    return dd, None, None, dW1, db1, dW2, db2


def _radial_backward(ctx, dR):
    return _radial_grads(ctx, dR, torch.ops.geoembodied.radial_mlp_bwd)


_radial_op.register_autograd(_radial_backward, setup_context=_radial_setup)


class _RadialEager(torch.autograd.Function):
    """Eager mode: the radial custom ops' implementations called directly (as _SE3ConvEager)."""

    @staticmethod
    def forward(ctx, *args):
        R = _radial_impl(*args)
        _radial_setup(ctx, args, R)
        return R

    @staticmethod
    def backward(ctx, dR):
        return _radial_grads(ctx, dR, _radial_bwd_impl)


def radial_mlp(dist: Tensor, freqs: Tensor, cutoff: float, W1: Tensor, b1: Tensor, W2: Tensor,
               b2: Tensor) -> Tensor:
    """Radial weights [E, P] of edge lengths ``dist`` [E] (fp32, on the GPU; any layer sizes:
    matrix-core kernels up to 16 basis functions, 64 hidden units and 16 outputs, LDS-tiled
    kernels beyond), differentiable with respect to dist and the four weights."""
    _require_gpu("radial_mlp", dist)
    f = torch.float32
    c = [x.to(f).contiguous() for x in (dist, freqs, W1, b1, W2, b2)]
    args = (c[0], c[1], float(cutoff), c[2], c[3], c[4], c[5])
    if _plain_eager(c[0]):
        return _RadialEager.apply(*args)
    return torch.ops.geoembodied.radial_mlp(*args)


class RadialBasis(nn.Module):
    """Radial weights of the edge lengths: sinusoidal basis sin(k pi d / cutoff) / d times the
    cosine envelope 0.5 (1 + cos(pi d / cutoff)) clamped at 0, through a two-layer SiLU MLP
    (se3_conv.py:238-282; same parameter names)."""

    def __init__(self, num_basis: int = 16, cutoff: float = 5.0, num_hidden: int = 64,
                 num_output: int = 1) -> None:
        super().__init__()
        self.cutoff = cutoff
        self.num_basis = num_basis
        freqs = torch.arange(1, num_basis + 1).float() * math.pi / cutoff
        self.register_buffer("freqs", freqs)
        self.mlp = nn.Sequential(nn.Linear(num_basis, num_hidden), nn.SiLU(),
                                 nn.Linear(num_hidden, num_output))

    def forward(self, dist: Tensor) -> Tensor:
        """[E] edge lengths -> [E, num_output] radial weights (one fused kernel; fp32)."""
        l1, l2 = self.mlp[0], self.mlp[2]
        R = radial_mlp(dist.reshape(-1), self.freqs, self.cutoff, l1.weight, l1.bias, l2.weight,
                       l2.bias)
        return R.reshape(*dist.shape, l2.weight.shape[0])


class SE3Conv(nn.Module):
    """SE(3)-equivariant continuous convolution (se3_conv.py:285-602): the reference's
    constructor, parameter names (``w_ss`` ... ``w_t2s`` as bias-free ``nn.Linear``,
    ``radial_basis``, ``scalar_bias``, buffer ``cg_11_2``) and forward contract, with the
    messages and their aggregation computed by the fused GPU kernels."""

    def __init__(self, in_scalar_channels: int, in_vector_channels: int, out_scalar_channels: int,
                 out_vector_channels: int, in_type2_channels: int = 0, out_type2_channels: int = 0,
                 radius: float = 2.0, max_num_neighbors: int = 32,
                 num_radial_basis: int = 16) -> None:
        super().__init__()
        self.in_scalar_channels = in_scalar_channels
        self.in_vector_channels = in_vector_channels
        self.out_scalar_channels = out_scalar_channels
        self.out_vector_channels = out_vector_channels
        self.in_type2_channels = in_type2_channels
        self.out_type2_channels = out_type2_channels
        self.radius = radius
        self.max_num_neighbors = max_num_neighbors
        cs, cv, ct = in_scalar_channels, in_vector_channels, in_type2_channels
        os_, ov, ot = out_scalar_channels, out_vector_channels, out_type2_channels
        spec = {
            "w_ss": (cs, os_), "w_sv": (cs, ov), "w_vv_scalar": (cv, ov), "w_vs": (cv, os_),
            "w_vv_cross": (cv, ov), "w_st2": (cs, ot), "w_t2t2": (ct, ot), "w_vt2": (cv, ot),
            "w_t2s": (ct, os_),
        }
        self._num_paths = 0
        for name in PATH_NAMES:
            i, o = spec[name]
            if i > 0 and o > 0:
                setattr(self, name, nn.Linear(i, o, bias=False))
                self._num_paths += 1
            else:
                setattr(self, name, None)
        if self.w_vt2 is not None:
            self.register_buffer("cg_11_2", cg_11_2_cartesian())
        else:
            self.register_buffer("cg_11_2", None)
        self.radial_basis = RadialBasis(num_basis=num_radial_basis, cutoff=radius, num_hidden=64,
                                        num_output=max(self._num_paths, 1))
        self.scalar_bias = nn.Parameter(torch.zeros(os_)) if os_ > 0 else None

    def forward(self, scalars: Tensor, vectors: Tensor, graph, mask: Optional[Tensor] = None,
                type2: Optional[Tensor] = None):
        """(s_out [N, Cs_out], v_out [N, Cv_out, 3]) or with type-2 input and output also
        t_out [N, Ct2_out, 5], in the input dtype (se3_conv.py:429-566)."""
        N = graph.N
        input_dtype = scalars.dtype
        has_type2 = type2 is not None and self.out_type2_channels > 0
        if graph.E == 0:
            s_out = scalars.new_zeros(N, self.out_scalar_channels)
            v_out = vectors.new_zeros(N, self.out_vector_channels, 3)
            s_out = s_out + (scalars.sum() * 0).unsqueeze(0)
            v_out = v_out + (vectors.sum() * 0).unsqueeze(0).unsqueeze(0)
            if self.scalar_bias is not None:
                s_out = s_out + self.scalar_bias
            if has_type2:
                return s_out, v_out, scalars.new_zeros(N, self.out_type2_channels, 5)
            return s_out, v_out
        with torch.autocast(scalars.device.type, enabled=False):
            R = self.radial_basis(graph.dist.to(torch.float32))
            weights = {k: (getattr(self, k).weight if getattr(self, k) is not None else None)
                       for k in PATH_NAMES}
            t_in = type2 if (type2 is not None and self.in_type2_channels > 0) else None
            out = se3_message_aggregate(
                scalars, vectors, graph, R, weights, self.out_scalar_channels,
                self.out_vector_channels, self.out_type2_channels, type2=t_in,
                cg_11_2=self.cg_11_2, bias=self.scalar_bias, mask=mask, return_type2=has_type2)
        if has_type2:
            s_out, v_out, t_out = out
            return s_out.to(input_dtype), v_out.to(input_dtype), t_out.to(input_dtype)
        s_out, v_out = out
        return s_out.to(input_dtype), v_out.to(input_dtype)

    def forward_legacy(self, pos: Tensor, scalars: Tensor, vectors: Tensor,
                       batch: Optional[Tensor] = None, mask: Optional[Tensor] = None,
                       edge_index: Optional[Tuple[Tensor, Tensor]] = None):
        """Builds the graph from ``pos`` (or ``edge_index``) first (se3_conv.py:581-596)."""
        from gdl_amd.graph import SpatialGraph
        if edge_index is not None:
            row, col = edge_index
            graph = SpatialGraph.from_edge_index(row, col, pos, pos.shape[0])
        else:
            graph = SpatialGraph.build(pos, self.radius, max_num_neighbors=self.max_num_neighbors,
                                       batch=batch, mask=mask)
        return self.forward(scalars, vectors, graph, mask=mask)

    def extra_repr(self) -> str:
        return (f"scalar: {self.in_scalar_channels}→{self.out_scalar_channels}, "
                f"vector: {self.in_vector_channels}→{self.out_vector_channels}, "
                f"type2: {self.in_type2_channels}→{self.out_type2_channels}, "
                f"radius={self.radius}, paths={self._num_paths}")
