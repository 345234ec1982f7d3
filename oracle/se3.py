"""SE3Conv message passing restated on the CPU in float64 — TEST INFRASTRUCTURE ONLY.

Follows the reference's operation sequence: per-edge messages of the nine tensor-product paths
(geoembodied/nn/modules/se3_conv.py:61-235 `_compute_messages`, with the runtime path numbering
of :149-233), concatenation and the segment sum over targets (:516-545), division by the
per-node average degree (:547-558), the scalar bias (:570-571) and the mask (:574-579).  Written
with torch float64 tensors on the CPU so that autograd provides the gradient oracle.

Pinning (tests/test_oracle.py): single-edge closed forms for every path (signs and index
orders of the dot, cross and CG products), rotation equivariance of all three output types,
the identity CG(d, d) = Y_2(d) / sqrt(15 / (8 pi)) tying the CG table to the spherical
harmonics, and the CG table's symmetric-traceless structure.
"""

from __future__ import annotations

import math
from typing import Dict, Optional

import torch

PATH_NAMES = ("w_ss", "w_sv", "w_vv_scalar", "w_vs", "w_vv_cross", "w_st2", "w_t2t2", "w_vt2", "w_t2s")


def cg_11_2_cartesian() -> torch.Tensor:
    """CG(1, 1 -> 2) as [3, 3, 5] in Cartesian (x, y, z) order: the symmetric traceless products
    (xy, yz, (2zz - xx - yy)/sqrt3, xz, (xx - yy)) / sqrt2, the basis order of Y_2
    (tensor_product.py:104-126 permuted to Cartesian as se3_conv.py:384-390 does)."""
    c = torch.zeros(3, 3, 5, dtype=torch.float64)
    h = math.sqrt(0.5)
    x, y, z = 0, 1, 2
    c[x, y, 0] = c[y, x, 0] = h
    c[y, z, 1] = c[z, y, 1] = h
    c[z, z, 2] = 2.0 / math.sqrt(6.0)
    c[x, x, 2] = c[y, y, 2] = -1.0 / math.sqrt(6.0)
    c[x, z, 3] = c[z, x, 3] = h
    c[x, x, 4] = 1.0 / math.sqrt(2.0)
    c[y, y, 4] = -1.0 / math.sqrt(2.0)
    return c


def path_columns(weights: Dict[str, Optional[torch.Tensor]], has_t2_src: bool, has_y2: bool,
                 Ct2_out: int) -> list:
    """Column of R used by each path, -1 where the path does not run (se3_conv.py:149-233: a
    path runs when its weight exists and, for the type-2 paths, its inputs do)."""
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


def se3_conv(s, v, t, row, col, direction, Y, R, weights, cg, Cs_out: int, Cv_out: int,
             Ct2_out: int, avg_degree, bias=None, mask=None):
    """(s_out [N, Cs_out], v_out [N, Cv_out, 3], t_out [N, Ct2_out, 5] or None) in float64."""
    f = torch.float64
    N = s.shape[0]
    E = row.shape[0]
    s_src = s.to(f)[row]
    v_src = v.to(f)[row]
    t_src = t.to(f)[row] if t is not None else None
    d = direction.to(f)
    Y = Y.to(f)
    y0 = Y[:, 0:1]
    y2 = Y[:, 4:9] if Y.shape[1] >= 9 else None
    R = R.to(f)
    W = {k: (w.to(f) if w is not None else None) for k, w in weights.items()}
    pc = path_columns(W, t_src is not None, y2 is not None, Ct2_out)
    sm = torch.zeros(E, Cs_out, dtype=f)
    vm = torch.zeros(E, Cv_out, 3, dtype=f)
    tm = torch.zeros(E, Ct2_out, 5, dtype=f) if Ct2_out > 0 else None

    def r(i):
        return R[:, pc[i]:pc[i] + 1]

    if pc[0] >= 0:
        sm = sm + r(0) * y0 * (s_src @ W["w_ss"].t())
    if pc[1] >= 0:
        vm = vm + (r(1) * (s_src @ W["w_sv"].t())).unsqueeze(-1) * d.unsqueeze(-2)
    if pc[2] >= 0:
        mixed = (v_src.transpose(-1, -2) @ W["w_vv_scalar"].t()).transpose(-1, -2)
        vm = vm + r(2).unsqueeze(-1) * y0.unsqueeze(-1) * mixed
    if pc[3] >= 0:
        dot = (d.unsqueeze(-2) * v_src).sum(-1)
        sm = sm + r(3) * (dot @ W["w_vs"].t())
    if pc[4] >= 0:
        cross = torch.linalg.cross(d.unsqueeze(-2).expand_as(v_src), v_src, dim=-1)
        vm = vm + r(4).unsqueeze(-1) * (cross.transpose(-1, -2) @ W["w_vv_cross"].t()).transpose(-1, -2)
    if pc[5] >= 0:
        tm = tm + (r(5) * (s_src @ W["w_st2"].t())).unsqueeze(-1) * y2.unsqueeze(-2)
    if pc[6] >= 0:
        mixed = (t_src.transpose(-1, -2) @ W["w_t2t2"].t()).transpose(-1, -2)
        tm = tm + r(6).unsqueeze(-1) * y0.unsqueeze(-1) * mixed
    if pc[7] >= 0:
        outer = d.unsqueeze(1).unsqueeze(-1) * v_src.unsqueeze(-2)          # [E, Cv, 3, 3]
        tp = outer.reshape(E, v_src.shape[1], 9) @ cg.to(f).reshape(9, 5)  # [E, Cv, 5]
        tm = tm + r(7).unsqueeze(-1) * (tp.transpose(-1, -2) @ W["w_vt2"].t()).transpose(-1, -2)
    if pc[8] >= 0:
        sm = sm + r(8) * ((t_src * t_src).sum(-1) @ W["w_t2s"].t())

    def agg(m):
        out = torch.zeros((N,) + tuple(m.shape[1:]), dtype=f)
        return out.index_add(0, col, m)

    avg = avg_degree.to(f)
    s_out = agg(sm) / avg.view(N, 1)
    v_out = agg(vm) / avg.view(N, 1, 1)
    t_out = agg(tm) / avg.view(N, 1, 1) if tm is not None else None
    if bias is not None:
        s_out = s_out + bias.to(f)
    if mask is not None:
        keep = mask.view(N, 1).to(f)
        s_out = s_out * keep
        v_out = v_out * keep.unsqueeze(-1)
        if t_out is not None:
            t_out = t_out * keep.unsqueeze(-1)
    return s_out, v_out, t_out


def radial_basis(dist, freqs, cutoff: float, W1, b1, W2, b2):
    """RadialBasis.forward (se3_conv.py:270-282) in float64:
    mlp(sin(freqs d) / max(d, 1e-8) * max(0.5 (1 + cos(pi d / cutoff)), 0))."""
    f = torch.float64
    d = dist.to(f).unsqueeze(-1)
    basis = torch.sin(freqs.to(f) * d) / d.clamp(min=1e-8)
    env = (0.5 * (1.0 + torch.cos(math.pi * dist.to(f) / cutoff))).clamp(min=0.0).unsqueeze(-1)
    h = torch.nn.functional.silu(torch.nn.functional.linear(basis * env, W1.to(f), b1.to(f)))
    return torch.nn.functional.linear(h, W2.to(f), b2.to(f))
