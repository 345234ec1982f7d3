"""Real spherical harmonics Y_l^m(r) for l <= 2 on the GPU (drop-in for
geoembodied/kernels/triton_sph_harm.py, whose Triton kernels it replaces with the gfx950 kernels
of the geometry library).

Channel layout (l = 0..2, 9 channels): Y_0^0 | Y_1^{-1,0,1} | Y_2^{-2,-1,0,1,2}, orthonormal on
the sphere:

    Y_0^0 = 1/(2 sqrt(pi)),   Y_1^{-1,0,1} = sqrt(3/(4 pi)) (y, z, x),
    Y_2^{-2,-1,0,1,2} = sqrt(15/(4 pi)) xy, sqrt(15/(4 pi)) yz, sqrt(5/(16 pi)) (3z^2 - 1),
                        sqrt(15/(4 pi)) xz, sqrt(15/(16 pi)) (x^2 - y^2).

``spherical_harmonics(xyz, max_l, normalize)`` normalises the vectors first when asked
(``xyz / max(|xyz|, 1e-8)``) and is differentiable through the normalisation.
"""

from __future__ import annotations

from typing import List

import torch
from torch import Tensor

from gdl_amd.csrc import (
    edge_geometry_backward_hip,
    spherical_harmonics_backward_hip,
    spherical_harmonics_hip,
)


class SphericalHarmonicsFunction(torch.autograd.Function):
    """Y_l(xyz) for l = 0..max_l with an analytic backward (normalising first when asked)."""

    @staticmethod
    def forward(ctx, xyz: Tensor, max_l: int = 2, normalize: bool = False) -> Tensor:
        Y, unit, norm = spherical_harmonics_hip(xyz, max_l, normalize)
        ctx.max_l, ctx.normalize = max_l, normalize
        ctx.save_for_backward(xyz if not normalize else unit, norm if normalize else xyz)
        return Y

    @staticmethod
    def backward(ctx, grad_Y: Tensor):
        a, b = ctx.saved_tensors
        if ctx.normalize:
            g = edge_geometry_backward_hip(a, b, None, None, grad_Y, ctx.max_l)
        else:
            g = spherical_harmonics_backward_hip(a.to(torch.float32).contiguous(), grad_Y, ctx.max_l)
        return g, None, None


def spherical_harmonics(xyz: Tensor, max_l: int = 2, normalize: bool = True) -> Tensor:
    """Real spherical harmonics of ``xyz [..., 3]`` -> ``[..., (max_l + 1)^2]`` (float32)."""
    if max_l not in (0, 1, 2):
        raise ValueError(f"max_l must be 0, 1, or 2, got {max_l}")
    shape = xyz.shape[:-1]
    out = SphericalHarmonicsFunction.apply(xyz.reshape(-1, 3), max_l, normalize)
    return out.reshape(*shape, (max_l + 1) ** 2)


def get_l_channels(max_l: int) -> List[int]:
    """Channels per degree: [1, 3, 5][: max_l + 1]."""
    return [2 * l + 1 for l in range(max_l + 1)]
