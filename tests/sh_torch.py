"""Real spherical harmonics (l <= 2) in torch, differentiable: the reference's PyTorch formula
(geoembodied/kernels/triton_sph_harm.py:177-220), used by the GPU tests to build float64
autograd references.  The constants are pinned by tests/test_oracle.py (orthonormality on the
sphere and the addition theorem)."""

import math

import torch


def sh_torch(v, max_l):
    x, y, z = v[..., 0], v[..., 1], v[..., 2]
    out = [torch.full_like(x, math.sqrt(1 / (4 * math.pi)))]
    if max_l >= 1:
        c1 = math.sqrt(3 / (4 * math.pi))
        out += [c1 * y, c1 * z, c1 * x]
    if max_l >= 2:
        c20, c21, c22 = math.sqrt(5 / (16 * math.pi)), math.sqrt(15 / (4 * math.pi)), math.sqrt(15 / (16 * math.pi))
        out += [c21 * x * y, c21 * y * z, c20 * (3 * z * z - 1), c21 * x * z, c22 * (x * x - y * y)]
    return torch.stack(out, -1)
