"""Checks of one segment-reduce leg of a BASELINE configuration, shared by the GPU tests.

``reduce_leg_oracle`` compares against the CPU oracle (per-segment fp64 sums, exact max / argmax
and exact backward values), for graphs of up to ~10^6 edges.  ``reduce_leg_fp64`` compares the
largest legs (C3's 4M x 128, C5's 5M-edge lidar graph) against float64 library routines on the
GPU instead of the oracle's per-segment loop: ``index_add`` in float64 for sum and mean (with the
same per-element bound TOL * sum |msg|), torch's ``scatter_reduce('amax', include_self=False)``
and its autograd backward for max (exact), and the gather formulas of the backward (exact).

Bars (the survey's D5-D7): sum / mean within 1e-5 * sum|msg| (fp32), 2e-2 * sum|msg| plus the
final bf16 rounding (bf16); max, every backward and the CSR arrays bit-exact.
"""

import numpy as np
import torch

import oracle

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float64: 1e-12}
CSR_NAMES = ("col_sorted", "perm", "node_start", "node_end")


def _np(t):
    t = t.detach().cpu()
    return t.float().numpy() if t.dtype == torch.bfloat16 else t.numpy()


def csr_checked(dev, col, N):
    """sort_and_build_csr on the GPU, asserted equal to the oracle's stable CSR."""
    from geoembodied.functional.segment_reduce import sort_and_build_csr
    got = sort_and_build_csr(col.to(dev), N)
    want = oracle.sort_and_build_csr(col.cpu().numpy(), N)
    for g, w, name in zip(got, want, CSR_NAMES):
        np.testing.assert_array_equal(g.cpu().numpy(), w, err_msg=name)
    return got


def _assert_within(got, ref, scale, dtype):
    bound = TOL[dtype] * scale + 1e-30
    if dtype == torch.bfloat16:
        bound = bound + np.abs(ref) * 2.0 ** -8
    err = np.abs(got - ref) - bound
    assert np.all(err <= 0), float(err.max())


def reduce_leg_oracle(dev, msg, col, N, reduce, seed=0):
    """segment_reduce(msg [E, C], by target col over N nodes) forward and backward on the GPU
    against the oracle.  Returns the forward output."""
    from geoembodied.functional.segment_reduce import segment_reduce
    cs, pm, ns, ne = csr_checked(dev, col, N)
    E, C = msg.shape
    x = msg.to(dev).detach().clone().requires_grad_(True)
    out = segment_reduce(x, cs, pm, ns, ne, N, reduce=reduce)
    m = _np(msg)
    pm_n, ns_n, ne_n, cs_n = (t.cpu().numpy() for t in (pm, ns, ne, cs))
    ref, aux = oracle.segment_reduce_fwd(m, pm_n, ns_n, ne_n, N, reduce)
    got = _np(out).astype(np.float64)
    if reduce == "max":
        np.testing.assert_array_equal(got, ref)
    else:
        _assert_within(got, ref, aux, msg.dtype)
    g = torch.randn(N, C, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)
    g = g.to(msg.dtype)
    out.backward(g.to(dev))
    want = oracle.segment_reduce_bwd(_np(g), cs_n, pm_n, ns_n, ne_n, E, reduce, msg=m, out=ref,
                                     arg=aux if reduce == "max" else None,
                                     dtype={torch.float32: "float32", torch.bfloat16: "bfloat16",
                                            torch.float64: "float64"}[msg.dtype])
    np.testing.assert_array_equal(_np(x.grad).astype(np.float64), want)
    return out.detach()


def reduce_leg_fp64(msg, cs, pm, ns, ne, N, reduce, grad):
    """The same checks for a large leg, with msg, the CSR arrays and grad [N, C] on the GPU,
    against float64 library routines on the GPU (see the module docstring)."""
    from geoembodied.functional.segment_reduce import segment_reduce
    dev = msg.device
    E, C = msg.shape
    seg_of_pos = cs.long()
    pos_row = pm.long()
    seg_of_row = torch.empty(E, dtype=torch.long, device=dev)
    seg_of_row[pos_row] = seg_of_pos
    count = (ne - ns).long()
    x = msg.detach().clone().requires_grad_(True)
    out = segment_reduce(x, cs, pm, ns, ne, N, reduce=reduce)
    out.backward(grad)
    if reduce in ("sum", "mean"):
        m64 = msg.double()
        ref = torch.zeros(N, C, dtype=torch.float64, device=dev).index_add_(0, seg_of_row, m64)
        scale = torch.zeros(N, C, dtype=torch.float64, device=dev).index_add_(0, seg_of_row,
                                                                              m64.abs())
        del m64
        if reduce == "mean":
            d = count.clamp(min=1).unsqueeze(1).double()
            ref, scale = ref / d, scale / d
        _assert_within(_np(out).astype(np.float64), ref.cpu().numpy(), scale.cpu().numpy(),
                       msg.dtype)
        # backward: grad_msg[row] = grad[segment of row] (/ count for the mean), in msg's dtype
        want = grad[seg_of_row]
        if reduce == "mean":
            want = (grad.float()[seg_of_row] / count[seg_of_row].clamp(min=1).unsqueeze(1).float()
                    ).to(msg.dtype)
        assert torch.equal(x.grad, want)
    else:
        r = msg.detach().clone().requires_grad_(True)
        idx = seg_of_row.unsqueeze(1).expand(E, C)
        ref = torch.zeros(N, C, dtype=msg.dtype, device=dev).scatter_reduce(
            0, idx, r, reduce="amax", include_self=False)
        # torch's backward counts the zero-initialised output as a tie when a maximum is
        # exactly 0; no such segment may occur for this comparison
        assert not bool(((ref == 0) & (count > 0).unsqueeze(1)).any())
        ref.backward(grad)
        assert torch.equal(out.detach(), ref.detach())
        assert torch.equal(x.grad, r.grad)
    return out.detach()
