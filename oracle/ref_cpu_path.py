"""Restatement of the reference's CPU path, used as bench.py's timed CPU baseline.

TEST / BENCH INFRASTRUCTURE ONLY (never imported by the product).  Each function performs the
same sequence of PyTorch operations as the reference's CPU fallback it names, so its run time
is what a user of the reference pays on the CPU:

* ``fps``            — _fps_iterative_fallback, geoembodied/csrc/__init__.py:600-654: a Python
                       loop over clouds and samples, 4 tensor ops per sample.
* ``radius_graph``   — _radius_graph_batched, geoembodied/functional/radius_graph.py:204-275:
                       one batched cdist [B, N, N], squared, masked, top-k along the sources.
* ``knn``            — _knn_bruteforce, geoembodied/csrc/__init__.py:435-492: per cloud, the
                       [n_q, n_s, 3] difference tensor, squared sum, top-k.
* ``sort_and_build_csr`` / ``segment_sum`` — _sort_and_build_csr_pytorch and
                       _segment_reduce_pytorch, geoembodied/functional/segment_reduce.py:77-199:
                       argsort + bincount/cumsum, then a Python loop over segments.
* ``segment_mean`` / ``segment_max`` — the pooling scatters, nn/modules/se3_net.py:226-270 and
                       nn/modules/invariant_attention.py:212-219.
* ``idw_interpolate`` — the interpolation layer's IDW weights and neighbourhood sum,
                       geoembodied/nn/modules/equivariant_interp.py:95-125.
* ``sparse_softmax`` — _sparse_softmax, geoembodied/nn/modules/invariant_attention.py:202-230:
                       scatter 'amax', exp, scatter_add, divide.

Outputs follow those CPU semantics (cdist distances, topk tie order), which differ from the
exact semantics of the GPU kernels at boundary pairs; they are timed, not used as the oracle.
"""

from __future__ import annotations

import torch
from torch import Tensor


def fps(pos: Tensor, ptr: Tensor, k_per_batch: Tensor, max_steps: int | None = None) -> Tensor:
    """``max_steps`` stops each cloud's loop early (a bounded timing sample)."""
    picks = []
    for b in range(ptr.shape[0] - 1):
        lo, hi = int(ptr[b]), int(ptr[b + 1])
        n = hi - lo
        k = min(int(k_per_batch[b]), n)
        if k <= 0:
            continue
        if k >= n:
            picks.append(torch.arange(lo, hi))
            continue
        cloud = pos[lo:hi]
        chosen = torch.zeros(k, dtype=torch.long)
        nearest = torch.full((n,), float("inf"))
        for step in range(k if max_steps is None else min(k, max_steps)):
            centre = cloud[chosen[step]]
            d = (cloud - centre.unsqueeze(0)).pow(2).sum(-1)
            nearest = torch.minimum(nearest, d)
            if step + 1 < k:
                chosen[step + 1] = nearest.argmax()
        picks.append(chosen + lo)
    return torch.cat(picks) if picks else torch.empty(0, dtype=torch.int64)


def radius_graph(x: Tensor, r: float, B: int, max_num_neighbors: int = 32, loop: bool = False):
    n = x.shape[0] // B
    K = min(max_num_neighbors, n)
    pts = x.reshape(B, n, 3)
    d2 = torch.cdist(pts, pts, p=2.0).pow(2)
    d2.masked_fill_(d2 >= r * r, float("inf"))
    if not loop:
        d2.masked_fill_(torch.eye(n, dtype=torch.bool).unsqueeze(0), float("inf"))
    vals, src = d2.topk(K, dim=1, largest=False)
    keep = vals < float("inf")
    base = (torch.arange(B) * n).view(B, 1, 1)
    tgt = torch.arange(n).view(1, 1, n).expand(B, K, n)
    return (src + base)[keep], (tgt + base)[keep]


def knn(query: Tensor, source: Tensor, ptr_q: Tensor, ptr_s: Tensor, k: int):
    nq = query.shape[0]
    idx = torch.full((nq, k), -1, dtype=torch.int64)
    dist = torch.full((nq, k), 1e30, dtype=torch.float32)
    for b in range(ptr_q.shape[0] - 1):
        qa, qb = int(ptr_q[b]), int(ptr_q[b + 1])
        sa, sb = int(ptr_s[b]), int(ptr_s[b + 1])
        if qb <= qa or sb <= sa:
            continue
        diff = query[qa:qb].float().unsqueeze(1) - source[sa:sb].float().unsqueeze(0)
        d = (diff * diff).sum(-1)
        kk = min(k, d.shape[1])
        vals, loc = d.topk(kk, dim=1, largest=False)
        idx[qa:qb, :kk] = loc + sa
        dist[qa:qb, :kk] = vals
    return idx, dist


def sort_and_build_csr(col: Tensor, N: int):
    order = col.argsort()
    counts = torch.bincount(col.int(), minlength=N)
    end = counts.cumsum(0).int()
    start = torch.cat([torch.zeros(1, dtype=torch.int32), end[:-1]])
    return col[order].int(), order.int(), start, end


def segment_sum(msg: Tensor, perm: Tensor, node_start: Tensor, node_end: Tensor, N: int,
                max_segments: int | None = None) -> Tensor:
    """Python loop over segments; ``max_segments`` bounds the sample for timing."""
    out = torch.zeros(N, msg.shape[1], dtype=msg.dtype)
    stop = N if max_segments is None else min(N, max_segments)
    for n in range(stop):
        a = node_start[n].item()
        b = node_end[n].item()
        if a < b:
            out[n] = msg[perm[a:b].long()].sum(dim=0)
    return out


def segment_mean(msg: Tensor, col: Tensor, N: int) -> Tensor:
    """global_mean_pool's scatter formulation, geoembodied/nn/modules/se3_net.py:226-270:
    scatter_add of the rows, divided by bincount clamped at 1."""
    out = torch.zeros(N, msg.shape[1], dtype=msg.dtype)
    out.scatter_add_(0, col.unsqueeze(1).expand_as(msg), msg)
    return out / torch.bincount(col, minlength=N).clamp(min=1).unsqueeze(1).to(msg.dtype)


def segment_max(msg: Tensor, col: Tensor, N: int) -> Tensor:
    """scatter_reduce 'amax' into zeros with include_self=False,
    geoembodied/nn/modules/invariant_attention.py:212-219."""
    out = torch.zeros(N, msg.shape[1], dtype=msg.dtype)
    return out.scatter_reduce_(0, col.unsqueeze(1).expand_as(msg), msg, reduce="amax",
                               include_self=False)


def sparse_softmax(scores: Tensor, index: Tensor, num_nodes: int) -> Tensor:
    """_sparse_softmax, geoembodied/nn/modules/invariant_attention.py:202-230: scatter 'amax'
    into zeros with include_self=False, gather, exp, scatter_add, gather, divide by the sum
    clamped at 1e-8 (the max buffers take the scores' dtype here so float64 runs stay float64)."""
    max_scores = torch.zeros(num_nodes, scores.shape[-1], dtype=scores.dtype)
    max_scores.scatter_reduce_(0, index.unsqueeze(-1).expand_as(scores), scores, reduce="amax",
                               include_self=False)
    shifted = scores - max_scores[index]
    exp_scores = shifted.exp()
    sum_exp = torch.zeros(num_nodes, scores.shape[-1], dtype=scores.dtype)
    sum_exp.scatter_add_(0, index.unsqueeze(-1).expand_as(exp_scores), exp_scores)
    return exp_scores / sum_exp[index].clamp(min=1e-8)


def idw_interpolate(feat: Tensor, knn_idx: Tensor, knn_dists: Tensor) -> Tensor:
    """The interpolation layer's weights and aggregation, geoembodied/nn/modules/
    equivariant_interp.py:95-125: IDW weights, gather with idx.clamp(min=0), weighted sum over
    the neighbours, rows without a valid neighbour set to 0."""
    valid_mask = knn_idx >= 0
    inv_dist = 1.0 / knn_dists.clamp(min=1e-4).sqrt()
    inv_dist = inv_dist.masked_fill(~valid_mask, 0.0)
    weight_sum = inv_dist.sum(dim=-1, keepdim=True).clamp(min=1e-8)
    weights = inv_dist / weight_sum
    safe_idx = knn_idx.clamp(min=0)
    out = (weights.unsqueeze(-1) * feat[safe_idx]).sum(dim=1)
    all_invalid = ~valid_mask.any(dim=1)
    out[all_invalid] = 0.0
    return out
