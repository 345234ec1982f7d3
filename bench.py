#!/usr/bin/env python3
"""Benchmark of the gfx950 geometry kernels on the reference's headline workloads.

Headline (``value``): wall time per batch of farthest point sampling + radius graph on
configuration C2 — 16 clouds x 4096 points on unit spheres with 0.01 jitter, FPS to 1024 per
cloud, radius graph r = 0.1 with at most 32 neighbours over all 65,536 points — including each
op's single output-size host sync (as the reference's examples/registration/diagnose_perf.py
times ops: perf_counter around synchronize).

Roofline (``roofline``): segment-reduce forward sum on configuration C3 (E = 4,194,304 edges
sorted by destination over S = 262,144 Zipf(1.2) segments capped at 64, C = 128 fp32), kernel
time from HIP events on the launch stream, algorithmic bytes E*C*4 + S*C*4 + (S+1)*4.

CPU baseline (``cpu_baseline``): the reference's CPU path (oracle/ref_cpu_path.py, same torch op
sequences) on the same C2 batch, on this host's cores.

``legs`` holds every configuration (c1 ... c5): GPU times of each op, the fused-row kernels on
the C2 graph, every C3 segment-reduce leg, and beside each configuration a CPU baseline of the
reference's CPU path (bounded samples extrapolated where the full run would take minutes or
would not fit in memory; each entry says what was timed).

Usage: python bench.py [--steps K] [--warmup W] [--no-cpu] [--only LEG] [--iters I]
One JSON line goes to stdout; progress goes to stderr.  ``--only`` with a single-kernel leg
(fps_c2, knn_c5, c3max, ...) runs just that op, for counter collection with rocprofv3.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np
import torch

METRIC = "ms/batch FPS+radius_graph (B=16,N=4096); segment_reduce GB/s vs HBM peak"
HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of seg_fwd_merge_kernel<float,16,SUM,perm> on C3, from rocprofv3 FETCH_SIZE x 2.0 +
# WRITE_SIZE x 1.0 (factors from a plain 1 GiB elementwise pass); the run and its arithmetic are
# in profiles/seg_fwd_merge_kernel_c3_fp32.md.
C3_SUM_TRAFFIC_BYTES = 2_327_800_000


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ═══════════════════════════════════════════════════════════════════
# Synthetic configurations (deterministic, CPU generators)
# ═══════════════════════════════════════════════════════════════════


def make_c1():
    """C1: 2048 points uniform in [-1, 1]^3, FPS 512 from index 0, radius r = 0.2 / K = 32 over
    the 512 centres, C = 32 N(0, 1) features summed over that graph."""
    g = torch.Generator().manual_seed(0)
    pos = torch.rand(2048, 3, generator=g) * 2 - 1
    feat = torch.randn(512, 32, generator=g)
    return dict(pos=pos, M=512, r=0.2, K=32, feat=feat)


def make_c2(B: int = 16, N: int = 4096):
    """C2: B clouds of N points on the unit sphere + N(0, 0.01) jitter; FPS 1024 per cloud;
    radius r = 0.1, K = 32; KNN k = 16 from the centres."""
    g = torch.Generator().manual_seed(0)
    clouds = []
    for _ in range(B):
        d = torch.randn(N, 3, generator=g)
        clouds.append(d / d.norm(dim=1, keepdim=True) + 0.01 * torch.randn(N, 3, generator=g))
    pos = torch.cat(clouds)
    batch = torch.arange(B).repeat_interleave(N)
    ptr = torch.arange(B + 1, dtype=torch.int64) * N
    return dict(pos=pos, batch=batch, ptr=ptr, B=B, N=N, M=1024, r=0.1, K=32, k=16)


def make_c3_offsets(S: int = 262144, E: int = 4194304):
    """C3 segment sizes: min(zipf(1.2), 64) drawn with default_rng(0), accumulated until the sum
    reaches E (the last one truncated, the rest empty), then permuted with default_rng(1)."""
    rng = np.random.default_rng(0)
    raw = np.minimum(rng.zipf(1.2, S), 64).astype(np.int64)
    cs = np.cumsum(raw)
    cut = int(np.searchsorted(cs, E))
    sizes = raw.copy()
    sizes[cut] = E - (cs[cut - 1] if cut > 0 else 0)
    sizes[cut + 1:] = 0
    sizes = sizes[np.random.default_rng(1).permutation(S)]
    off = np.zeros(S + 1, dtype=np.int64)
    off[1:] = np.cumsum(sizes)
    assert off[-1] == E
    return off


def make_c4(B: int = 32, n: int = 2048):
    """C4: B random superquadrics (exponents U(0.3, 3), random SO(3) rotation), n samples each."""
    g = torch.Generator().manual_seed(0)

    def spow(v, e):
        return torch.sign(v) * v.abs().pow(e)

    shapes = []
    for _ in range(B):
        e1, e2 = (torch.rand(2, generator=g) * 2.7 + 0.3).tolist()
        eta = (torch.rand(n, generator=g) - 0.5) * math.pi
        om = (torch.rand(n, generator=g) * 2 - 1) * math.pi
        ce = spow(torch.cos(eta), e1)
        p = torch.stack([ce * spow(torch.cos(om), e2), ce * spow(torch.sin(om), e2),
                         spow(torch.sin(eta), e1)], dim=1)
        q = torch.randn(4, generator=g)
        w, x, y, z = (q / q.norm()).tolist()
        R = torch.tensor([[1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w)],
                          [2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w)],
                          [2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)]])
        shapes.append(p @ R.T)
    pos = torch.cat(shapes).float()
    ptr = torch.arange(B + 1, dtype=torch.int64) * n
    return dict(pos=pos, ptr=ptr, B=B, n=n, levels=(512, 128), radii=(0.2, 0.4), K=64,
                channels=(64, 128))


def make_c5():
    """C5: one 64-ring spinning-lidar frame, 131,072 points: elevations linspace(-24.8, 2) deg,
    2048 azimuths, range U(1, 80) m + N(0, 0.02), rays clipped to the ground plane z = -1.7."""
    g = torch.Generator().manual_seed(0)
    el = torch.deg2rad(torch.linspace(-24.8, 2.0, 64, dtype=torch.float64))
    az = torch.arange(2048, dtype=torch.float64) * (2 * math.pi / 2048)
    E_, A_ = torch.meshgrid(el, az, indexing="ij")
    rng = torch.rand(64, 2048, generator=g, dtype=torch.float64) * 79 + 1
    rng = rng + 0.02 * torch.randn(64, 2048, generator=g, dtype=torch.float64)
    down = E_ < 0
    t_hit = torch.where(down, 1.7 / torch.sin(-E_).clamp(min=1e-12), torch.full_like(E_, math.inf))
    rng = torch.minimum(rng, t_hit)
    pts = torch.stack([rng * torch.cos(E_) * torch.cos(A_), rng * torch.cos(E_) * torch.sin(A_),
                       rng * torch.sin(E_)], dim=-1).reshape(-1, 3).float()
    return dict(pos=pts, M=16384, r=0.5, K=64, k=8, C=32)


# ═══════════════════════════════════════════════════════════════════
# Timing helpers
# ═══════════════════════════════════════════════════════════════════


def _se3_reference_torch(conv, s, v, gr):
    """SE3Conv.forward as the reference computes it (se3_conv.py:61-235, :482-566: radial MLP
    in PyTorch ops, per-edge messages of paths 0-4 from gathered source features, concatenation,
    segment sum over the target CSR, division by the average degree, bias), on the same GPU;
    the segment sum is this library's kernel, so the comparison isolates the fusion."""
    from geoembodied.functional.segment_reduce import segment_reduce
    rb = conv.radial_basis
    d = gr.dist.unsqueeze(-1)
    basis = torch.sin(rb.freqs * d) / d.clamp(min=1e-8)
    env = (0.5 * (1.0 + torch.cos(math.pi * gr.dist / rb.cutoff))).clamp(min=0.0).unsqueeze(-1)
    R = rb.mlp(basis * env)
    s_src, v_src = s[gr.row], v[gr.row]
    y0, dr = gr.Y[:, 0:1], gr.direction
    sm = R[:, 0:1] * y0 * (s_src @ conv.w_ss.weight.t())
    vm = (R[:, 1:2] * (s_src @ conv.w_sv.weight.t())).unsqueeze(-1) * dr.unsqueeze(-2)
    mixed = (v_src.transpose(-1, -2) @ conv.w_vv_scalar.weight.t()).transpose(-1, -2)
    vm = vm + R[:, 2:3].unsqueeze(-1) * y0.unsqueeze(-1) * mixed
    dot = (dr.unsqueeze(-2) * v_src).sum(-1)
    sm = sm + R[:, 3:4] * (dot @ conv.w_vs.weight.t())
    cross = torch.linalg.cross(dr.unsqueeze(-2).expand_as(v_src), v_src, dim=-1)
    vm = vm + R[:, 4:5].unsqueeze(-1) * (cross.transpose(-1, -2) @ conv.w_vv_cross.weight.t()).transpose(-1, -2)
    msg = torch.cat([sm, vm.reshape(gr.E, -1)], dim=-1)
    out = segment_reduce(msg, gr.col_sorted, gr.perm, gr.node_start, gr.node_end, gr.N)
    out = out / gr.avg_degree.unsqueeze(1)
    return out[:, :64] + conv.scalar_bias, out[:, 64:].reshape(gr.N, 16, 3)


def _fused_rooflines(args, dev, pos, row, col, perm, ns, ne, scores, feats, idx, dist, gr, conv,
                     fs, fv) -> dict:
    """HIP-event time of single kernels of the fused rows on the C2 graph.  ``bytes`` are the
    compulsory bytes (every input element read once, however often it is gathered, every output
    written once) and ``frac`` their fraction of the 8 TB/s HBM peak; ``gathered_bytes`` counts a
    gathered row once per gather (the traffic the kernel's access pattern asks of L2, of which
    the L2 serves the repeats)."""
    from gdl_amd import _native as nat
    from gdl_amd.csrc import edge_geometry_hip
    from gdl_amd.functional.gather import gather_weighted_sum, idw_weights
    from gdl_amd.functional.segment_softmax import segment_softmax
    from gdl_amd.se3_conv import PATH_NAMES, _Plan, _pack, _pad16, _pad64, path_columns

    def entry(us, nbytes, gathered=None):
        gbs = nbytes / (us * 1e-6) / 1e9
        e = {"us": round(us, 2), "bytes": int(nbytes), "GB/s": round(gbs, 1),
             "frac": round(gbs / 8000.0, 4)}
        if gathered is not None:
            e["gathered_bytes"] = int(gathered)
            e["gathered_GB/s"] = round(gathered / (us * 1e-6) / 1e9, 1)
        return e

    out = {}
    E, N, H = row.numel(), pos.shape[0], scores.shape[1]
    # the softmax kernel (~9 us) is as short as the Python wrapper's own host time, so it is
    # launched here through the library's C entry point into a preallocated output, which the
    # host issues faster than the GPU runs it
    lib, st = nat.lib(), nat.stream_of(dev)
    w_sm = torch.empty_like(scores)
    sm_args = (nat.DTYPE_CODES[scores.dtype], nat.ptr(scores), nat.ptr(perm), nat.ptr(ns),
               nat.ptr(ne), E, N, H, 1, nat.ptr(w_sm), st)
    nat.check(lib.geo_segment_softmax_fwd(*sm_args), "geo_segment_softmax_fwd")
    if not torch.equal(w_sm, segment_softmax(scores, perm, ns, ne, N, contiguous_csr=True)):
        raise RuntimeError("segment softmax: C entry point and API call disagree")
    us = 1e3 * event_ms(lambda: lib.geo_segment_softmax_fwd(*sm_args), args.iters, 5)
    out["segment_softmax_fwd"] = entry(us, 2 * E * H * 4 + E * 4 + 2 * N * 4)
    # the gather and edge-geometry kernels (13-14 us) are shorter than their wrappers' host
    # time too: the same C-entry-point timing, each checked once against the API call
    w = idw_weights(idx, dist)
    n_out, K = idx.shape
    C = feats.shape[1]
    idx64, feats_c = idx.contiguous(), feats.contiguous()
    g_out = torch.empty(n_out, C, device=dev)
    gw_args = (nat.DTYPE_CODES[torch.float32], nat.ptr(feats_c), feats_c.shape[0], C, nat.ptr(idx64),
               nat.ptr(w), n_out, K, nat.ptr(g_out), st)
    nat.check(lib.geo_gather_weighted_sum(*gw_args), "geo_gather_weighted_sum")
    if not torch.equal(g_out, gather_weighted_sum(feats, idx, w)):
        raise RuntimeError("gather_weighted_sum: C entry point and API call disagree")
    us = 1e3 * event_ms(lambda: lib.geo_gather_weighted_sum(*gw_args), args.iters, 5)
    out["gather_weighted_sum_k3_c112"] = entry(
        us, feats.shape[0] * C * 4 + n_out * K * (8 + 4) + n_out * C * 4,
        n_out * K * (8 + 4 + C * 4) + n_out * C * 4)
    pos_c, row64, col64 = pos.contiguous(), row.contiguous(), col.contiguous()
    e_dir, e_dist, e_Y = (torch.empty(E, 3, device=dev), torch.empty(E, device=dev),
                          torch.empty(E, 9, device=dev))
    eg_args = (nat.ptr(pos_c), N, nat.ptr(row64), nat.ptr(col64), E, 2, nat.ptr(e_dir),
               nat.ptr(e_dist), nat.ptr(e_Y), st)
    nat.check(lib.geo_edge_geometry(*eg_args), "geo_edge_geometry")
    with torch.no_grad():
        ref_geom = edge_geometry_hip(pos, row, col, 2)
    if not all(torch.equal(a, b) for a, b in zip((e_dir, e_dist, e_Y), ref_geom)):
        raise RuntimeError("edge_geometry: C entry point and API call disagree")
    us = 1e3 * event_ms(lambda: lib.geo_edge_geometry(*eg_args), args.iters, 5)
    out["edge_geometry_l2"] = entry(us, N * 12 + E * (16 + 52), E * (16 + 24 + 52))
    # the SE3 forward aggregate alone (sums of r-weighted source features per target)
    Cs, Cv = fs.shape[1], fv.shape[1]
    weights = {k: getattr(conv, k).weight if getattr(conv, k) is not None else None for k in PATH_NAMES}
    pc = path_columns(weights, False, True, 0)
    with torch.no_grad():
        R = conv.radial_basis(gr.dist)
    P = R.shape[1]
    plan = _Plan(Cs, Cv, 0, conv.out_scalar_channels, conv.out_vector_channels, 0, pc, P, 9, False)
    Xs = torch.empty(N, plan.Ks, device=dev)
    Xv = torch.empty(N, 3, plan.Kv, device=dev)
    assert pc[7] < 0   # no type-2 path: the kernels take no CG table
    s_, v_ = fs.detach().contiguous(), fv.detach().contiguous()
    Y, d = gr.Y.detach().contiguous(), gr.direction.detach().contiguous()

    def agg():
        nat.check(nat.lib().geo_se3_aggregate_fwd(
            nat.ptr(s_), nat.ptr(v_), None, N, Cs, Cv, 0, nat.ptr(gr.row), None, nat.ptr(gr.node_start),
            nat.ptr(gr.node_end), E, nat.ptr(d), nat.ptr(Y), 9, nat.ptr(R), P, plan.pc_c, None,
            nat.ptr(Xs), plan.Ks, nat.ptr(Xv), plan.Kv, None, 0, nat.stream_of(dev)), "aggregate")

    us = 1e3 * event_ms(agg, args.iters, 5)
    per_edge = E * (8 + 4 * P + 12 + 4)        # source id, R row, direction, Y_0
    out["se3_fwd_aggregate_64s16v"] = entry(
        us, N * (Cs + 3 * Cv) * 4 + per_edge + 2 * N * 4 + N * (plan.Ks + 3 * plan.Kv) * 4,
        E * (Cs + 3 * Cv) * 4 + per_edge + 2 * N * 4 + N * (plan.Ks + 3 * plan.Kv) * 4)
    assert _pad16(Cs + 2 * Cv) == plan.Kv
    # the whole forward in one launch (aggregates in LDS, weights applied there): what
    # SE3Conv.forward runs when no weight gradient is wanted
    Os, Ov = plan.Os, plan.Ov
    Ws, Wv, _ = _pack(plan, [weights[k] for k in PATH_NAMES],
                      [(0, _pad64(Os), plan.Ks), (1, _pad64(Ov), plan.Kv), (2, 0, plan.Kt)], dev)
    s_out = torch.empty(N, Os, device=dev)
    v_out = torch.empty(N, Ov, 3, device=dev)
    avg = gr.avg_degree.contiguous()
    bias = conv.scalar_bias.detach().contiguous()
    assert lib.geo_se3_fwd_fused_lds_bytes(Os, Ov, 0, plan.Ks, plan.Kv, plan.Kt) > 0

    def fused():
        nat.check(lib.geo_se3_fwd_fused(
            nat.ptr(s_), nat.ptr(v_), None, N, Cs, Cv, 0, nat.ptr(gr.row), None,
            nat.ptr(gr.node_start), nat.ptr(gr.node_end), E, nat.ptr(d), nat.ptr(Y), 9, nat.ptr(R),
            P, plan.pc_c, None, nat.ptr(Ws), Ws.shape[0], nat.ptr(Wv), Wv.shape[0], None, 0, Os, Ov,
            0, plan.Ks, plan.Kv, plan.Kt, nat.ptr(avg), nat.ptr(bias), None, nat.ptr(s_out),
            nat.ptr(v_out), None, None, None, None, st), "fused forward")

    us = 1e3 * event_ms(fused, args.iters, 5)
    w_bytes = (Ws.numel() + Wv.numel()) * 4
    out["se3_fwd_fused_64s16v"] = entry(
        us, N * (Cs + 3 * Cv) * 4 + per_edge + 2 * N * 4 + N * 4 + w_bytes + N * (Os + 3 * Ov) * 4,
        E * (Cs + 3 * Cv) * 4 + per_edge + 2 * N * 4 + N * 4 + w_bytes + N * (Os + 3 * Ov) * 4)
    return out


def _se3_two_kernel_forward(conv, fs, fv, gr, dev):
    """The SE3Conv forward of a layer as the two-kernel path runs it (per-node aggregates to HBM,
    then the MFMA GEMMs; what layers too large for the fused kernel take), through the C entry
    points with the layer's weights and radial weights: for counters beside the fused forward."""
    from gdl_amd import _native as nat
    from gdl_amd.se3_conv import PATH_NAMES, _Plan, _gemm, _pack, _pad64, path_columns
    weights = {k: getattr(conv, k).weight if getattr(conv, k) is not None else None for k in PATH_NAMES}
    pc = path_columns(weights, False, True, 0)
    with torch.no_grad():
        R = conv.radial_basis(gr.dist)
    Cs, Cv, N, E = fs.shape[1], fv.shape[1], gr.N, gr.E
    plan = _Plan(Cs, Cv, 0, conv.out_scalar_channels, conv.out_vector_channels, 0, pc, R.shape[1],
                 gr.Y.shape[1], False)
    Ws, Wv, _ = _pack(plan, [weights[k] for k in PATH_NAMES],
                      [(0, _pad64(plan.Os), plan.Ks), (1, _pad64(plan.Ov), plan.Kv), (2, 0, plan.Kt)],
                      dev)
    Xs = torch.empty(N, plan.Ks, device=dev)
    Xv = torch.empty(N, 3, plan.Kv, device=dev)
    s_out = torch.empty(N, plan.Os, device=dev)
    v_out = torch.empty(N, plan.Ov, 3, device=dev)
    bias = conv.scalar_bias.detach().contiguous()

    def fn():
        nat.check(nat.lib().geo_se3_aggregate_fwd(
            nat.ptr(fs), nat.ptr(fv), None, N, Cs, Cv, 0, nat.ptr(gr.row), None,
            nat.ptr(gr.node_start), nat.ptr(gr.node_end), E, nat.ptr(gr.direction), nat.ptr(gr.Y),
            gr.Y.shape[1], nat.ptr(R), R.shape[1], plan.pc_c, None, nat.ptr(Xs), plan.Ks,
            nat.ptr(Xv), plan.Kv, None, 0, nat.stream_of(dev)), "geo_se3_aggregate_fwd")
        _gemm(Xs, N, plan.Ks, Ws, plan.Os, 1, s_out, plan.Os, gr.avg_degree, bias, None)
        _gemm(Xv, 3 * N, plan.Kv, Wv, plan.Ov, 3, v_out, 3 * plan.Ov, gr.avg_degree, None, None)
    return fn


def wall_ms(fn, steps: int, warmup: int) -> float:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1000.0 / steps


def event_ms(fn, iters: int, warmup: int) -> float:
    """Average GPU time per call between HIP events recorded on the current stream (the stream
    every op of this library launches on)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(iters):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / iters


def cpu_ms(fn, runs: int = 3) -> float:
    """Median wall time of ``runs`` calls on the host (ms)."""
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1e3)
    return sorted(ts)[len(ts) // 2]


def cpu_threads() -> dict:
    """The host's CPU counts and the threads the CPU baselines run on.  The baselines run with
    every CPU this process may use (its affinity set, at most OMP_NUM_THREADS when that is set:
    a GPU box allots a fixed CPU share to each GPU whatever os.cpu_count() reports); the counts
    are reported beside every CPU figure."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = os.cpu_count() or 1
    use = affinity
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        use = min(use, int(omp))
    return {"os_cpu_count": os.cpu_count(), "affinity": affinity, "threads": use}


def _cpu_entry(value_ms: float, unit: str, sample: str) -> dict:
    t = cpu_threads()
    return {"value": round(value_ms, 2), "unit": unit, "cores": torch.get_num_threads(),
            "os_cpu_count": t["os_cpu_count"], "kind": "port", "sample": sample}


def compulsory(nbytes: int, ms: float) -> dict:
    """Compulsory HBM bytes of one call (inputs read once, outputs written once) and the fraction
    of the 8 TB/s peak they make at the measured time."""
    return {"bytes": int(nbytes), "ms": round(ms, 4),
            "frac": round(nbytes / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 5)}


def fps_bytes(n_points: int, n_samples: int) -> int:
    """FPS: positions read once (12 B per point), int64 sample indices written."""
    return n_points * 12 + n_samples * 8


def knn_bytes(n_q: int, n_s: int, k: int, n_clouds: int) -> int:
    """KNN: queries and sources read once, both cloud offset arrays, [n_q, k] int64 indices and
    fp32 distances written."""
    return (n_q + n_s) * 12 + 2 * (n_clouds + 1) * 8 + n_q * k * 12


def radius_bytes(n_points: int, n_edges: int, batch: bool) -> int:
    """Radius graph: positions read once (and the int64 batch vector when given), int64 row and
    col written."""
    return n_points * 12 + (n_points * 8 if batch else 0) + n_edges * 16


def csr_bytes(n_edges: int, n_nodes: int) -> int:
    """CSR build: int64 targets read, int32 col_sorted and perm written, int32 node_start and
    node_end written."""
    return n_edges * 8 + n_edges * 8 + n_nodes * 8


def _ops():
    import geoembodied  # noqa: F401  (registers the drop-in module paths)
    from geoembodied.functional.fps import farthest_point_sampling
    from geoembodied.functional.knn import knn
    from geoembodied.functional.radius_graph import radius_graph
    from geoembodied.functional.segment_reduce import segment_reduce, sort_and_build_csr
    return farthest_point_sampling, knn, radius_graph, segment_reduce, sort_and_build_csr


def _pair_keys(row, col, n) -> np.ndarray:
    return np.asarray(row, dtype=np.int64) * n + np.asarray(col, dtype=np.int64)


# ═══════════════════════════════════════════════════════════════════
# Configuration legs
# ═══════════════════════════════════════════════════════════════════


def leg_c2(args, dev) -> tuple:
    """The headline step, its parts, the fused-row kernels on the C2 graph and the CPU baseline
    of the step (the reference's CPU path) with the cdist disagreement diagnostic."""
    fps, knn, radius_graph, _, sort_and_build_csr = _ops()
    c2 = make_c2()
    pos = c2["pos"].to(dev)
    batch = c2["batch"].to(dev)
    ptr = c2["ptr"].to(dev)
    leg: dict = {}

    # FPS runs one workgroup per cloud (16 of 256 CUs) and the radius graph over all points does
    # not depend on it, so the radius graph runs on a second stream (default priority) beside
    # FPS on the current stream and is joined back at the end of the step.  FPS stays on the
    # current stream: every cross-stream event adds a packet to the queue it is recorded on or
    # waited on, ~10 us each on FPS's critical path.
    s_rad = torch.cuda.Stream(device=dev)

    def step():
        main = torch.cuda.current_stream(dev)
        s_rad.wait_stream(main)
        idx = fps(pos, c2["M"], ptr=ptr)
        with torch.cuda.stream(s_rad):
            row, col = radius_graph(pos, c2["r"], max_num_neighbors=c2["K"], batch=batch,
                                    num_batch_elements=c2["B"])
        main.wait_stream(s_rad)
        for x in (row, col):
            x.record_stream(main)
        return idx, row, col

    def step_one_stream():
        idx = fps(pos, c2["M"], ptr=ptr)
        row, col = radius_graph(pos, c2["r"], max_num_neighbors=c2["K"], batch=batch,
                                num_batch_elements=c2["B"])
        return idx, row, col

    log("C2: FPS + radius_graph ...")
    ms_step = wall_ms(step, args.steps, args.warmup)
    idx, row, col = step()
    leg["step_ms"] = round(ms_step, 4)
    leg["step_one_stream_ms"] = round(wall_ms(step_one_stream, args.steps, 3), 4)
    leg["fps_ms"] = round(wall_ms(lambda: fps(pos, c2["M"], ptr=ptr), args.steps, 3), 4)
    leg["radius_ms"] = round(wall_ms(lambda: radius_graph(
        pos, c2["r"], max_num_neighbors=c2["K"], batch=batch, num_batch_elements=c2["B"]),
        args.steps, 3), 4)
    leg["edges"] = int(row.numel())
    leg["points_per_s"] = round(pos.shape[0] / (ms_step / 1e3))
    leg["edges_per_s"] = round(row.numel() / (leg["radius_ms"] / 1e3))
    leg["fps_point_updates_per_s"] = round(c2["B"] * c2["N"] * c2["M"] / (leg["fps_ms"] / 1e3))
    cent = pos[idx]
    ptr_q = torch.arange(c2["B"] + 1, device=dev, dtype=torch.int64) * c2["M"]
    leg["knn_k16_ms"] = round(wall_ms(lambda: knn(cent, pos, ptr_q, ptr, c2["k"]), args.steps, 3), 4)
    leg["radius_centres_ms"] = round(wall_ms(
        lambda: radius_graph(cent, c2["r"], max_num_neighbors=c2["K"], num_batch_elements=c2["B"]),
        args.steps, 3), 4)
    e_cent = int(radius_graph(cent, c2["r"], max_num_neighbors=c2["K"],
                              num_batch_elements=c2["B"])[0].numel())
    leg["csr_build_ms"] = round(wall_ms(lambda: sort_and_build_csr(col, pos.shape[0]),
                                        args.steps, 3), 4)
    n2, m2 = pos.shape[0], c2["B"] * c2["M"]
    leg["compulsory"] = {
        "fps": compulsory(fps_bytes(n2, m2), leg["fps_ms"]),
        "radius_all_points": compulsory(radius_bytes(n2, leg["edges"], True), leg["radius_ms"]),
        "radius_centres": compulsory(radius_bytes(m2, e_cent, False), leg["radius_centres_ms"]),
        "knn_k16": compulsory(knn_bytes(m2, n2, c2["k"], c2["B"]), leg["knn_k16_ms"]),
        "csr_build": compulsory(csr_bytes(leg["edges"], n2), leg["csr_build_ms"]),
    }
    log(f"  step {ms_step:.3f} ms (one stream {leg['step_one_stream_ms']:.3f})  fps "
        f"{leg['fps_ms']:.3f}  radius {leg['radius_ms']:.3f}  knn {leg['knn_k16_ms']:.3f}  "
        f"edges {leg['edges']}")
    # attention softmax over the C2 graph (4 heads): CSR from the radius graph's target order
    from gdl_amd.functional.segment_softmax import segment_softmax, sparse_softmax
    cs, pm, ns, ne = sort_and_build_csr(col, pos.shape[0])
    scores = torch.randn(row.numel(), 4, device=dev, generator=torch.Generator(device=dev).manual_seed(0))
    leg["softmax_fwd_us"] = round(1e3 * event_ms(
        lambda: segment_softmax(scores, pm, ns, ne, pos.shape[0], contiguous_csr=True),
        args.iters, 5), 2)
    leg["sparse_softmax_us"] = round(1e3 * wall_ms(
        lambda: sparse_softmax(scores, col, pos.shape[0]), args.steps, 3), 2)
    log(f"  segment softmax (E={row.numel()}, H=4): {leg['softmax_fwd_us']} us on the CSR, "
        f"{leg['sparse_softmax_us']} us from the target index")
    # interpolation of 112-channel features (64 scalars + 16 vectors) from the centres back to
    # every point with k = 3 IDW (the interpolation layer's shape)
    from gdl_amd.functional.gather import knn_interpolate
    ii, dd = knn(pos, cent, ptr, ptr_q, 3)
    feats = torch.randn(cent.shape[0], 112, device=dev)
    leg["interp_k3_c112_us"] = round(1e3 * event_ms(lambda: knn_interpolate(feats, ii, dd),
                                                    args.iters, 5), 2)
    log(f"  knn_interpolate (65536 x k=3 x 112 ch): {leg['interp_k3_c112_us']} us")
    # the whole spatial graph: radius graph + CSR + directions, distances, SH (l <= 2) and
    # average degrees, as one call
    from gdl_amd.graph import SpatialGraph
    leg["spatial_graph_ms"] = round(wall_ms(
        lambda: SpatialGraph.build(pos, c2["r"], max_num_neighbors=c2["K"], batch=batch,
                                   num_batch_elements=c2["B"]), args.steps, 3), 4)
    log(f"  SpatialGraph.build: {leg['spatial_graph_ms']:.3f} ms")
    # one SE3Conv layer (64 scalar + 16 vector channels in and out, paths 0-4) on the C2 graph:
    # fused message passing vs the reference's op sequence in PyTorch on the same GPU
    from gdl_amd.se3_conv import SE3Conv
    gr = SpatialGraph.build(pos, c2["r"], max_num_neighbors=c2["K"], batch=batch,
                            num_batch_elements=c2["B"])
    torch.manual_seed(0)
    conv = SE3Conv(64, 16, 64, 16, radius=c2["r"]).to(dev)
    fs = torch.randn(gr.N, 64, device=dev, requires_grad=True)
    fv = torch.randn(gr.N, 16, 3, device=dev, requires_grad=True)

    def se3_fwd():
        with torch.no_grad():
            return conv(fs, fv, gr)

    # a training step's backward: gradients start empty (zero_grad(set_to_none=True)), so no
    # accumulation adds enter either side's timing
    def clear_grads():
        conv.zero_grad(set_to_none=True)
        fs.grad = None
        fv.grad = None

    def se3_fb():
        clear_grads()
        so, vo = conv(fs, fv, gr)
        torch.autograd.backward((so, vo), (torch.ones_like(so), torch.ones_like(vo)))

    def ref_fwd():
        with torch.no_grad():
            return _se3_reference_torch(conv, fs, fv, gr)

    def ref_fb():
        clear_grads()
        so, vo = _se3_reference_torch(conv, fs, fv, gr)
        torch.autograd.backward((so, vo), (torch.ones_like(so), torch.ones_like(vo)))

    leg["se3conv_fwd_ms"] = round(wall_ms(se3_fwd, args.steps, 3), 4)
    leg["se3conv_fwd_bwd_ms"] = round(wall_ms(se3_fb, args.steps, 3), 4)
    leg["se3conv_torch_ref_fwd_ms"] = round(wall_ms(ref_fwd, args.steps, 3), 4)
    leg["se3conv_torch_ref_fwd_bwd_ms"] = round(wall_ms(ref_fb, args.steps, 3), 4)
    log(f"  SE3Conv 64s+16v (E={gr.E}): fused {leg['se3conv_fwd_ms']:.3f} ms fwd, "
        f"{leg['se3conv_fwd_bwd_ms']:.3f} ms fwd+bwd; reference op sequence in PyTorch "
        f"{leg['se3conv_torch_ref_fwd_ms']:.3f} / {leg['se3conv_torch_ref_fwd_bwd_ms']:.3f} ms")
    leg["fused_rooflines"] = _fused_rooflines(args, dev, pos, row, col, pm, ns, ne, scores, feats,
                                              ii, dd, gr, conv, fs, fv)
    for name, r in leg["fused_rooflines"].items():
        log(f"  {name}: {r['us']} us, {r['GB/s']} GB/s = {100 * r['frac']:.1f}% of 8 TB/s "
            f"({r['bytes']} algorithmic bytes)")

    cpu = None
    if not args.no_cpu:
        from oracle import ref_cpu_path
        threads = torch.get_num_threads()
        log(f"C2 CPU baseline (reference CPU path, {threads} threads) ...")
        pc, ptrc = c2["pos"], c2["ptr"]
        kc = torch.full((c2["B"],), c2["M"], dtype=torch.int64)
        runs = []
        for _ in range(3):
            t0 = time.perf_counter()
            ref_cpu_path.fps(pc, ptrc, kc)
            t1 = time.perf_counter()
            rr, rc = ref_cpu_path.radius_graph(pc, c2["r"], c2["B"], c2["K"])
            t2 = time.perf_counter()
            runs.append((t2 - t0, t1 - t0, t2 - t1))
        tot, t_fps, t_rad = sorted(runs)[1]
        cpu = {"value": round(tot * 1e3, 1), "unit": "ms/batch", "cores": threads,
               "os_cpu_count": os.cpu_count(), "kind": "port",
               "sample": f"reference CPU path (iterative FPS + batched cdist/topk radius graph, "
                         f"oracle/ref_cpu_path.py) on the full C2 batch, median of 3; fps "
                         f"{t_fps:.2f} s, radius {t_rad:.2f} s",
               "cpu_model": _cpu_model()}
        log(f"  CPU: {tot * 1e3:.0f} ms/batch")
        # the survey's D3 diagnostic on the real batch: edges of the exact semantics (this GPU
        # output) that the reference's cdist path does not produce, and the reverse
        n = pos.shape[0]
        mine = _pair_keys(row.cpu().numpy(), col.cpu().numpy(), n)
        theirs = _pair_keys(rr.numpy(), rc.numpy(), n)
        diff = np.setxor1d(mine, theirs)
        p64 = c2["pos"].double().numpy()
        r2 = float(np.float32(c2["r"] * c2["r"]))
        rel = [abs(((p64[k // n] - p64[k % n]) ** 2).sum() - r2) / r2 for k in diff.tolist()]
        leg["cdist_disagreement"] = {"directed_edges": int(diff.size),
                                     "max_rel_dist_from_r2": float(max(rel)) if rel else 0.0}
        log(f"  cdist-path disagreement: {diff.size} directed edges of {row.numel()}")
    return ms_step, leg, cpu


def leg_c3(args, dev) -> tuple:
    """Segment reduce on C3: the roofline kernel (fp32 sum) and every other leg, the CSR build,
    and the CPU baseline of the reference's loop."""
    _, _, _, segment_reduce, sort_and_build_csr = _ops()
    from gdl_amd.csrc import segment_reduce_backward_hip, segment_reduce_forward_hip
    log("C3: segment reduce ...")
    off = make_c3_offsets()
    S, E, C = off.shape[0] - 1, int(off[-1]), 128
    ns = torch.from_numpy(off[:-1].astype(np.int32)).to(dev)
    ne = torch.from_numpy(off[1:].astype(np.int32)).to(dev)
    col_sorted = torch.repeat_interleave(torch.arange(S, device=dev, dtype=torch.int32),
                                         (ne - ns).long())
    perm = torch.arange(E, device=dev, dtype=torch.int32)
    gen = torch.Generator(device=dev).manual_seed(0)
    msg = torch.randn(E, C, device=dev, generator=gen)
    bytes_fwd = E * C * 4 + S * C * 4 + (S + 1) * 4
    iters = args.iters
    # Warm-up of each timed C3 kernel: ~20 ms of launches.  The C2 CPU baseline before this leg
    # leaves the GPU idle for seconds, and with 5 warm-up launches the first timed launches of a
    # 0.4 ms kernel still run at a lower clock (0.415 against 0.397 ms per launch in steady state).
    wu = 50
    leg: dict = {}
    roof = None
    if args.only in (None, "c3"):
        ms = event_ms(lambda: segment_reduce(msg, col_sorted, perm, ns, ne, S), iters, wu)
        gbs = bytes_fwd / (ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": C3_SUM_TRAFFIC_BYTES,
                "kernel": "seg_fwd_merge_kernel<float,16,SUM,perm>", "ms_per_launch": round(ms, 4),
                "algorithmic_bytes": bytes_fwd}
        leg["sum_fp32_ms"] = round(ms, 4)
        log(f"  fwd sum fp32: {ms:.4f} ms  {gbs:.0f} GB/s  ({gbs / HBM_PEAK_GBS:.1%} of peak)")
        for red in ("mean", "max"):
            extra = S * C * 4 if red == "max" else 0
            msr = event_ms(lambda: segment_reduce(msg, col_sorted, perm, ns, ne, S, reduce=red),
                           iters, wu)
            leg[f"{red}_fp32_ms"] = round(msr, 4)
            leg[f"{red}_fp32_gbs"] = round((bytes_fwd + extra) / (msr * 1e-3) / 1e9, 1)
            log(f"  fwd {red} fp32: {msr:.4f} ms  {leg[f'{red}_fp32_gbs']} GB/s")
    if args.only in (None, "c3bf16"):
        mb = msg.bfloat16()
        bytes_b = E * C * 2 + S * C * 2 + (S + 1) * 4
        msb = event_ms(lambda: segment_reduce(mb, col_sorted, perm, ns, ne, S), iters, wu)
        leg["sum_bf16_ms"] = round(msb, 4)
        leg["sum_bf16_gbs"] = round(bytes_b / (msb * 1e-3) / 1e9, 1)
        log(f"  fwd sum bf16: {msb:.4f} ms  {leg['sum_bf16_gbs']} GB/s")
        del mb
    if args.only in (None, "c3bwd"):
        grad = torch.randn(S, C, device=dev, generator=gen)
        bytes_bwd = S * C * 4 + E * C * 4 + (S + 1) * 4
        for red in ("sum", "mean"):
            msb = event_ms(lambda: segment_reduce_backward_hip(grad, col_sorted, perm, ns, ne, E, red),
                           iters, wu)
            leg[f"bwd_{red}_fp32_gbs"] = round(bytes_bwd / (msb * 1e-3) / 1e9, 1)
            log(f"  bwd {red} fp32: {msb:.4f} ms  {leg[f'bwd_{red}_fp32_gbs']} GB/s")
        out, arg = segment_reduce_forward_hip(msg, perm, ns, ne, S, "max")
        msb = event_ms(lambda: segment_reduce_backward_hip(grad, col_sorted, perm, ns, ne, E, "max",
                                                           msg=msg, out=out, arg=arg), iters, wu)
        leg["bwd_max_fp32_gbs"] = round((bytes_bwd + S * C * 4) / (msb * 1e-3) / 1e9, 1)
        log(f"  bwd max fp32: {msb:.4f} ms  {leg['bwd_max_fp32_gbs']} GB/s")
        del out, arg, grad
    col64 = col_sorted.long()
    leg["csr_build_ms"] = round(wall_ms(lambda: sort_and_build_csr(col64, S), 10, 2), 4)
    # the same targets in random order (the sorted-input identity path does not apply)
    col_sh = col64[torch.randperm(E, device=dev, generator=gen)]
    leg["csr_build_shuffled_ms"] = round(wall_ms(lambda: sort_and_build_csr(col_sh, S), 10, 2), 4)
    leg["compulsory"] = {"csr_build_sorted": compulsory(csr_bytes(E, S), leg["csr_build_ms"]),
                         "csr_build_shuffled": compulsory(csr_bytes(E, S),
                                                          leg["csr_build_shuffled_ms"])}
    log(f"  CSR build: {leg['csr_build_ms']} ms sorted, {leg['csr_build_shuffled_ms']} ms shuffled")
    del col_sh, msg
    if not args.no_cpu and args.only is None:
        from oracle import ref_cpu_path
        # the reference's CPU path: argsort + bincount CSR of all E targets, then its Python loop
        # over segments (two .item() per segment) on a sample of 32,768 of the 262,144 segments
        # (rows for those segments only), extrapolated linearly to S
        sample = 32768
        col_cpu = col64.cpu()
        t_csr = cpu_ms(lambda: ref_cpu_path.sort_and_build_csr(col_cpu, S), 1)
        rows = int(off[sample])
        msg_cpu = torch.randn(rows, C, generator=torch.Generator().manual_seed(0))
        perm_cpu = torch.arange(rows, dtype=torch.int32)
        t_loop = cpu_ms(lambda: ref_cpu_path.segment_sum(
            msg_cpu, perm_cpu, torch.from_numpy(off[:sample].astype(np.int32)),
            torch.from_numpy(off[1:sample + 1].astype(np.int32)), sample), 1)
        total = t_csr + t_loop * S / sample
        leg["cpu"] = _cpu_entry(total, "ms/call", (
            f"reference CPU path: sort_and_build_csr (argsort + bincount) of all {E} targets "
            f"{t_csr:.0f} ms + the per-segment loop of segment_reduce on {sample} of {S} segments "
            f"({rows} rows) {t_loop:.0f} ms, extrapolated x{S / sample:.0f}"))
        log(f"  CPU: {total:.0f} ms (extrapolated)")
    return roof, leg


def leg_c1(args, dev) -> dict:
    """C1: FPS 2048 -> 512, radius graph over the centres, CSR, segment sum of C = 32 features
    gathered along the edges."""
    fps, _, radius_graph, segment_reduce, sort_and_build_csr = _ops()
    c1 = make_c1()
    p1 = c1["pos"].to(dev)
    f1 = c1["feat"].to(dev)

    def c1_step():
        i = fps(p1, c1["M"])
        cen = p1[i]
        row, col = radius_graph(cen, c1["r"], max_num_neighbors=c1["K"])
        cs, pm, a, b = sort_and_build_csr(col, c1["M"])
        return segment_reduce(f1[row], cs, pm, a, b, c1["M"])

    leg = {"step_ms": round(wall_ms(c1_step, 20, 3), 4)}
    leg["fps_ms"] = round(wall_ms(lambda: fps(p1, c1["M"]), 20, 3), 4)
    leg["compulsory"] = {"fps": compulsory(fps_bytes(2048, c1["M"]), leg["fps_ms"])}
    log(f"C1: step {leg['step_ms']} ms (fps {leg['fps_ms']} ms)")
    if not args.no_cpu:
        from oracle import ref_cpu_path
        pc, fc = c1["pos"], c1["feat"]

        def cpu_step():
            i = ref_cpu_path.fps(pc, torch.tensor([0, 2048]), torch.tensor([c1["M"]]))
            row, col = ref_cpu_path.radius_graph(pc[i], c1["r"], 1, c1["K"])
            cs, pm, a, b = ref_cpu_path.sort_and_build_csr(col, c1["M"])
            return ref_cpu_path.segment_sum(fc[row], pm, a, b, c1["M"])

        leg["cpu"] = _cpu_entry(cpu_ms(cpu_step, 3), "ms/step",
                                "reference CPU path (iterative FPS, cdist radius graph, argsort "
                                "CSR, per-segment loop) on the full C1 step, median of 3")
        log(f"  CPU: {leg['cpu']['value']} ms")
    return leg


def leg_c4(args, dev) -> dict:
    """C4: 32 superquadrics, FPS 2048 -> 512 -> 128, radius graphs r = 0.2 / 0.4 (K = 64), and
    max + mean pooling of N(0, 1) features (C = 64 / 128) gathered along the edges."""
    fps, _, radius_graph, segment_reduce, sort_and_build_csr = _ops()
    c4 = make_c4()
    p4, ptr4 = c4["pos"].to(dev), c4["ptr"].to(dev)
    B = c4["B"]
    g = torch.Generator(device=dev).manual_seed(4)
    f1 = torch.randn(B * 512, 64, device=dev, generator=g)
    f2 = torch.randn(B * 128, 128, device=dev, generator=g)
    ptr1 = torch.arange(B + 1, device=dev, dtype=torch.int64) * 512

    def c4_step():
        i1 = fps(p4, 512, ptr=ptr4)
        q1 = p4[i1]
        i2 = fps(q1, 128, ptr=ptr1)
        q2 = q1[i2]
        outs = []
        for pts, r, f in ((q1, 0.2, f1), (q2, 0.4, f2)):
            row, col = radius_graph(pts, r, max_num_neighbors=64, num_batch_elements=B)
            cs, pm, a, b = sort_and_build_csr(col, pts.shape[0])
            msg = f[row]
            outs.append(segment_reduce(msg, cs, pm, a, b, pts.shape[0], reduce="max"))
            outs.append(segment_reduce(msg, cs, pm, a, b, pts.shape[0], reduce="mean"))
        return outs

    leg = {"step_ms": round(wall_ms(c4_step, 10, 2), 4)}
    log(f"C4: step {leg['step_ms']} ms")
    if not args.no_cpu:
        from oracle import ref_cpu_path
        pc, ptrc = c4["pos"], c4["ptr"]
        f1c, f2c = f1.cpu(), f2.cpu()

        def cpu_step():
            i1 = ref_cpu_path.fps(pc, ptrc, torch.full((B,), 512))
            q1 = pc[i1]
            i2 = ref_cpu_path.fps(q1, torch.arange(B + 1) * 512, torch.full((B,), 128))
            q2 = q1[i2]
            for pts, r, f in ((q1, 0.2, f1c), (q2, 0.4, f2c)):
                row, col = ref_cpu_path.radius_graph(pts, r, B, 64)
                msg = f[row]
                ref_cpu_path.segment_max(msg, col, pts.shape[0])
                ref_cpu_path.segment_mean(msg, col, pts.shape[0])

        leg["cpu"] = _cpu_entry(cpu_ms(cpu_step, 3), "ms/step",
                                "reference CPU path (iterative FPS at both levels, batched cdist "
                                "radius graphs, scatter max / mean pooling) on the full C4 step, "
                                "median of 3")
        log(f"  CPU: {leg['cpu']['value']} ms")
    return leg


def leg_c5(args, dev) -> dict:
    """C5: one 131,072-point lidar frame: FPS to 16,384, radius graph r = 0.5 (K = 64) over the
    centres (empty: the centres lie about a metre apart) and over all points (5.3 M edges),
    KNN k = 8 from the centres, segment sum of C = 32 features over the all-points graph."""
    fps, knn, radius_graph, segment_reduce, sort_and_build_csr = _ops()
    c5 = make_c5()
    p5 = c5["pos"].to(dev)
    N, M = p5.shape[0], c5["M"]
    leg = {"fps_ms": round(wall_ms(lambda: fps(p5, M), 3, 1), 3)}
    i5 = fps(p5, M)
    cen5 = p5[i5]
    leg["radius_centres_ms"] = round(wall_ms(
        lambda: radius_graph(cen5, c5["r"], max_num_neighbors=c5["K"]), 10, 2), 4)
    leg["radius_all_points_ms"] = round(wall_ms(
        lambda: radius_graph(p5, c5["r"], max_num_neighbors=c5["K"]), 10, 2), 4)
    row, col = radius_graph(p5, c5["r"], max_num_neighbors=c5["K"])
    leg["edges_all_points"] = int(row.numel())
    pq = torch.tensor([0, M], device=dev, dtype=torch.int64)
    ps = torch.tensor([0, N], device=dev, dtype=torch.int64)
    leg["knn_k8_ms"] = round(wall_ms(lambda: knn(cen5, p5, pq, ps, c5["k"]), 10, 2), 4)
    cs, pm, a, b = sort_and_build_csr(col, N)
    feat = torch.randn(N, c5["C"], device=dev, generator=torch.Generator(device=dev).manual_seed(5))
    msg = feat[row]
    E = msg.shape[0]
    ms = event_ms(lambda: segment_reduce(msg, cs, pm, a, b, N), args.iters, 3)
    leg["segsum_all_points_ms"] = round(ms, 4)
    leg["segsum_all_points_gbs"] = round((E * c5["C"] * 4 + N * c5["C"] * 4 + (N + 1) * 4 + E * 4)
                                         / (ms * 1e-3) / 1e9, 1)
    leg["frame_ms"] = round(leg["fps_ms"] + leg["radius_all_points_ms"] + leg["knn_k8_ms"] + ms, 3)
    leg["csr_build_ms"] = round(wall_ms(lambda: sort_and_build_csr(col, N), 10, 2), 4)
    leg["compulsory"] = {
        "fps": compulsory(fps_bytes(N, M), leg["fps_ms"]),
        "radius_all_points": compulsory(radius_bytes(N, E, False), leg["radius_all_points_ms"]),
        "knn_k8": compulsory(knn_bytes(M, N, c5["k"], 1), leg["knn_k8_ms"]),
        "csr_build": compulsory(csr_bytes(E, N), leg["csr_build_ms"]),
    }
    log(f"C5: fps {leg['fps_ms']} ms, radius centres {leg['radius_centres_ms']} ms, all points "
        f"{leg['radius_all_points_ms']} ms ({E} edges), knn {leg['knn_k8_ms']} ms, segment sum "
        f"{ms:.4f} ms ({leg['segsum_all_points_gbs']} GB/s)")
    del msg
    if not args.no_cpu:
        from oracle import ref_cpu_path
        pc = c5["pos"]
        # FPS: the reference's Python loop for the first 512 of 16,384 steps (each step costs the
        # same: one pass over all 131,072 points), extrapolated x32; KNN: the brute force over
        # 256 of the 16,384 queries ([256, 131072, 3] difference tensor; the full one would be
        # 25.8 GB), extrapolated x64; the all-points radius graph: the cdist rows of 2,048 of
        # the 131,072 targets ([2048, 131072] distances; the full [N, N] matrix would be 68.7
        # GB), extrapolated x64
        steps = 512
        t_fps = cpu_ms(lambda: ref_cpu_path.fps(pc, torch.tensor([0, N]), torch.tensor([M]),
                                                max_steps=steps), 1)
        cen_c = cen5.cpu()
        nq = 256
        t_knn = cpu_ms(lambda: ref_cpu_path.knn(cen_c[:nq], pc, torch.tensor([0, nq]),
                                                torch.tensor([0, N]), c5["k"]), 1)
        nt = 2048
        r2 = c5["r"] * c5["r"]

        def radius_rows():
            d2 = torch.cdist(pc[:nt], pc).pow(2)
            d2.masked_fill_(d2 >= r2, float("inf"))
            vals, src = d2.topk(c5["K"], dim=1, largest=False)
            return src[vals < float("inf")]

        t_rad = cpu_ms(radius_rows, 1)
        total = t_fps * M / steps + t_knn * M / nq + t_rad * N / nt
        leg["cpu"] = _cpu_entry(total, "ms/frame", (
            f"reference CPU path, extrapolated from samples: FPS loop {steps} of {M} steps "
            f"{t_fps:.0f} ms (x{M // steps}), brute-force KNN {nq} of {M} queries {t_knn:.0f} ms "
            f"(x{M // nq}), cdist radius rows of {nt} of {N} targets {t_rad:.0f} ms (x{N // nt})"))
        log(f"  CPU: {total:.0f} ms/frame (extrapolated)")
    return leg


# ═══════════════════════════════════════════════════════════════════
# Single-kernel legs for counter collection (rocprofv3 --pmc)
# ═══════════════════════════════════════════════════════════════════

PROFILE_LEGS = ("fps_c2", "fps_c5", "knn_c2", "knn_c5", "radius_c2", "radius_c5_all", "c3sum",
                "c3max", "c3sum_bf16", "softmax_c2", "se3_fwd_c2", "se3_unfused_c2", "se3_train_c2",
                "radial_c2", "gather_c2",
                "csr_c3_sorted", "csr_c3_shuffled", "csr_c2", "sparse_softmax_c2")


def profile_leg(name: str, args, dev) -> dict:
    """Runs one op of one configuration ``args.iters`` times after one warm-up call, so that a
    counter run (rocprofv3 --pmc) sees a few dispatches of that kernel and little else."""
    fps, knn, radius_graph, segment_reduce, sort_and_build_csr = _ops()
    if name.endswith("c2"):
        c2 = make_c2()
        pos, ptr, batch = c2["pos"].to(dev), c2["ptr"].to(dev), c2["batch"].to(dev)
    if name == "fps_c2":
        fn = lambda: fps(pos, c2["M"], ptr=ptr)  # noqa: E731
    elif name == "radius_c2":
        fn = lambda: radius_graph(pos, c2["r"], max_num_neighbors=c2["K"], batch=batch,  # noqa: E731
                                  num_batch_elements=c2["B"])
    elif name == "knn_c2":
        cent = pos[fps(pos, c2["M"], ptr=ptr)]
        ptr_q = torch.arange(c2["B"] + 1, device=dev, dtype=torch.int64) * c2["M"]
        fn = lambda: knn(cent, pos, ptr_q, ptr, c2["k"])  # noqa: E731
    elif name in ("fps_c5", "knn_c5", "radius_c5_all"):
        c5 = make_c5()
        p5 = c5["pos"].to(dev)
        if name == "fps_c5":
            fn = lambda: fps(p5, c5["M"])  # noqa: E731
        elif name == "radius_c5_all":
            fn = lambda: radius_graph(p5, c5["r"], max_num_neighbors=c5["K"])  # noqa: E731
        else:
            cen = p5[fps(p5, c5["M"])]
            pq = torch.tensor([0, c5["M"]], device=dev)
            ps = torch.tensor([0, p5.shape[0]], device=dev)
            fn = lambda: knn(cen, p5, pq, ps, c5["k"])  # noqa: E731
    elif name in ("c3sum", "c3max", "c3sum_bf16"):
        off = make_c3_offsets()
        S, E, C = off.shape[0] - 1, int(off[-1]), 128
        ns = torch.from_numpy(off[:-1].astype(np.int32)).to(dev)
        ne = torch.from_numpy(off[1:].astype(np.int32)).to(dev)
        cs = torch.repeat_interleave(torch.arange(S, device=dev, dtype=torch.int32), (ne - ns).long())
        perm = torch.arange(E, device=dev, dtype=torch.int32)
        msg = torch.randn(E, C, device=dev, generator=torch.Generator(device=dev).manual_seed(0))
        if name == "c3sum":
            fn = lambda: segment_reduce(msg, cs, perm, ns, ne, S)  # noqa: E731
        elif name == "c3max":
            fn = lambda: segment_reduce(msg, cs, perm, ns, ne, S, reduce="max")  # noqa: E731
        else:
            mb = msg.bfloat16()
            del msg
            fn = lambda: segment_reduce(mb, cs, perm, ns, ne, S)  # noqa: E731
    elif name in ("csr_c3_sorted", "csr_c3_shuffled"):
        off = make_c3_offsets()
        S = off.shape[0] - 1
        col = torch.repeat_interleave(torch.arange(S, device=dev),
                                      torch.from_numpy(np.diff(off)).to(dev))
        if name == "csr_c3_shuffled":
            gen = torch.Generator(device=dev).manual_seed(0)
            col = col[torch.randperm(col.numel(), device=dev, generator=gen)]
        fn = lambda: sort_and_build_csr(col, S)  # noqa: E731
    elif name == "csr_c2":  # the radius graph's targets, already in order
        row, col = radius_graph(pos, c2["r"], max_num_neighbors=c2["K"], batch=batch,
                                num_batch_elements=c2["B"])
        fn = lambda: sort_and_build_csr(col, pos.shape[0])  # noqa: E731
    elif name == "sparse_softmax_c2":
        from gdl_amd.functional.segment_softmax import sparse_softmax
        row, col = radius_graph(pos, c2["r"], max_num_neighbors=c2["K"], batch=batch,
                                num_batch_elements=c2["B"])
        scores = torch.randn(col.numel(), 4, device=dev)
        fn = lambda: sparse_softmax(scores, col, pos.shape[0])  # noqa: E731
    elif name in ("softmax_c2", "se3_fwd_c2", "se3_unfused_c2", "se3_train_c2", "radial_c2",
                  "gather_c2"):
        from gdl_amd.graph import SpatialGraph
        gr = SpatialGraph.build(pos, c2["r"], max_num_neighbors=c2["K"], batch=batch,
                                num_batch_elements=c2["B"])
        if name == "softmax_c2":
            from gdl_amd.functional.segment_softmax import segment_softmax
            scores = torch.randn(gr.E, 4, device=dev)
            fn = lambda: segment_softmax(scores, None, gr.node_start, gr.node_end, gr.N,  # noqa: E731
                                         contiguous_csr=True)
        elif name == "gather_c2":
            from gdl_amd.functional.gather import knn_interpolate
            cent = pos[fps(pos, c2["M"], ptr=ptr)]
            ptr_q = torch.arange(c2["B"] + 1, device=dev, dtype=torch.int64) * c2["M"]
            ii, dd = knn(pos, cent, ptr, ptr_q, 3)
            feats = torch.randn(cent.shape[0], 112, device=dev)
            fn = lambda: knn_interpolate(feats, ii, dd)  # noqa: E731
        else:
            from gdl_amd.se3_conv import SE3Conv
            torch.manual_seed(0)
            conv = SE3Conv(64, 16, 64, 16, radius=c2["r"]).to(dev)
            fs = torch.randn(gr.N, 64, device=dev)
            fv = torch.randn(gr.N, 16, 3, device=dev)
            if name == "radial_c2":
                fn = lambda: conv.radial_basis(gr.dist)  # noqa: E731
            elif name == "se3_unfused_c2":
                fn = _se3_two_kernel_forward(conv, fs, fv, gr, dev)
            elif name == "se3_train_c2":  # forward + backward, gradients cleared as in the c2 leg
                fs.requires_grad_(True)
                fv.requires_grad_(True)

                def fn():
                    conv.zero_grad(set_to_none=True)
                    fs.grad = None
                    fv.grad = None
                    so, vo = conv(fs, fv, gr)
                    torch.autograd.backward((so, vo), (torch.ones_like(so), torch.ones_like(vo)))
            else:
                def fn():
                    with torch.no_grad():
                        return conv(fs, fv, gr)
    else:
        raise SystemExit(f"unknown leg {name!r}; profile legs: {', '.join(PROFILE_LEGS)}")
    fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.iters):
        fn()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.iters
    log(f"{name}: {ms:.4f} ms per call over {args.iters} calls")
    return {"leg": name, "ms_per_call": round(ms, 4), "calls": args.iters}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--only", default=None,
                    help="run one leg: c2 | c3 | c3bf16 | c3bwd | copy (HBM counter calibration) "
                         f"| one of the single-kernel profiling legs: {', '.join(PROFILE_LEGS)}")
    ap.add_argument("--iters", type=int, default=50, help="timed launches per kernel leg")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        log("bench.py measures one GPU: this build has no multi-GPU path (each op's work is a "
            "single-GPU kernel; see DESIGN.md for how it would shard). Run with --gpus 1.")
        return 2
    if not torch.cuda.is_available():
        log("bench.py needs a GPU")
        return 2

    from gdl_amd import _native

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.only in PROFILE_LEGS:
        print(json.dumps(profile_leg(args.only, args, dev)), flush=True)
        return 0
    if args.only == "copy":
        # A plain elementwise pass over 1 GiB (read 1 GiB, write 1 GiB with 16-byte vector
        # accesses): the reference point that scales rocprofv3's FETCH_SIZE / WRITE_SIZE.
        src = torch.empty(256 * 1024 * 1024, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        ms = event_ms(lambda: torch.add(src, 1.0, out=dst), args.iters, 3)
        gbs = 2 * src.numel() * 4 / (ms * 1e-3) / 1e9
        log(f"  copy 1 GiB: {ms:.4f} ms  {gbs:.1f} GB/s")
        print(json.dumps({"leg": "copy", "ms": round(ms, 4), "gbs": round(gbs, 1)}), flush=True)
        return 0

    if not args.no_cpu:
        torch.set_num_threads(cpu_threads()["threads"])
    legs: dict = {}
    ms_step = cpu = roof = None
    if args.only in (None, "c2"):
        ms_step, legs["c2"], cpu = leg_c2(args, dev)
    if args.only in (None, "c3", "c3bf16", "c3bwd"):
        roof, legs["c3"] = leg_c3(args, dev)
    if args.only is None:
        legs["c1"] = leg_c1(args, dev)
        legs["c4"] = leg_c4(args, dev)
        legs["c5"] = leg_c5(args, dev)

    result = {
        "metric": METRIC,
        "value": round(ms_step, 4) if ms_step is not None else None,
        "unit": "ms/batch",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4) if ms_step is not None else None,
        "c2_step_sequential_ms": legs.get("c2", {}).get("step_one_stream_ms"),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded generators of the five BASELINE configs, see bench.py)",
        "config": {
            "workload": "C2: FPS 4096->1024 per cloud + radius_graph(r=0.1, K=32) over 16x4096 "
                        "unit-sphere points (step); roofline leg: C3 segment_reduce sum fp32, "
                        "E=4194304, S=262144, C=128",
            "global_batch": 16, "points_per_cloud": 4096, "fps_samples": 1024,
            "radius": 0.1, "max_num_neighbors": 32, "parallelism": "single GPU",
        },
        "roofline": roof,
        "cpu_baseline": cpu,
        "legs": legs,
        "host_cpu": {**cpu_threads(), "torch_threads": torch.get_num_threads(),
                     "model": _cpu_model()},
        "library": _native.build_info(),
        "device": torch.cuda.get_device_name(dev),
    }
    if ms_step is not None:
        log(f"headline: {ms_step:.4f} ms/batch (two streams), "
            f"{result['c2_step_sequential_ms']} ms/batch sequential on one stream")
    print(json.dumps(result), flush=True)
    return 0


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    sys.exit(main())
