"""GPU test of geo_csr_build_noalloc, the CSR build that allocates nothing (its radix scratch is a
fixed device array of the library): called through the C ABI, its four int32 arrays must equal
geo_csr_build's bit for bit, on consecutive calls that share the scratch (the second smaller than
the first, then one sorted input that takes the identity path), when captured in a HIP graph and
replayed on new inputs, and without taking device memory."""


import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

MAX_EDGES = 1 << 20


def _csr_ws(nat, col, N):
    """The existing entry point, with a caller workspace."""
    L = nat.lib()
    dev = col.device
    E = col.numel()
    outs = [torch.empty(E, dtype=torch.int32, device=dev) for _ in range(2)] + \
           [torch.empty(N, dtype=torch.int32, device=dev) for _ in range(2)]
    ws_bytes = L.geo_csr_workspace_bytes(E, N)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    nat.check(L.geo_csr_build(col.data_ptr(), E, N, *[o.data_ptr() for o in outs], ws.data_ptr(),
                              ws_bytes, nat.stream_of(dev)), "geo_csr_build")
    return outs


def _csr_noalloc(nat, col, N):
    L = nat.lib()
    dev = col.device
    E = col.numel()
    outs = [torch.full((E,), -7, dtype=torch.int32, device=dev) for _ in range(2)] + \
           [torch.full((N,), -7, dtype=torch.int32, device=dev) for _ in range(2)]
    nat.check(L.geo_csr_build_noalloc(col.data_ptr(), E, N, *[o.data_ptr() for o in outs],
                                      nat.stream_of(dev)), "geo_csr_build_noalloc")
    return outs


def _targets(E, N, seed, sort=False):
    g = torch.Generator().manual_seed(seed)
    col = torch.randint(0, N, (E,), generator=g)
    col[::97] = -2              # outside [0, N): sorted after every valid target
    col[3::89] = N + 5
    if sort:
        col = col.clamp(0, N).sort().values
    return col


def test_noalloc_matches_workspace_entry(dev):
    from gdl_amd import _native as nat
    import oracle
    cases = [(MAX_EDGES, 300_000, 1, False),   # the largest input: two radix passes
             (70_000, 1_000, 2, False),         # smaller, one pass, on the same scratch
             (200_000, 50_000, 3, True),        # sorted targets: identity path
             (MAX_EDGES, 1 << 30, 4, False)]    # 31-bit keys: three passes, the most scratch
    for E, N, seed, srt in cases:
        print(f"[noalloc] E={E} N={N} seed={seed} sorted={srt}", flush=True)
        col = _targets(E, N, seed, srt).to(dev)
        want = _csr_ws(nat, col, N)
        got = _csr_noalloc(nat, col, N)
        torch.cuda.synchronize()
        for g_, w_, name in zip(got, want, ("col_sorted", "perm", "node_start", "node_end")):
            assert torch.equal(g_, w_), (name, E, N)
        # and both equal the oracle's stable CSR (numpy's stable argsort: a second at 2^20)
        ref = oracle.sort_and_build_csr(col.cpu().numpy(), N)
        for g_, r_ in zip(got, ref):
            np.testing.assert_array_equal(g_.cpu().numpy(), r_)


def test_noalloc_rejects_oversize(dev):
    from gdl_amd import _native as nat
    L = nat.lib()
    col = torch.zeros(MAX_EDGES + 1, dtype=torch.int64, device=dev)
    out = torch.empty(MAX_EDGES + 1, dtype=torch.int32, device=dev)
    ns = torch.empty(4, dtype=torch.int32, device=dev)
    rc = L.geo_csr_build_noalloc(col.data_ptr(), MAX_EDGES + 1, 4, out.data_ptr(), out.data_ptr(),
                                 ns.data_ptr(), ns.data_ptr(), nat.stream_of(dev))
    assert rc == 1 and "exceed" in nat.last_error()
    # empty input: node ranges all zero, nothing else touched
    e = torch.empty(0, dtype=torch.int64, device=dev)
    ns = torch.full((5,), 9, dtype=torch.int32, device=dev)
    ne = torch.full((5,), 9, dtype=torch.int32, device=dev)
    nat.check(L.geo_csr_build_noalloc(e.data_ptr(), 0, 5, None, None, ns.data_ptr(), ne.data_ptr(),
                                      nat.stream_of(dev)), "geo_csr_build_noalloc")
    assert ns.tolist() == [0] * 5 and ne.tolist() == [0] * 5


def test_noalloc_graph_replay_and_no_memory(dev):
    """Captured once in a HIP graph, replays on refilled inputs give geo_csr_build's arrays (eager
    work and synchronisations between the replays); repeated calls leave the free device memory
    where it was."""
    from gdl_amd import _native as nat
    L = nat.lib()
    E, N = 300_000, 20_000
    col = _targets(E, N, 7).to(dev)
    outs = [torch.empty(E, dtype=torch.int32, device=dev) for _ in range(2)] + \
           [torch.empty(N, dtype=torch.int32, device=dev) for _ in range(2)]

    def call():
        nat.check(L.geo_csr_build_noalloc(col.data_ptr(), E, N, *[o.data_ptr() for o in outs],
                                          nat.stream_of(dev)), "geo_csr_build_noalloc")

    call()  # warm-up: looks up the scratch address of this device
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(5):
        call()
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] >= free0
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for seed, srt in ((8, False), (9, True), (10, False)):
        print(f"[noalloc graph] replay seed={seed} sorted={srt}", flush=True)
        col.copy_(_targets(E, N, seed, srt).to(dev))
        for o in outs:
            o.fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        want = _csr_ws(nat, col, N)   # eager work between the replays
        torch.cuda.synchronize()
        for g_, w_, name in zip(outs, want, ("col_sorted", "perm", "node_start", "node_end")):
            assert torch.equal(g_, w_), (name, seed)
