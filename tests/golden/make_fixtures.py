"""Writes the golden fixtures in this directory (``*.json``): small inputs with expected outputs
derived independently of the oracle and of the GPU library — closed forms and exact integer
brute force in plain Python (integer coordinates and integer-valued features make every fp32
result exact, so the fixtures hold bit-exact answers).

Cases restate the reference's own known-answer tests where it has them:
  * FPS on a line and on a permuted lattice (tests/test_fps_cuda_remote.py:63-90 checks only
    shapes, uniqueness and batch isolation; the values here follow the greedy definition,
    geoembodied/csrc/__init__.py:600-654);
  * radius graph KATs of tests/test_phase1.py:258-298 and tests/test_radius_graph_cuda.py:166-192;
  * segment sum KATs of tests/test_segment_reduce.py:118-141.

Usage: python tests/golden/make_fixtures.py   (rewrites the JSON files; output is deterministic)
"""

from __future__ import annotations

import json
import random
from pathlib import Path

HERE = Path(__file__).resolve().parent


def d2(a, b):
    return sum((x - y) * (x - y) for x, y in zip(a, b))


def lattice(n, seed):
    pts = [[x, y, z] for x in range(n) for y in range(n) for z in range(n)]
    random.Random(seed).shuffle(pts)
    return pts


def fps_greedy(pts, ptr, ks):
    out = []
    for b in range(len(ptr) - 1):
        s, e = ptr[b], ptr[b + 1]
        n, k = e - s, max(0, min(ks[b], e - s))
        if k == 0:
            continue
        if k == n:
            out += list(range(s, e))
            continue
        md = [float("inf")] * n
        cur = 0
        sel = [s]
        for _ in range(k - 1):
            for i in range(n):
                md[i] = min(md[i], d2(pts[s + i], pts[s + cur]))
            best = max(md)
            cur = md.index(best)  # lowest index attaining the max
            sel.append(s + cur)
        out += sel
    return out


def knn_brute(q, s, pq, ps, k):
    idx, dist = [], []
    for b in range(len(pq) - 1):
        for qi in range(pq[b], pq[b + 1]):
            keys = sorted((d2(q[qi], s[j]), j) for j in range(ps[b], ps[b + 1]))[:k]
            idx.append([j for _, j in keys] + [-1] * (k - len(keys)))
            dist.append([float(d) for d, _ in keys] + [1e30] * (k - len(keys)))
    return idx, dist


def radius_brute(x, r2, K, loop=False, batch=None):
    rows, cols = [], []
    for i in range(len(x)):
        cand = sorted((d2(x[i], x[j]), j) for j in range(len(x))
                      if (loop or j != i) and (batch is None or batch[i] == batch[j])
                      and d2(x[i], x[j]) < r2)[:K]
        for _, j in sorted(cand, key=lambda t: t[1]):
            rows.append(j)
            cols.append(i)
    return rows, cols


def csr_stable(col, N):
    order = sorted(range(len(col)), key=lambda e: (col[e] if 0 <= col[e] < N else N, e))
    col_sorted = [col[e] if 0 <= col[e] < N else N for e in order]
    start, end = [], []
    for n in range(N):
        start.append(sum(1 for c in col_sorted if c < n))
        end.append(sum(1 for c in col_sorted if c <= n))
    return col_sorted, order, start, end


def seg_reduce(msg, perm, start, end, reduce):
    C = len(msg[0]) if msg else 0
    out, arg = [], []
    for a, b in zip(start, end):
        rows = [msg[perm[e]] for e in range(a, b)]
        if reduce == "sum":
            out.append([sum(r[c] for r in rows) for c in range(C)])
        elif reduce == "mean":
            out.append([sum(r[c] for r in rows) / max(b - a, 1) for c in range(C)])
        else:
            o, g = [], []
            for c in range(C):
                if not rows:
                    o.append(0.0)
                    g.append(-1)
                    continue
                m = max(r[c] for r in rows)
                hits = [a + t for t, r in enumerate(rows) if r[c] == m]
                o.append(m)
                g.append(hits[0] if len(hits) == 1 else -len(hits))
            out.append(o)
            arg.append(g)
    return out, arg


def main():
    fx = {}
    line = [[float(i), 0.0, 0.0] for i in range(11)]
    fx["fps_line"] = dict(pos=line, ptr=[0, 11], k=[5], want=[0, 10, 5, 2, 7])
    lat = lattice(4, 1) + lattice(3, 2)
    fx["fps_lattice"] = dict(pos=lat, ptr=[0, 64, 91], k=[20, 27],
                             want=fps_greedy(lat, [0, 64, 91], [20, 27]))
    src = lattice(4, 3)
    qry = [[x + 0.5 * (i % 2), y, z] for i, (x, y, z) in enumerate(lattice(3, 4))]
    fx["knn_lattice"] = dict(query=qry, source=src, ptr_q=[0, 20, 27], ptr_s=[0, 40, 64], k=6)
    fx["knn_lattice"]["want_idx"], fx["knn_lattice"]["want_dist"] = knn_brute(
        qry, src, [0, 20, 27], [0, 40, 64], 6)
    rl = lattice(4, 5)
    fx["radius_lattice"] = dict(x=rl, r=1.5, K=4, loop=False)
    fx["radius_lattice"]["want_row"], fx["radius_lattice"]["want_col"] = radius_brute(rl, 2.25, 4)
    fx["radius_kat_three_points"] = dict(x=[[0, 0, 0], [0.5, 0, 0], [10, 0, 0]], r=1.0, K=32,
                                         loop=False, want_row=[1, 0], want_col=[0, 1])
    fx["radius_kat_batches"] = dict(x=[[0, 0, 0], [0.5, 0, 0]], r=100.0, K=32, loop=False,
                                    batch=[0, 1], want_row=[], want_col=[])
    col = [3, 1, 3, 0, 1, 3, -2, 7, 2, 3, 1, 0]
    cs, pm, st, en = csr_stable(col, 5)
    fx["csr"] = dict(col=col, N=5, col_sorted=cs, perm=pm, start=st, end=en)
    rnd = random.Random(6)
    msg = [[float(rnd.randint(-3, 3)) for _ in range(4)] for _ in range(len(col))]
    for red in ("sum", "mean", "max"):
        out, arg = seg_reduce(msg, pm, st, en, red)
        fx[f"segment_{red}"] = dict(msg=msg, perm=pm, start=st, end=en, reduce=red, want=out,
                                    want_arg=arg)
    fx["segment_sum_all_to_one"] = dict(msg=[[1.0] * 4] * 10, perm=list(range(10)), start=[0],
                                        end=[10], reduce="sum", want=[[10.0] * 4], want_arg=[])
    for name, v in fx.items():
        (HERE / f"{name}.json").write_text(json.dumps(v, sort_keys=True) + "\n")
    print(f"wrote {len(fx)} fixtures to {HERE}")


if __name__ == "__main__":
    main()
