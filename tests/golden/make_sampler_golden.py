"""Write the sampler golden fixtures (tests/golden/sampler_*.npz).

Runs the reference's own C++ sampler, compiled from its sources by
``make -C oracle ref`` into oracle/_ref/, on small seeded inputs and stores
inputs and outputs. Run in the build container (it needs /root/reference to
compile the checker); the fixtures are data and travel with the repository.

    python tests/golden/make_sampler_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle", "_ref"))

import libstarrygl_sampler_ref as ref  # noqa: E402


def _zipf_ids(rng, n, size, s):
    w = 1.0 / np.arange(1, n + 1, dtype=np.float64) ** s
    w /= w.sum()
    perm = rng.permutation(n)
    return perm[rng.choice(n, size=size, p=w)]


def run_ref(name, num_nodes, row, col, eid, ts, nodes, q_ts, fanouts):
    t = lambda a: torch.as_tensor(np.ascontiguousarray(a, dtype=np.int64))
    tnb = ref.get_neighbors(name, t(row), t(col), int(num_nodes), 0, t(eid), None, None, t(ts))
    ne = len(row)
    ps = ref.ParallelSampler(tnb, int(num_nodes), int(ne), 1, list(fanouts), len(fanouts), "recent", -1,
                             torch.zeros(ne, dtype=torch.int32), torch.zeros(num_nodes, dtype=torch.int32), 1.0)
    ps.neighbor_sample_from_nodes(t(nodes), t(q_ts), None)
    blocks = ps.get_ret()
    out = {}
    for h, b in enumerate(blocks):
        out[f"src_index_{h}"] = b.src_index().clone().numpy()
        out[f"sample_nodes_{h}"] = b.sample_nodes().clone().numpy()
        out[f"sample_nodes_ts_{h}"] = b.sample_nodes_ts().clone().numpy()
        out[f"eid_{h}"] = b.eid().clone().numpy()
        out[f"delta_ts_{h}"] = b.delta_ts().clone().numpy()
        out[f"sample_weight_{h}"] = b.sample_weight().clone().numpy()
    deg = np.asarray(tnb.deg, dtype=np.int64)
    return out, deg


def save(case, num_nodes, row, col, eid, ts, nodes, q_ts, fanouts):
    out, deg = run_ref(f"golden_{case}", num_nodes, row, col, eid, ts, nodes, q_ts, fanouts)
    path = os.path.join(HERE, f"sampler_{case}.npz")
    np.savez_compressed(
        path,
        num_nodes=np.int64(num_nodes), row=np.asarray(row, np.int64), col=np.asarray(col, np.int64),
        eid=np.asarray(eid, np.int64), ts=np.asarray(ts, np.int64), nodes=np.asarray(nodes, np.int64),
        q_ts=np.asarray(q_ts, np.int64), fanouts=np.asarray(fanouts, np.int64), deg=deg, **out)
    print(case, {k: v.shape for k, v in out.items() if k.startswith("eid_")}, os.path.getsize(path), "bytes")


def main():
    # 1. hand-made edge cases: ties, zero-history nodes, deg<=k and deg>k,
    #    query time equal to an edge time (strict <), fanout larger than history.
    row = [1, 2, 3, 1, 2, 4, 5, 5, 6, 1, 2, 3]
    col = [0, 0, 0, 4, 0, 0, 0, 4, 0, 7, 7, 7]
    ts = [1, 2, 2, 3, 5, 5, 5, 8, 9, 9, 9, 9]
    eid = list(range(len(row)))
    nodes = [0, 0, 0, 4, 4, 7, 7, 3, 8, 0, 0]
    q_ts = [0, 2, 5, 3, 100, 9, 10, 50, 1, 6, 10]
    save("edge_cases", 9, row, col, eid, ts, nodes, q_ts, [3])
    save("edge_cases_2hop", 9, row, col, eid, ts, nodes, q_ts, [3, 2])
    save("edge_cases_k0", 9, row, col, eid, ts, nodes, q_ts, [0])

    # 2. unsorted per-node timestamps: pins the lower_bound probe sequence.
    rng = np.random.default_rng(7)
    n, e = 6, 40
    row = rng.integers(0, n, e)
    col = rng.integers(0, n, e)
    ts = rng.integers(0, 20, e)
    save("unsorted", n, row, col, np.arange(e), ts, rng.integers(0, n, 30), rng.integers(0, 22, 30), [4, 3])

    # 3. cfg1-like small bipartite stream (Zipf 1.2 endpoints, sorted float32
    #    times truncated to int64 as in data.py:228), queries = one batch's roots
    #    at floor(max batch ts) (runtime.py:141-142, sampler.py:113).
    rng = np.random.default_rng(1)
    ns, nd, e = 300, 60, 4000
    src = _zipf_ids(rng, ns, e, 1.2)
    dst = ns + _zipf_ids(rng, nd, e, 1.2)
    tsf = np.sort(rng.uniform(0, 2.7e6, e)).astype(np.float32)
    ts_i = tsf.astype(np.int64)
    b0, b1 = 3000, 3200
    roots = np.unique(np.concatenate([src[b0:b1], dst[b0:b1]]))
    tq = np.full(roots.shape, int(np.float32(tsf[b0:b1].max())), dtype=np.int64)
    save("bipartite", ns + nd, src, dst, np.arange(e), ts_i, roots, tq, [10])
    save("bipartite_2hop", ns + nd, src, dst, np.arange(e), ts_i, roots, tq, [10, 10])

    # 3b. cfg4/cfg5-like small unipartite stream (Zipf 1.5), 2 hops of k=20.
    rng = np.random.default_rng(2)
    n, e = 400, 5000
    src = _zipf_ids(rng, n, e, 1.5)
    dst = _zipf_ids(rng, n, e, 1.5)
    tsf = np.sort(rng.uniform(0, 2.0e8, e)).astype(np.float32)
    ts_i = tsf.astype(np.int64)
    b0, b1 = 4000, 4400
    roots = np.unique(np.concatenate([src[b0:b1], dst[b0:b1]]))
    tq = np.full(roots.shape, int(np.float32(tsf[b0:b1].max())), dtype=np.int64)
    save("unipartite_2hop", n, src, dst, np.arange(e), ts_i, roots, tq, [20, 20])

    # 4. large timestamps near 2^53 and a power-law degree mix.
    rng = np.random.default_rng(3)
    n, e = 500, 6000
    deg = np.minimum(np.floor(rng.pareto(1.1, n) + 1).astype(np.int64), 400)
    col = np.repeat(np.arange(n), deg)[:e]
    e = col.shape[0]
    row = rng.integers(0, n, e)
    base = np.int64(2) ** 53 - np.int64(10 ** 7)
    ts = base + np.sort(rng.integers(0, 10 ** 6, e))
    order = np.argsort(ts, kind="stable")
    col, row, ts = col[order], row[order], ts[order]
    q = rng.integers(0, n, 700)
    tq = base + rng.integers(0, 10 ** 6 + 5, 700)
    save("large_ts", n, row, col, np.arange(e), ts, q, tq, [20])

    # 5. empty query list
    save("empty_queries", 9, [1, 2], [0, 0], [0, 1], [1, 2], [], [], [5])


if __name__ == "__main__":
    main()
