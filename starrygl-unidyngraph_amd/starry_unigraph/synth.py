"""Seeded synthetic event streams for the benchmark configurations.

All generators use ``numpy.random.Generator(PCG64(seed))`` and return numpy
arrays; nothing is downloaded.

* ``bipartite_stream``  -- configs 1/2: 8,227 sources + 1,000 destinations,
  157,474 events, Zipf(1.2) endpoints per side, sorted Uniform[0, 2.7e6]
  float32 times, 172-d N(0,1) edge features.
* ``unipartite_stream`` -- configs 4/5: 1,140,149 nodes, 7,833,140 events,
  Zipf(1.5) endpoints, sorted Uniform[0, 2.0e8] float32 times, 16-d features.
* ``powerlaw_sampler_graph`` / ``degree_weighted_queries`` -- config 3: 1e7
  nodes, 1e8 time-ordered edges with power-law (alpha 2.1, max 1e5) in-degrees,
  int64 Uniform[0, 1e9] times; 4e6 (node, t) queries, node drawn by degree.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def _rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


@dataclass
class EventStream:
    src: np.ndarray        # int64 [E]
    dst: np.ndarray        # int64 [E]
    ts: np.ndarray         # float32 [E], non-decreasing
    edge_feat: np.ndarray  # float32 [E, F]
    num_nodes: int
    name: str = "synthetic"

    @property
    def num_events(self) -> int:
        return int(self.src.shape[0])


def bounded_zipf(rng: np.random.Generator, n: int, size: int, s: float) -> np.ndarray:
    """Ids in [0, n) with P(rank r) ∝ r^-s, ranks mapped to ids by a seeded permutation."""
    w = np.arange(1, n + 1, dtype=np.float64) ** (-s)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    ranks = np.searchsorted(cdf, rng.random(size), side="right")
    np.minimum(ranks, n - 1, out=ranks)
    perm = rng.permutation(n)
    return perm[ranks].astype(np.int64)


def sorted_uniform(rng: np.random.Generator, size: int, t_max: float) -> np.ndarray:
    """Order statistics of Uniform[0, t_max] (normalised exponential spacings), float64."""
    gaps = rng.standard_exponential(size + 1)
    c = np.cumsum(gaps)
    return c[:-1] / c[-1] * t_max


def bipartite_stream(num_src: int = 8227, num_dst: int = 1000, num_events: int = 157474,
                     zipf_s: float = 1.2, t_max: float = 2.7e6, edge_dim: int = 172,
                     seed: int = 0) -> EventStream:
    rng = _rng(seed)
    src = bounded_zipf(rng, num_src, num_events, zipf_s)
    dst = num_src + bounded_zipf(rng, num_dst, num_events, zipf_s)
    ts = sorted_uniform(rng, num_events, t_max).astype(np.float32)
    feat = rng.standard_normal((num_events, edge_dim), dtype=np.float32)
    return EventStream(src, dst, ts, feat, num_src + num_dst, name="bipartite")


def unipartite_stream(num_nodes: int = 1140149, num_events: int = 7833140, zipf_s: float = 1.5,
                      t_max: float = 2.0e8, edge_dim: int = 16, seed: int = 0) -> EventStream:
    rng = _rng(seed)
    src = bounded_zipf(rng, num_nodes, num_events, zipf_s)
    dst = bounded_zipf(rng, num_nodes, num_events, zipf_s)
    ts = sorted_uniform(rng, num_events, t_max).astype(np.float32)
    feat = rng.standard_normal((num_events, edge_dim), dtype=np.float32)
    return EventStream(src, dst, ts, feat, num_nodes, name="unipartite")


def powerlaw_degrees(rng: np.random.Generator, num_nodes: int, num_edges: int, alpha: float = 2.1,
                     max_deg: int = 100000) -> np.ndarray:
    """Degrees with P(d) ∝ d^-alpha on [1, max_deg], rescaled to sum exactly to
    num_edges by largest-remainder rounding, each capped at max_deg (excess
    re-spread over the nodes below the cap)."""
    d = np.arange(1, max_deg + 1, dtype=np.float64)
    p = d ** (-alpha)
    cdf = np.cumsum(p)
    cdf /= cdf[-1]
    raw = (np.searchsorted(cdf, rng.random(num_nodes), side="right") + 1).astype(np.float64)
    raw = np.minimum(raw, max_deg)
    target = float(num_edges)
    deg = np.zeros(num_nodes, dtype=np.int64)
    for _ in range(64):
        scaled = raw * (target / raw.sum())
        scaled = np.minimum(scaled, max_deg)
        deg = np.floor(scaled).astype(np.int64)
        rem = num_edges - int(deg.sum())
        if rem <= 0:
            break
        room = deg < max_deg
        frac = np.where(room, scaled - deg, -1.0)
        k = min(rem, int(room.sum()))
        top = np.argpartition(-frac, k - 1)[:k] if k > 0 else np.empty(0, dtype=np.int64)
        deg[top] += 1
        rem -= k
        if rem == 0:
            break
        raw = np.where(deg < max_deg, raw * 1.01, raw)
    if int(deg.sum()) != num_edges:
        raise RuntimeError("powerlaw_degrees: could not hit the edge count")
    return np.maximum(deg, 0)


@dataclass
class SamplerGraph:
    row: np.ndarray   # int64 [E] neighbour (src) id, global time order
    col: np.ndarray   # int64 [E] node (dst) id
    ts: np.ndarray    # int64 [E] non-decreasing
    num_nodes: int

    @property
    def num_edges(self) -> int:
        return int(self.row.shape[0])


def powerlaw_sampler_graph(num_nodes: int = 10_000_000, num_edges: int = 100_000_000, alpha: float = 2.1,
                           max_deg: int = 100000, t_max: int = 1_000_000_000, seed: int = 0) -> SamplerGraph:
    """Config 3 graph, fed in global time order (eid = position), so every
    node's list is time-sorted."""
    rng = _rng(seed)
    deg = powerlaw_degrees(rng, num_nodes, num_edges, alpha, max_deg)
    col = np.repeat(np.arange(num_nodes, dtype=np.int64), deg)
    rng.shuffle(col)                                   # random position in time
    ts = np.floor(sorted_uniform(rng, num_edges, float(t_max))).astype(np.int64)
    row = rng.integers(0, num_nodes, num_edges, dtype=np.int64)
    return SamplerGraph(row, col, ts, num_nodes)


def degree_weighted_queries(g: SamplerGraph, num_queries: int = 4_000_000, t_max: int = 1_000_000_000,
                            seed: int = 1) -> tuple[np.ndarray, np.ndarray]:
    """Node ∝ in-degree (the dst of a uniformly drawn edge); t ~ Uniform int [0, t_max]."""
    rng = _rng(seed)
    nodes = g.col[rng.integers(0, g.num_edges, num_queries)]
    t = rng.integers(0, t_max + 1, num_queries, dtype=np.int64)
    return nodes, t
