"""TEST INFRASTRUCTURE ONLY -- numpy/ctypes driver of the C sampler oracle.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this module, and only as the checker. The product path never
imports it.

Restates, on the CPU:
  * ``get_neighbors``  (vendor/bts_sampler/sampler/include/neighbors.h:209-284)
  * ``ParallelSampler.neighbor_sample_from_nodes`` with policy ``recent``
    (sampler.h:69-90 -> _with_before sampler.h:393-399 ->
    _with_before_layer sampler.h:213-391)
  * the query-time chain of ``BTSNativeSampler.sample_from_nodes``
    (native/bts_sampler.py:77-82: ``ts.to(int64)``).

Pinned by: tests/test_oracle_sampler.py (brute force on tiny graphs, closed
form properties) and tests/golden/sampler_*.npz, which were written by the
reference's own C++ sampler compiled from its sources (oracle/Makefile ``ref``).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

_i64p = ctypes.POINTER(ctypes.c_int64)
_f32p = ctypes.POINTER(ctypes.c_float)


def _lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run `make -C oracle`)")
        lib = ctypes.CDLL(path)
        lib.orc_tcsr_build.restype = ctypes.c_int
        lib.orc_tcsr_build.argtypes = [ctypes.c_int64, ctypes.c_int64] + [_i64p] * 8
        lib.orc_recent_search.restype = ctypes.c_int
        lib.orc_recent_search.argtypes = [_i64p, _i64p, ctypes.c_int64, ctypes.c_int64,
                                          _i64p, _i64p, ctypes.c_int, _i64p, _i64p]
        lib.orc_recent_fill.restype = None
        lib.orc_recent_fill.argtypes = [_i64p, _i64p, _i64p, ctypes.c_int64, _i64p, _i64p,
                                        _i64p, _i64p, _i64p, _i64p, _i64p, _i64p, _i64p, _f32p]
        lib.orc_set_threads.argtypes = [ctypes.c_int]
        lib.orc_get_threads.restype = ctypes.c_int
        _LIB = lib
    return _LIB


def _p(a: np.ndarray, ptype=_i64p):
    return a.ctypes.data_as(ptype)


def set_threads(n: int) -> None:
    _lib().orc_set_threads(int(n))


def get_threads() -> int:
    return int(_lib().orc_get_threads())


@dataclass
class OracleTCSR:
    num_nodes: int
    indptr: np.ndarray   # int64 [N+1]
    nbr: np.ndarray      # int64 [E]
    eid: np.ndarray      # int64 [E]
    ts: np.ndarray       # int64 [E]

    @property
    def deg(self) -> np.ndarray:
        return np.diff(self.indptr)


def build_tcsr(num_nodes: int, row, col, eid, ts) -> OracleTCSR:
    """neighbors.h:209-284 restated: in-neighbour lists keyed by ``col``."""
    row = np.ascontiguousarray(row, dtype=np.int64)
    col = np.ascontiguousarray(col, dtype=np.int64)
    eid = np.ascontiguousarray(eid, dtype=np.int64)
    ts = np.ascontiguousarray(ts, dtype=np.int64)
    e = row.shape[0]
    indptr = np.zeros(num_nodes + 1, dtype=np.int64)
    nbr = np.empty(e, dtype=np.int64)
    eo = np.empty(e, dtype=np.int64)
    to = np.empty(e, dtype=np.int64)
    rc = _lib().orc_tcsr_build(num_nodes, e, _p(row), _p(col), _p(eid), _p(ts),
                               _p(indptr), _p(nbr), _p(eo), _p(to))
    if rc != 0:
        raise RuntimeError("oracle tcsr: node id out of range")
    return OracleTCSR(num_nodes, indptr, nbr, eo, to)


def sample_layer(g: OracleTCSR, nodes, ts, fanout: int) -> dict[str, np.ndarray]:
    """One hop of sampler.h:213-391 with policy ``recent``."""
    nodes = np.ascontiguousarray(nodes, dtype=np.int64)
    ts = np.ascontiguousarray(ts, dtype=np.int64)
    nq = nodes.shape[0]
    begin = np.empty(nq, dtype=np.int64)
    cnt = np.empty(nq, dtype=np.int64)
    rc = _lib().orc_recent_search(_p(g.indptr), _p(g.ts), g.num_nodes, nq, _p(nodes), _p(ts),
                                  int(fanout), _p(begin), _p(cnt))
    if rc != 0:
        raise RuntimeError("oracle sampler: query node out of range")
    offsets = np.zeros(nq + 1, dtype=np.int64)
    np.cumsum(cnt, out=offsets[1:])
    total = int(offsets[-1])
    out = {k: np.empty(total, dtype=np.int64) for k in
           ("src_index", "sample_nodes", "sample_nodes_ts", "eid", "delta_ts")}
    out["sample_weight"] = np.empty(total, dtype=np.float32)
    _lib().orc_recent_fill(_p(g.nbr), _p(g.eid), _p(g.ts), nq, _p(ts), _p(begin), _p(cnt),
                           _p(offsets), _p(out["src_index"]), _p(out["sample_nodes"]),
                           _p(out["sample_nodes_ts"]), _p(out["eid"]), _p(out["delta_ts"]),
                           _p(out["sample_weight"], _f32p))
    out["ptr"] = offsets
    return out


def sample_recent(g: OracleTCSR, nodes, ts, fanouts: list[int]) -> list[dict[str, np.ndarray]]:
    """sampler.h:393-399: hop l+1 queries are hop l's (sample_nodes, sample_nodes_ts)."""
    blocks = []
    q_nodes, q_ts = np.asarray(nodes, dtype=np.int64), np.asarray(ts, dtype=np.int64)
    for k in fanouts:
        blk = sample_layer(g, q_nodes, q_ts, int(k))
        blocks.append(blk)
        q_nodes, q_ts = blk["sample_nodes"], blk["sample_nodes_ts"]
    return blocks


def brute_force_layer(num_nodes: int, row, col, eid, ts, nodes, q_ts, fanout: int):
    """Pure-Python statement of the recent policy for SORTED per-node timestamps:
    the node's in-events (col == node) with ts < t, the last ``fanout`` of them in
    event order, emitted oldest first. Small inputs only."""
    row, col, eid, ts = (list(map(int, a)) for a in (row, col, eid, ts))
    out = {k: [] for k in ("src_index", "sample_nodes", "sample_nodes_ts", "eid", "delta_ts", "sample_weight")}
    for i, (n, t) in enumerate(zip(map(int, nodes), map(int, q_ts))):
        hist = [j for j in range(len(col)) if col[j] == n and ts[j] < t]
        win = hist[max(0, len(hist) - fanout):] if fanout > 0 else []
        for w, j in enumerate(win):
            out["src_index"].append(i)
            out["sample_nodes"].append(row[j])
            out["sample_nodes_ts"].append(ts[j])
            out["eid"].append(eid[j])
            out["delta_ts"].append(t - ts[j])
            out["sample_weight"].append(float(w))
    res = {k: np.asarray(v, dtype=np.int64) for k, v in out.items() if k != "sample_weight"}
    res["sample_weight"] = np.asarray(out["sample_weight"], dtype=np.float32)
    return res
