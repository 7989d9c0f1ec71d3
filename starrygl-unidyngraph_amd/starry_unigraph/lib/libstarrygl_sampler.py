"""Module surface of the reference's native sampler, backed by HIP kernels.

The reference imports ``starry_unigraph.lib.libstarrygl_sampler``, a pybind11
module built from vendor/bts_sampler/sampler/export.cpp:10-106. This module
keeps the names and argument meaning that the CTDG path binds:

* ``get_neighbors(graph_name, row, col, num_nodes, is_distinct, eid, dist_eid,
  edge_weight, time)``  (export.cpp:13-15, neighbors.h:209-284)
* ``ParallelSampler(tnb, num_nodes, num_edges, threads, fanouts, num_layers,
  policy, local_part, part, node_part, p)`` with ``neighbor_sample_from_nodes``,
  ``get_ret``, ``reset`` and ``ret`` (export.cpp:73-79, sampler.h:30-90)
* ``TemporalGraphBlock`` getters ``sample_nodes/eid/src_index/delta_ts/
  sample_nodes_ts/sample_weight/row/col`` and the read-only ``sample_time``,
  ``tot_time``, ``sample_edge_num`` (export.cpp:30-45, output.h:4-30)
* ``TemporalNeighborBlock`` with ``deg``, ``with_eid``, ``with_timestamp``,
  ``weighted`` (export.cpp:47-71)

Differences, by design: graphs live in HBM and sampling runs on the GPU;
getters return int64/float32 tensors on the GPU holding the same values the
reference returns on the CPU (every caller casts with ``.long()``,
``.float()``, ``.to(device)``). Only the ``recent`` policy -- the one the CTDG
path configures -- is implemented; other policy names raise RuntimeError.
"""
from __future__ import annotations

import time

import torch

from starry_unigraph.lib import _capi
from starry_unigraph.native.tcsr import DeviceTCSR, RecentSampler, SampleHop, build_tcsr

_TNB_CACHE: dict[str, "TemporalNeighborBlock"] = {}

_KNOWN_POLICIES = ("recent", "uniform", "weighted", "boundery_recent_decay",
                   "boundery_recent_uniform", "boundery_uniform")


class TemporalNeighborBlock:
    """HBM-resident in-neighbour lists (neighbors.h:7-207)."""

    def __init__(self, graph: DeviceTCSR, with_eid: bool, with_timestamp: bool, weighted: bool):
        self.graph = graph
        self.with_eid = with_eid
        self.with_timestamp = with_timestamp
        self.weighted = weighted

    @property
    def deg(self) -> torch.Tensor:
        return self.graph.deg

    def _lists(self, arr: torch.Tensor) -> list[torch.Tensor]:
        ip = self.graph.indptr.cpu().tolist()
        a = arr.long().cpu()
        return [a[ip[i]:ip[i + 1]] for i in range(self.graph.num_nodes)]

    @property
    def neighbors(self) -> list[torch.Tensor]:
        return self._lists(self.graph.nbr)

    @property
    def timestamp(self) -> list[torch.Tensor]:
        return self._lists(self.graph.ts)

    @property
    def eid(self) -> list[torch.Tensor]:
        return self._lists(self.graph.eid)

    def empty(self) -> bool:
        return self.graph.num_nodes == 0


def get_neighbors(graph_name: str, row: torch.Tensor, col: torch.Tensor, num_nodes: int, is_distinct: int = 0,
                  eid: torch.Tensor | None = None, dist_eid: torch.Tensor | None = None,
                  edge_weight: torch.Tensor | None = None, time: torch.Tensor | None = None) -> TemporalNeighborBlock:
    """neighbors.h:209-284. Like the reference, a graph name seen before returns
    the cached block even if the arrays differ (neighbors.h:219-221)."""
    cached = _TNB_CACHE.get(graph_name)
    if cached is not None:
        return cached
    for name, t in (("row", row), ("col", col), ("eid", eid), ("time", time)):
        if t is not None and t.dim() != 1:
            raise RuntimeError(f"get_neighbors: {name} tensor must be one-dimensional")
    if time is None:
        raise RuntimeError("get_neighbors: the MI355X sampler implements temporal (recent) sampling; "
                           "time must be given")
    g = build_tcsr(int(num_nodes), row, col, eid=eid, ts=time)
    tnb = TemporalNeighborBlock(g, with_eid=eid is not None, with_timestamp=True, weighted=edge_weight is not None)
    _TNB_CACHE[graph_name] = tnb
    return tnb


class TemporalGraphBlock:
    """One hop of output (output.h:4-30). Arrays are GPU tensors."""

    def __init__(self, hop: SampleHop | None = None):
        self._hop = hop
        self.sample_time = 0.0
        self.tot_time = 0.0
        self.sample_edge_num = 0

    def _count(self) -> int:
        return 0 if self._hop is None else self._hop.count()

    def _empty(self, dtype=torch.int64) -> torch.Tensor:
        return torch.empty(0, dtype=dtype)

    def sample_nodes(self) -> torch.Tensor:
        return self._empty() if self._hop is None else self._hop.nbr[:self._count()].long()

    def eid(self) -> torch.Tensor:
        return self._empty() if self._hop is None else self._hop.eid[:self._count()].long()

    def src_index(self) -> torch.Tensor:
        if self._hop is None:
            return self._empty()
        cnt = self._hop.ptr[1:] - self._hop.ptr[:-1]
        q = torch.arange(cnt.numel(), device=cnt.device, dtype=torch.int64)
        return torch.repeat_interleave(q, cnt, output_size=self._count())

    def sample_nodes_ts(self) -> torch.Tensor:
        if self._hop is None:
            return self._empty()
        return self._hop.ts[:self._count()].clone()

    def delta_ts(self) -> torch.Tensor:
        if self._hop is None:
            return self._empty()
        return self._hop.q_ts[self.src_index()] - self._hop.ts[:self._count()]

    def sample_weight(self) -> torch.Tensor:
        if self._hop is None:
            return self._empty(torch.float32)
        si = self.src_index()
        pos = torch.arange(si.numel(), device=si.device, dtype=torch.int64) - self._hop.ptr[si]
        return pos.float()

    def row(self) -> torch.Tensor:
        return self._empty()

    def col(self) -> torch.Tensor:
        return self._empty()

    def dt_f32(self) -> torch.Tensor:
        """float32(delta_ts) straight from the kernel (what build_dgl_block uses)."""
        return torch.empty(0) if self._hop is None else self._hop.dt[:self._count()]


class ParallelSampler:
    """sampler.h:6-65. ``threads`` is accepted and ignored (GPU sampling)."""

    def __init__(self, tnb: TemporalNeighborBlock, num_nodes: int, num_edges: int, threads: int,
                 fanouts: list[int], num_layers: int, policy: str, local_part: int = -1,
                 part: torch.Tensor | None = None, node_part: torch.Tensor | None = None, p: float = 1.0):
        self.tnb = tnb
        self.num_nodes = int(num_nodes)
        self.num_edges = int(num_edges)
        self.threads = int(threads)
        self.fanouts = [int(f) for f in fanouts]
        self.num_layers = int(num_layers)
        self.policy = str(policy)
        self.local_part = int(local_part)
        self.boundery_probility = float(p)
        if self.num_layers > len(self.fanouts):
            raise RuntimeError(f"ParallelSampler: num_layers {self.num_layers} > len(fanouts) {len(self.fanouts)}")
        self._sampler = RecentSampler.for_graph(tnb.graph)
        self.ret: list[TemporalGraphBlock] = [TemporalGraphBlock() for _ in range(self.num_layers)]

    def reset(self) -> None:
        self.ret = [TemporalGraphBlock() for _ in range(self.num_layers)]

    def neighbor_sample_from_nodes(self, nodes: torch.Tensor, root_ts: torch.Tensor | None = None,
                                   part_unique: bool | None = None) -> None:
        """sampler.h:69-90 -> _with_before (sampler.h:393-399)."""
        if self.policy not in _KNOWN_POLICIES:
            raise RuntimeError(f'The policy "{self.policy}" is not exit!')
        if self.policy != "recent":
            raise RuntimeError(f'policy "{self.policy}" is not implemented by the MI355X sampler '
                               '(the CTDG path configures "recent")')
        if not self.tnb.with_timestamp:
            raise RuntimeError("Tnb has no timestamp infomation!")
        if root_ts is None:
            raise RuntimeError("Parameter mismatch!")
        for name, t in (("nodes", nodes), ("root_ts", root_ts)):
            if t.dim() != 1:
                raise RuntimeError(f"{name} tensor must be one-dimensional")
        t0 = time.perf_counter()
        self._sampler.err.reset()
        hops = self._sampler.sample_hops(nodes, root_ts.to(torch.int64), self.fanouts[:self.num_layers],
                                         want_last_ts=True)
        self._sampler.err.raise_if_set("neighbor_sample_from_nodes")
        self.ret = []
        total = 0
        for hop in hops:
            blk = TemporalGraphBlock(hop)
            total += blk._count()
            self.ret.append(blk)
        if self.ret:
            self.ret[0].tot_time = time.perf_counter() - t0
            self.ret[0].sample_time = self.ret[0].tot_time
            self.ret[0].sample_edge_num = total

    def get_ret(self) -> list[TemporalGraphBlock]:
        return list(self.ret)


def is_available() -> bool:
    try:
        _capi.lib()
        return torch.cuda.is_available()
    except Exception:
        return False
