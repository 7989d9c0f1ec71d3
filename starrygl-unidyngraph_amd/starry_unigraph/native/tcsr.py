"""Device temporal CSR and recent-k sampling over the C ABI.

``DeviceTCSR`` is the HBM-resident form of the reference's
``TemporalNeighborBlock`` (vendor/bts_sampler/sampler/include/neighbors.h:7-207):
per-node in-neighbour lists keyed by dst, in event order, laid out as a CSR
(``indptr`` int64 [N+1]; ``nbr``/``eid`` int32 [E]; ``ts`` int64 [E]).

``recent_sample`` is one hop of ``ParallelSampler`` with policy ``recent``
(sampler.h:213-261): per query the last ``fanout`` in-events strictly before
``t``, concatenated in query order, described by ``ptr`` (int64 [Q+1]).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from starry_unigraph.lib import _capi


@dataclass
class DeviceTCSR:
    num_nodes: int
    num_edges: int
    indptr: torch.Tensor   # int64 [N+1]
    nbr: torch.Tensor      # int32 [E]
    eid: torch.Tensor      # int32 [E]
    ts: torch.Tensor       # int64 [E]

    @property
    def device(self) -> torch.device:
        return self.indptr.device

    @property
    def deg(self) -> torch.Tensor:
        return self.indptr[1:] - self.indptr[:-1]

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.indptr, self.nbr, self.eid, self.ts))


@dataclass
class PaddedHop:
    """One hop of recent-k output in the padded layout: row q of the [Q, k]
    arrays holds ``cnt[q]`` valid entries, oldest first."""
    cnt: torch.Tensor              # int32 [Q]
    nbr: torch.Tensor              # int32 [Q*k]
    eid: torch.Tensor              # int32 [Q*k]
    dt: torch.Tensor               # float32 [Q*k]
    ts: torch.Tensor | None        # int64 [Q*k] (entry timestamps) or None
    q_ts: torch.Tensor             # int64 [Q]
    fanout: int

    @property
    def num_queries(self) -> int:
        return self.cnt.numel()


@dataclass
class SampleHop:
    """One hop in the reference's concatenated layout, ``ptr`` int64 [Q+1]."""
    ptr: torch.Tensor
    nbr: torch.Tensor              # int32 [M]
    eid: torch.Tensor              # int32 [M]
    dt: torch.Tensor               # float32 [M]
    ts: torch.Tensor | None        # int64 [M]
    q_ts: torch.Tensor             # int64 [Q]

    @property
    def num_queries(self) -> int:
        return self.ptr.numel() - 1

    def count(self) -> int:
        return int(self.nbr.numel())


def _as_i64(t, device) -> torch.Tensor:
    t = torch.as_tensor(t)
    return t.to(device=device, dtype=torch.int64).contiguous()


def build_tcsr(num_nodes: int, row, col, eid=None, ts=None, device=None, check: bool = True) -> DeviceTCSR:
    """Build the device CSR from event-ordered (row=src, col=dst, eid, ts).

    Follows get_neighbors (neighbors.h:209-284): lists keyed by ``col`` in
    input order. ``ts`` is required (the recent policy needs it).
    """
    dev = _capi.require_gpu(device)
    lib = _capi.lib()
    if ts is None:
        raise RuntimeError("build_tcsr: timestamps are required for temporal sampling")
    row = _as_i64(row, dev)
    col = _as_i64(col, dev)
    ts = _as_i64(ts, dev)
    eid = None if eid is None else _as_i64(eid, dev)
    e = row.numel()
    if col.numel() != e or ts.numel() != e or (eid is not None and eid.numel() != e):
        raise RuntimeError("build_tcsr: row/col/eid/ts lengths differ")
    n = int(num_nodes)
    with torch.cuda.device(dev):
        indptr = torch.empty(n + 1, dtype=torch.int64, device=dev)
        # never-NULL storage (an empty graph still hands valid pointers to kernels)
        nbr = torch.empty(max(e, 1), dtype=torch.int32, device=dev)[:e]
        eo = torch.empty(max(e, 1), dtype=torch.int32, device=dev)[:e]
        to = torch.empty(max(e, 1), dtype=torch.int64, device=dev)[:e]
        ws_bytes = lib.sgl_tcsr_workspace_bytes(n, e)
        ws = _capi.workspace(ws_bytes, dev)
        err = _capi.ErrorFlag(dev)
        _capi.check(lib.sgl_tcsr_build(n, e, _capi.ptr(row), _capi.ptr(col), _capi.ptr(eid), _capi.ptr(ts),
                                       _capi.ptr(indptr), _capi.ptr(nbr), _capi.ptr(eo), _capi.ptr(to),
                                       _capi.ptr(ws), ws_bytes, _capi.ptr(err.t), _capi.stream_of(dev)),
                    "sgl_tcsr_build")
        if check:
            err.raise_if_set("build_tcsr")
    return DeviceTCSR(n, e, indptr, nbr, eo, to)


class RecentSampler:
    """Recent-k sampler bound to one DeviceTCSR. When every timestamp of the
    graph fits in int32 (checked once here), the sampler reads a packed copy:
    int32 timestamps and interleaved (nbr, eid) pairs (sgl_recent_sample_packed:
    identical results, half the bytes per probe, one run of ids per window);
    ``narrow_ts=False`` keeps the int64 arrays. When moreover every node's
    list is sorted by time, every 32nd timestamp goes into a fence array that
    large query batches search first."""

    def __init__(self, graph: DeviceTCSR, narrow_ts: bool = True):
        self.g = graph
        self.dev = graph.device
        self.err = _capi.ErrorFlag(self.dev)
        self.ts32: torch.Tensor | None = None
        self.ids: torch.Tensor | None = None
        self.fence: torch.Tensor | None = None
        if narrow_ts and graph.num_edges > 0:
            lo, hi = int(graph.ts.min().item()), int(graph.ts.max().item())
            if -2 ** 31 <= lo and hi < 2 ** 31:
                self.ts32 = graph.ts.to(torch.int32)
                self.ids = torch.stack([graph.nbr, graph.eid], dim=1).contiguous()
                # sorted lists: every decrease of ts is at a list boundary
                down = torch.nonzero(graph.ts[1:] < graph.ts[:-1]).flatten() + 1
                if down.numel() == 0 or bool(torch.isin(down, graph.indptr).all()):
                    self.fence = self.ts32[::32].contiguous()

    @classmethod
    def for_graph(cls, graph: DeviceTCSR) -> "RecentSampler":
        """The one sampler of ``graph`` (made on first use, then kept on the
        graph): its packed copy and fences are built once per CSR."""
        r = getattr(graph, "_recent_sampler", None)
        if r is None:
            r = cls(graph)
            graph._recent_sampler = r
        return r

    def sample(self, nodes: torch.Tensor, q_ts: torch.Tensor, fanout: int, want_ts: bool = False,
               valid_cnt: torch.Tensor | None = None, stride: int = 0,
               out: PaddedHop | None = None, num_live: torch.Tensor | None = None) -> PaddedHop:
        """One hop, padded layout, no host synchronisation. With ``valid_cnt``,
        query i is live only if ``i % stride < valid_cnt[i // stride]``; with
        ``num_live`` (a device int64 scalar) only queries i < num_live are."""
        dev = self.dev
        if nodes.device != dev or nodes.dtype not in (torch.int64, torch.int32):
            nodes = nodes.to(device=dev, dtype=torch.int64)
        nodes = nodes.contiguous()
        if q_ts.device != dev or q_ts.dtype != torch.int64:
            q_ts = q_ts.to(device=dev, dtype=torch.int64)
        q_ts = q_ts.contiguous()
        nq = nodes.numel()
        if q_ts.numel() != nq:
            raise RuntimeError(f"recent_sample: {nq} nodes but {q_ts.numel()} timestamps")
        fanout = int(fanout)
        if fanout < 0:
            raise RuntimeError(f"recent_sample: fanout {fanout} < 0")
        if valid_cnt is not None:
            if stride <= 0 or valid_cnt.dtype != torch.int32 or valid_cnt.numel() * stride < nq:
                raise RuntimeError("recent_sample: valid_cnt must be int32 with len*stride >= num queries")
        cap = nq * fanout
        if out is not None and out.num_queries == nq and out.fanout == fanout and (out.ts is not None) == want_ts:
            hop = PaddedHop(out.cnt, out.nbr, out.eid, out.dt, out.ts, q_ts, fanout)
        else:
            hop = PaddedHop(
                cnt=torch.empty(nq, dtype=torch.int32, device=dev),
                nbr=torch.empty(cap, dtype=torch.int32, device=dev),
                eid=torch.empty(cap, dtype=torch.int32, device=dev),
                dt=torch.empty(cap, dtype=torch.float32, device=dev),
                ts=torch.empty(cap, dtype=torch.int64, device=dev) if want_ts else None,
                q_ts=q_ts, fanout=fanout)
        g = self.g
        if self.ts32 is not None:
            fn, graph_args = "sgl_recent_sample_packed", (_capi.ptr(g.indptr), _capi.ptr(self.ids),
                                                          _capi.ptr(self.ts32), _capi.ptr(self.fence))
        else:
            fn, graph_args = "sgl_recent_sample", (_capi.ptr(g.indptr), _capi.ptr(g.nbr), _capi.ptr(g.eid),
                                                   _capi.ptr(g.ts))
        with torch.cuda.device(dev):
            _capi.check(_capi.call(fn, *graph_args, g.num_nodes,
                _capi.ptr(nodes), 1 if nodes.dtype == torch.int64 else 0, _capi.ptr(q_ts), nq,
                _capi.ptr(num_live), _capi.ptr(valid_cnt), int(stride), fanout,
                _capi.ptr(hop.cnt), _capi.ptr(hop.nbr), _capi.ptr(hop.eid), _capi.ptr(hop.dt),
                _capi.ptr(hop.ts), _capi.ptr(self.err.t), _capi.stream_of(dev)), fn)
        return hop

    def sample_padded_hops(self, nodes: torch.Tensor, q_ts: torch.Tensor, fanouts: list[int],
                           want_last_ts: bool = False) -> list[PaddedHop]:
        """sampler.h:393-399 without host syncs: hop l+1 queries are hop l's
        padded (nbr, ts) rows, masked by hop l's counts."""
        hops: list[PaddedHop] = []
        valid, stride = None, 0
        for li, k in enumerate(fanouts):
            last = li == len(fanouts) - 1
            hop = self.sample(nodes, q_ts, k, want_ts=(not last) or want_last_ts, valid_cnt=valid, stride=stride)
            hops.append(hop)
            nodes, q_ts, valid, stride = hop.nbr, hop.ts, hop.cnt, k
        return hops

    def compact(self, hop: PaddedHop) -> SampleHop:
        """Padded -> concatenated (the reference's TemporalGraphBlock layout).
        Synchronises once to size the output."""
        dev = self.dev
        nq = hop.num_queries
        ptr = torch.empty(nq + 1, dtype=torch.int64, device=dev)
        with torch.cuda.device(dev):
            if nq > 0:
                torch.cumsum(hop.cnt, 0, out=ptr[1:])
                ptr[0] = 0
                m = int(ptr[-1].item())
            else:
                ptr.zero_()
                m = 0
            # at least one element each, so no output pointer is NULL
            mm = max(m, 1)
            nbr = torch.empty(mm, dtype=torch.int32, device=dev)
            eid = torch.empty(mm, dtype=torch.int32, device=dev)
            dt = torch.empty(mm, dtype=torch.float32, device=dev)
            ts = torch.empty(mm, dtype=torch.int64, device=dev) if hop.ts is not None else None
            pad = [hop.nbr, hop.eid, hop.dt, hop.ts]
            if hop.nbr.numel() == 0:  # fanout 0: nothing to read, but keep pointers valid
                one = torch.empty(1, dtype=torch.int64, device=dev)
                pad = [one.view(torch.int32)[:1], one.view(torch.int32)[:1], one.view(torch.float32)[:1],
                       one if hop.ts is not None else None]
            ws_bytes = _capi.lib().sgl_compact_workspace_bytes(nq)
            ws = _capi.workspace(ws_bytes, dev)
            _capi.check(_capi.lib().sgl_recent_compact(
                nq, hop.fanout, _capi.ptr(hop.cnt), _capi.ptr(pad[0]), _capi.ptr(pad[1]), _capi.ptr(pad[2]),
                _capi.ptr(pad[3]), _capi.ptr(ptr), _capi.ptr(nbr), _capi.ptr(eid), _capi.ptr(dt), _capi.ptr(ts),
                _capi.ptr(ws), ws_bytes, _capi.stream_of(dev)), "sgl_recent_compact")
        return SampleHop(ptr, nbr[:m], eid[:m], dt[:m], None if ts is None else ts[:m], hop.q_ts)

    def sample_hops(self, nodes: torch.Tensor, q_ts: torch.Tensor, fanouts: list[int],
                    want_last_ts: bool = False) -> list[SampleHop]:
        """The reference's concatenated multi-hop output (sampler.h:393-399):
        hop l+1 queries are hop l's concatenated (sample_nodes, sample_nodes_ts)."""
        hops: list[SampleHop] = []
        for li, k in enumerate(fanouts):
            last = li == len(fanouts) - 1
            hop = self.compact(self.sample(nodes, q_ts, k, want_ts=(not last) or want_last_ts))
            hops.append(hop)
            nodes, q_ts = hop.nbr, hop.ts
        return hops
