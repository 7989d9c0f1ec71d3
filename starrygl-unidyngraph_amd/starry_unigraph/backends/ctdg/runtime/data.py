"""CTDG event stream and batching (backends/ctdg/runtime/data.py:22-239 in
the reference): contiguous time-ordered batches of one split, and the
per-split sampler graph (every event before the split's end, so it includes
the current batch -- data.py:196-231)."""
from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path
from typing import Iterator

import numpy as np
import torch

from starry_unigraph.data import RawTemporalEvents, load_raw_temporal_events
from starry_unigraph.runtime._split import normalize_split_ratio, split_bounds


@dataclass
class CTDGDataBatch:
    index: int
    split: str
    event_ids: torch.Tensor
    src: torch.Tensor
    dst: torch.Tensor
    ts: torch.Tensor
    edge_feat: torch.Tensor
    src_node_feat: torch.Tensor | None = None
    dst_node_feat: torch.Tensor | None = None

    @property
    def size(self) -> int:
        return int(self.src.numel())

    @property
    def is_empty(self) -> bool:
        return self.size == 0

    @property
    def start(self) -> int:
        """First event id when the batch is a contiguous range, else -1
        (computed once: batches are immutable)."""
        st = self.__dict__.get("_start")
        if st is None:
            ids = self.event_ids
            if ids.numel() == 0:
                st = 0
            elif ids.numel() == 1 or bool((ids[1:] - ids[:-1]).eq(1).all()):
                st = int(ids[0])
            else:   # out-of-order or gapped ids: the step gathers the batch's own events
                st = -1
            self.__dict__["_start"] = st
        return st


class TGTemporalDataset:
    def __init__(self, root: str | Path, name: str, split_ratio: dict[str, float] | None = None,
                 config: dict | None = None, events: RawTemporalEvents | None = None):
        self.root = Path(root).expanduser().resolve() / name
        cfg = dict(config or {})
        cfg.setdefault("data", {})
        cfg["data"] = dict(cfg["data"])
        cfg["data"]["split_ratio"] = split_ratio or cfg["data"].get("split_ratio")
        raw = events if events is not None else load_raw_temporal_events(Path(root), name, cfg)
        self.event_ids = torch.arange(raw.num_edges, dtype=torch.long)
        self.src = raw.src.long()
        self.dst = raw.dst.long()
        self.ts = raw.ts.float()
        self.num_nodes = int(raw.num_nodes)
        self.num_edges = int(raw.num_edges)
        self.edge_feat = raw.edge_feat.float()
        self.edge_feat_dim = int(self.edge_feat.size(-1))
        self.node_temporal_features = getattr(raw, "node_temporal_features", None)
        nf = self.node_temporal_features
        self.node_feat_dim = 0 if nf is None else nf.dim
        self._node_hist = self._build_node_feat_history()
        self.split_ratio = normalize_split_ratio(cfg["data"].get("split_ratio"))
        self._split_cache: dict[str, torch.Tensor] = {}
        self._sampler_cache: dict[str, dict[str, torch.Tensor]] = {}
        self._device_cache: dict[str, dict[str, torch.Tensor]] = {}
        self.node_parts = None
        self.edge_parts = None
        self.partition_rank = 0
        self.partition_world_size = 1

    def configure_partition(self, *, node_parts, edge_parts, rank: int, world_size: int) -> None:
        self.node_parts, self.edge_parts = node_parts, edge_parts
        self.partition_rank, self.partition_world_size = rank, world_size

    def split_event_ids(self, split: str) -> torch.Tensor:
        ids = self._split_cache.get(split)
        if ids is None:
            a, b = split_bounds(self.num_edges, split, self.split_ratio)
            ids = self._split_cache[split] = torch.arange(a, b, dtype=torch.long)
        return ids

    def inter_event_stats(self, split: str = "train") -> tuple[float, float]:
        """(shift, scale) for the time-projection embedding: the mean of the
        times between a node's consecutive events (either endpoint) within
        the split, and 1 / their standard deviation (1 when undefined)."""
        ids = self.split_event_ids(split)
        if ids.numel() < 2:
            return 0.0, 1.0
        a, b = int(ids[0]), int(ids[-1]) + 1
        nodes = torch.cat([self.src[a:b], self.dst[a:b]]).numpy()
        ts = torch.cat([self.ts[a:b], self.ts[a:b]]).double().numpy()
        order = np.lexsort((ts, nodes))
        n, t = nodes[order], ts[order]
        same = n[1:] == n[:-1]
        gaps = (t[1:] - t[:-1])[same]
        if gaps.size < 2:
            return 0.0, 1.0
        sd = float(gaps.std())
        return float(gaps.mean()), (1.0 / sd if sd > 0 else 1.0)

    def _build_node_feat_history(self):
        """data.py:128-140: each node's feature rows in time order (rows of a
        node with equal times keep their order in the time-sorted table), as
        one array sorted by (node, time)."""
        nf = self.node_temporal_features
        if nf is None or nf.size == 0 or nf.dim == 0:
            return None
        ids, ts = nf.node_ids.numpy(), nf.ts.float().numpy()
        order = np.lexsort((ts, ids))   # stable: node, then time
        return ids[order], ts[order], nf.values.float()[torch.from_numpy(order)]

    def lookup_node_features(self, node_ids: torch.Tensor, ts: torch.Tensor) -> torch.Tensor | None:
        """data.py:142-157: for each (node, t) the node's latest feature row
        with time <= t (the last of equal times), zeros when it has none;
        None without node features."""
        if self.node_feat_dim <= 0 or self._node_hist is None:
            return None
        h_ids, h_ts, h_vals = self._node_hist
        q = node_ids.long().numpy()
        t = ts.float().numpy()
        lo = np.searchsorted(h_ids, q, side="left")
        hi = np.searchsorted(h_ids, q, side="right")
        # upper_bound of t inside [lo, hi), all queries at once
        a, b = lo.copy(), hi.copy()
        while True:
            act = a < b
            if not act.any():
                break
            mid = (a + b) // 2
            le = np.zeros_like(act)
            le[act] = h_ts[mid[act]] <= t[act]
            a = np.where(act & le, mid + 1, a)
            b = np.where(act & ~le, mid, b)
        idx = a - 1
        out = torch.zeros(q.size, self.node_feat_dim, dtype=torch.float32)
        hit = idx >= lo
        if hit.any():
            out[torch.from_numpy(np.nonzero(hit)[0])] = h_vals[torch.from_numpy(idx[hit])]
        return out

    def iter_batches(self, split: str, batch_size: int) -> Iterator[CTDGDataBatch]:
        """data.py:161-194: consecutive slices of the split."""
        ids = self.split_event_ids(split)
        step = batch_size * (self.partition_world_size if (self.partition_world_size > 1 and
                                                            self.edge_parts is not None) else 1)
        sharded = self.partition_world_size > 1 and self.edge_parts is not None
        base = int(ids[0]) if ids.numel() else 0
        for bi, start in enumerate(range(0, int(ids.numel()), step)):
            ev = ids[start:start + step]
            if sharded:
                ev = ev[self.edge_parts[ev] == self.partition_rank]
                s, d, t = self.src[ev], self.dst[ev], self.ts[ev]
                yield CTDGDataBatch(index=bi, split=split, event_ids=ev, src=s, dst=d, ts=t,
                                    edge_feat=self.edge_feat[ev], src_node_feat=self.lookup_node_features(s, t),
                                    dst_node_feat=self.lookup_node_features(d, t))
            else:  # splits are contiguous event ranges: views, no copies
                a, b = base + start, base + start + ev.numel()
                s, d, t = self.src[a:b], self.dst[a:b], self.ts[a:b]
                batch = CTDGDataBatch(index=bi, split=split, event_ids=ev, src=s, dst=d, ts=t,
                                      edge_feat=self.edge_feat[a:b], src_node_feat=self.lookup_node_features(s, t),
                                      dst_node_feat=self.lookup_node_features(d, t))
                batch.__dict__["_start"] = a   # contiguous by construction (CTDGDataBatch.start)
                yield batch

    def sampler_graph(self, split: str) -> dict[str, torch.Tensor]:
        """data.py:196-231: train = [0, train_end); val = [0, val_end);
        test = [0, test_end); ts is int64 of the float32 times (truncation)."""
        g = self._sampler_cache.get(split)
        if g is not None:
            return g
        _, train_end = split_bounds(self.num_edges, "train", self.split_ratio)
        _, val_end = split_bounds(self.num_edges, "val", self.split_ratio)
        _, test_end = split_bounds(self.num_edges, "test", self.split_ratio)
        end = {"train": train_end, "val": val_end, "test": test_end}.get(split)
        if end is None:
            raise KeyError(f"Unsupported CTDG split: {split}")
        idx = torch.arange(0, end, dtype=torch.long)
        g = {"row": self.src[idx], "col": self.dst[idx], "eid": idx, "ts": self.ts[idx].long()}
        self._sampler_cache[split] = g
        return g

    def device_arrays(self, device) -> dict[str, torch.Tensor]:
        """The whole stream resident in HBM (uploaded once)."""
        key = str(device)
        d = self._device_cache.get(key)
        if d is None:
            d = {"src": self.src.to(device), "dst": self.dst.to(device), "ts": self.ts.to(device),
                 "edge_feat": self.edge_feat.to(device).contiguous()}
            self._device_cache[key] = d
        return d

    def describe(self) -> dict[str, int]:
        return {"num_nodes": self.num_nodes, "num_edges": self.num_edges, "edge_feat_dim": self.edge_feat_dim,
                "node_feat_dim": self.node_feat_dim}
