"""Raw temporal event loading (the reference's data/raw_temporal.py, CTDG part).

Formats, selected by ``config["data"]["format"]``:
  * ``mock``      -- the reference's mock ring (data/raw_temporal.py:175-193):
                     >=16 events i -> i+1 over <=128 nodes, ts = i, 1-d ones.
  * ``synthetic`` -- seeded generators of starry_unigraph.synth, configured by
                     ``config["data"]["synthetic"]`` ({"kind": "bipartite" |
                     "unipartite", ...generator kwargs}).
  * ``auto``/``csv`` -- the reference's chain (raw_temporal.py:317-329):
      1. ``<root>/<name>/edges.csv`` with columns src, dst and time (or ts, or
         the last column), optional weight column w / weight, plus an
         optional ``edge_features.pt`` tensor (ones [E, 1] without one);
         raw_temporal.py:198-252;
      2. else an edge list ``<name>.edges`` / ``edges.txt`` / ``edges.csv``
         (comma- or whitespace-separated, ``%`` / ``#`` comment lines; rows
         "u v t", "u v w t" or "idx u v t ..."), events stably sorted by time
         and node ids remapped to 0..N-1 in sorted order (node-feature ids
         included), edge features ones [E, 1]; raw_temporal.py:255-314;
      3. else the mock ring.
    Both file formats also read node temporal features from
    ``node_temporal_features.csv`` / ``node_features.csv`` (a node column
    node_id / node / id, an optional time column time / ts / timestamp, every
    other numeric column a feature; rows stably sorted by time), which raise
    num_nodes to cover their ids (raw_temporal.py:11-163).
``write_ctdg_csv`` writes a stream in the edges.csv layout.
"""
from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path
from typing import Any

import numpy as np
import torch

NODE_FEATURE_FILES = ("node_temporal_features.csv", "node_features.csv")


@dataclass
class NodeTemporalFeatureTable:
    """raw_temporal.py:17-31: per-row node id, time and feature values,
    stably sorted by time."""
    node_ids: torch.Tensor   # int64 [M]
    ts: torch.Tensor         # float32 [M]
    values: torch.Tensor     # float32 [M, dim]
    feature_names: tuple[str, ...]
    source: str

    @property
    def dim(self) -> int:
        return int(self.values.size(-1)) if self.values.dim() == 2 else 0

    @property
    def size(self) -> int:
        return int(self.node_ids.numel())


@dataclass
class RawTemporalEvents:
    src: torch.Tensor        # int64 [E]
    dst: torch.Tensor        # int64 [E]
    ts: torch.Tensor         # float32 [E]
    weight: torch.Tensor     # float32 [E]
    edge_feat: torch.Tensor  # float32 [E, F]
    num_nodes: int
    num_edges: int
    source: str = ""
    node_temporal_features: NodeTemporalFeatureTable | None = None


def _mock_events(dataset_name: str, config: dict[str, Any]) -> RawTemporalEvents:
    try:
        snaps = int(config.get("train", {}).get("snaps", 8))
    except (TypeError, ValueError):
        snaps = 8
    e = max(16, max(1, snaps) * 4)
    n = max(8, min(128, e // 2))
    idx = torch.arange(e, dtype=torch.long)
    return RawTemporalEvents(src=idx % n, dst=(idx + 1) % n, ts=idx.float(), weight=torch.ones(e),
                             edge_feat=torch.ones(e, 1), num_nodes=n, num_edges=e, source=f"mock:{dataset_name}")


def _synthetic_events(config: dict[str, Any]) -> RawTemporalEvents:
    from starry_unigraph import synth
    spec = dict(config.get("data", {}).get("synthetic", {}) or {})
    kind = spec.pop("kind", "unipartite")
    gen = {"bipartite": synth.bipartite_stream, "unipartite": synth.unipartite_stream}.get(kind)
    if gen is None:
        raise KeyError(f"unknown synthetic stream kind {kind!r}")
    s = gen(**spec)
    return from_stream(s, source=f"synthetic:{kind}")


def from_stream(s, source: str = "synthetic") -> RawTemporalEvents:
    e = s.num_events
    return RawTemporalEvents(src=torch.from_numpy(np.ascontiguousarray(s.src)),
                             dst=torch.from_numpy(np.ascontiguousarray(s.dst)),
                             ts=torch.from_numpy(np.ascontiguousarray(s.ts, dtype=np.float32)),
                             weight=torch.ones(e), edge_feat=torch.from_numpy(np.ascontiguousarray(s.edge_feat)),
                             num_nodes=int(s.num_nodes), num_edges=e, source=source)


# --------------------------------------------------------------------------- node temporal features
def _load_node_temporal_features(dataset_dir: Path) -> NodeTemporalFeatureTable | None:
    """raw_temporal.py:85-122."""
    path = next((dataset_dir / n for n in NODE_FEATURE_FILES if (dataset_dir / n).exists()), None)
    if path is None:
        return None
    import pandas as pd
    frame = pd.read_csv(path)
    if frame.empty:
        return NodeTemporalFeatureTable(torch.empty(0, dtype=torch.long), torch.empty(0),
                                        torch.empty(0, 0), (), str(path))
    node_col = next((c for c in ("node_id", "node", "id") if c in frame.columns), None)
    if node_col is None:
        raise ValueError(f"Node feature file {path} must contain one of: node_id, node, id")
    ts_col = next((c for c in ("time", "ts", "timestamp") if c in frame.columns), None)
    reserved = {node_col} | ({ts_col} if ts_col else set())
    cols = [c for c in frame.columns if c not in reserved and pd.api.types.is_numeric_dtype(frame[c])]
    if not cols:
        raise ValueError(f"Node feature file {path} must contain at least one numeric feature column")
    ids = frame[node_col].to_numpy(dtype=np.int64)
    ts = frame[ts_col].to_numpy(dtype=np.float32) if ts_col else np.zeros(len(ids), dtype=np.float32)
    vals = frame[cols].to_numpy(dtype=np.float32)
    order = np.argsort(ts, kind="stable")
    return NodeTemporalFeatureTable(torch.from_numpy(ids[order].copy()), torch.from_numpy(ts[order].copy()),
                                    torch.from_numpy(np.ascontiguousarray(vals[order])), tuple(cols), str(path))


def _remap_node_features(table: NodeTemporalFeatureTable | None, uniq: np.ndarray):
    """raw_temporal.py:125-163: rows whose node is in ``uniq`` (sorted), ids
    replaced by their rank there; other rows dropped."""
    if table is None or table.size == 0:
        return table
    ids = table.node_ids.numpy()
    pos = np.searchsorted(uniq, ids)
    keep = (pos < uniq.size) & (uniq[np.minimum(pos, uniq.size - 1)] == ids)
    k = torch.from_numpy(np.nonzero(keep)[0])
    return NodeTemporalFeatureTable(torch.from_numpy(pos[keep].astype(np.int64)), table.ts[k].clone(),
                                    table.values[k].clone(), table.feature_names, table.source)


# --------------------------------------------------------------------------- edges.csv
def _load_ctdg_csv(dataset_dir: Path) -> RawTemporalEvents | None:
    """raw_temporal.py:198-252."""
    edges = dataset_dir / "edges.csv"
    if not edges.exists():
        return None
    import pandas as pd
    nf = _load_node_temporal_features(dataset_dir)
    frame = pd.read_csv(edges)
    if frame.empty:
        return RawTemporalEvents(torch.empty(0, dtype=torch.long), torch.empty(0, dtype=torch.long),
                                 torch.empty(0), torch.empty(0), torch.empty(0, 1), max(nf.size if nf else 0, 0), 0,
                                 str(edges), nf)
    src = torch.as_tensor(frame["src"].to_numpy(dtype="int64"))
    dst = torch.as_tensor(frame["dst"].to_numpy(dtype="int64"))
    tcol = "time" if "time" in frame.columns else ("ts" if "ts" in frame.columns else frame.columns[-1])
    ts = torch.as_tensor(frame[tcol].to_numpy(dtype="float32"))
    wcol = "w" if "w" in frame.columns else ("weight" if "weight" in frame.columns else None)
    weight = torch.ones(src.numel()) if wcol is None else torch.as_tensor(frame[wcol].to_numpy(dtype="float32"))
    n = int(max(int(src.max()), int(dst.max())) + 1)
    if nf is not None and nf.size > 0:
        n = max(n, int(nf.node_ids.max()) + 1)
    feat_path = dataset_dir / "edge_features.pt"
    if feat_path.exists():
        ef = torch.load(feat_path, map_location="cpu", weights_only=True).float()
        if ef.dim() == 1:
            ef = ef.view(-1, 1)
    else:
        ef = torch.ones(src.numel(), 1)
    return RawTemporalEvents(src, dst, ts, weight, ef, n, int(src.numel()), str(edges), nf)


# --------------------------------------------------------------------------- edge lists
def _parse_edge_row(parts: list[str]) -> tuple[int, int, float, float] | None:
    """raw_temporal.py:54-66: "u v t", "u v w t", or "idx u v t ..." (w = 1)."""
    if len(parts) == 3:
        u, v, t = parts
        w = "1"
    elif len(parts) == 4:
        u, v, w, t = parts
    elif len(parts) >= 5:
        u, v, t = parts[1], parts[2], parts[3]
        w = "1"
    else:
        return None
    return int(float(u)), int(float(v)), float(t), float(w)


def _load_from_edge_file(dataset_dir: Path, dataset_name: str) -> RawTemporalEvents | None:
    """raw_temporal.py:255-314."""
    path = next((p for p in (dataset_dir / f"{dataset_name}.edges", dataset_dir / "edges.txt",
                             dataset_dir / "edges.csv") if p.exists()), None)
    if path is None:
        return None
    nf = _load_node_temporal_features(dataset_dir)
    rows = []
    with path.open("r", encoding="utf-8") as fh:
        for raw in fh:
            line = raw.strip()
            if not line or line[0] in "%#":
                continue
            parts = [p.strip() for p in line.split(",")] if "," in line else line.split()
            r = _parse_edge_row(parts)
            if r is not None:
                rows.append(r)
    if not rows:
        return None
    src = np.fromiter((r[0] for r in rows), dtype=np.int64, count=len(rows))
    dst = np.fromiter((r[1] for r in rows), dtype=np.int64, count=len(rows))
    ts = np.fromiter((r[2] for r in rows), dtype=np.float64, count=len(rows)).astype(np.float32)
    w = np.fromiter((r[3] for r in rows), dtype=np.float64, count=len(rows)).astype(np.float32)
    order = np.argsort(ts, kind="stable")
    src, dst, ts, w = src[order], dst[order], ts[order], w[order]
    ids = [src, dst] + ([nf.node_ids.numpy()] if nf is not None and nf.size > 0 else [])
    uniq = np.unique(np.concatenate(ids))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    return RawTemporalEvents(t(np.searchsorted(uniq, src).astype(np.int64)),
                             t(np.searchsorted(uniq, dst).astype(np.int64)), t(ts), t(w),
                             torch.ones(len(rows), 1), int(uniq.size), len(rows), str(path),
                             _remap_node_features(nf, uniq))


def load_raw_temporal_events(root: Path | str, dataset_name: str, config: dict[str, Any]) -> RawTemporalEvents:
    fmt = str(config.get("data", {}).get("format", "auto")).lower()
    if fmt == "mock":
        return _mock_events(dataset_name, config)
    if fmt == "synthetic":
        return _synthetic_events(config)
    d = Path(root).expanduser().resolve() / dataset_name
    ev = _load_ctdg_csv(d)
    if ev is None:
        ev = _load_from_edge_file(d, dataset_name)
    if ev is None:
        return _mock_events(dataset_name, config)
    return ev


def write_ctdg_csv(dataset_dir: Path | str, src, dst, ts, edge_feat=None) -> Path:
    """Write edges.csv (src,dst,time) and edge_features.pt in the layout the
    loader above (and the reference's) reads."""
    import pandas as pd
    d = Path(dataset_dir)
    d.mkdir(parents=True, exist_ok=True)
    pd.DataFrame({"src": np.asarray(src, dtype=np.int64), "dst": np.asarray(dst, dtype=np.int64),
                  "time": np.asarray(ts, dtype=np.float32)}).to_csv(d / "edges.csv", index=False)
    if edge_feat is not None:
        torch.save(torch.as_tensor(np.asarray(edge_feat, dtype=np.float32)), d / "edge_features.pt")
    return d / "edges.csv"
