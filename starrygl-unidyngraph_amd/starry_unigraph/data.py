"""Raw temporal event loading (the reference's data/raw_temporal.py:175-329,
CTDG part).

Formats, selected by ``config["data"]["format"]``:
  * ``mock``      -- the reference's mock ring (data/raw_temporal.py:175-193):
                     >=16 events i -> i+1 over <=128 nodes, ts = i, 1-d ones.
  * ``synthetic`` -- seeded generators of starry_unigraph.synth, configured by
                     ``config["data"]["synthetic"]`` ({"kind": "bipartite" |
                     "unipartite", ...generator kwargs}).
  * ``auto``/``csv`` -- ``<root>/<name>/edges.csv`` with columns src, dst and
                     time (or ts, or the last column), plus an optional
                     ``edge_features.pt`` tensor (data/raw_temporal.py:200-252);
                     without one, edge features are ones [E, 1].
``write_ctdg_csv`` writes a stream in that on-disk format.
"""
from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path
from typing import Any

import numpy as np
import torch


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
    node_temporal_features: Any = None


def _mock_events(dataset_name: str, config: dict[str, Any]) -> RawTemporalEvents:
    snaps = max(1, int(config.get("train", {}).get("snaps", 8) or 8))
    e = max(16, snaps * 4)
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


def _load_ctdg_csv(dataset_dir: Path) -> RawTemporalEvents | None:
    edges = dataset_dir / "edges.csv"
    if not edges.exists():
        return None
    import pandas as pd
    frame = pd.read_csv(edges)
    if frame.empty:
        return RawTemporalEvents(torch.empty(0, dtype=torch.long), torch.empty(0, dtype=torch.long),
                                 torch.empty(0), torch.empty(0), torch.empty(0, 1), 0, 0, str(edges))
    src = torch.as_tensor(frame["src"].to_numpy(dtype="int64"))
    dst = torch.as_tensor(frame["dst"].to_numpy(dtype="int64"))
    tcol = "time" if "time" in frame.columns else ("ts" if "ts" in frame.columns else frame.columns[-1])
    ts = torch.as_tensor(frame[tcol].to_numpy(dtype="float32"))
    wcol = "w" if "w" in frame.columns else ("weight" if "weight" in frame.columns else None)
    weight = torch.ones(src.numel()) if wcol is None else torch.as_tensor(frame[wcol].to_numpy(dtype="float32"))
    feat_path = dataset_dir / "edge_features.pt"
    if feat_path.exists():
        ef = torch.load(feat_path, map_location="cpu", weights_only=True).float()
        if ef.dim() == 1:
            ef = ef.view(-1, 1)
    else:
        ef = torch.ones(src.numel(), 1)
    n = int(max(int(src.max()), int(dst.max())) + 1)
    return RawTemporalEvents(src, dst, ts, weight, ef, n, int(src.numel()), str(edges))


def load_raw_temporal_events(root: Path | str, dataset_name: str, config: dict[str, Any]) -> RawTemporalEvents:
    fmt = str(config.get("data", {}).get("format", "auto")).lower()
    if fmt == "mock":
        return _mock_events(dataset_name, config)
    if fmt == "synthetic":
        return _synthetic_events(config)
    ev = _load_ctdg_csv(Path(root).expanduser().resolve() / dataset_name)
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
