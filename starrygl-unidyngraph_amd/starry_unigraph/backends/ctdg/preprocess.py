"""Artifact manifest for the CTDG path (backends/ctdg/preprocess.py:15-137 in
the reference, single rank: no partitioning)."""
from __future__ import annotations

import json
from pathlib import Path

from starry_unigraph.types import PreparedArtifacts, SessionContext

ARTIFACT_VERSION = 1


class CTDGPreprocessor:
    def run(self, session_ctx: SessionContext) -> PreparedArtifacts:
        root = Path(session_ctx.artifact_root)
        meta_dir = root / "meta"
        meta_dir.mkdir(parents=True, exist_ok=True)
        cfg = session_ctx.config
        meta = {"graph_mode": "ctdg", "artifact_version": ARTIFACT_VERSION, "num_parts": 1,
                "dataset": cfg["data"]["name"], "feature_route_plan": {"route_type": cfg["graph"]["route"],
                                                                      "world_size": 1}}
        path = meta_dir / "artifacts.json"
        path.write_text(json.dumps(meta, indent=2))
        return PreparedArtifacts(meta_path=path, directories={"meta": meta_dir}, provider_meta=meta)


def load_prepared_from_disk(artifact_root: Path) -> PreparedArtifacts:
    path = Path(artifact_root) / "meta" / "artifacts.json"
    if not path.exists():
        raise FileNotFoundError(f"Missing prepared artifacts: {path} (call prepare_data() first)")
    meta = json.loads(path.read_text())
    if int(meta.get("artifact_version", -1)) != ARTIFACT_VERSION:
        raise ValueError(f"artifact_version mismatch: {meta.get('artifact_version')} != {ARTIFACT_VERSION}")
    return PreparedArtifacts(meta_path=path, directories={"meta": path.parent}, provider_meta=meta)
