"""Config loading: YAML deep-merged over the defaults (config/schema.py:53-150
in the reference, CTDG part)."""
from __future__ import annotations

import copy
from pathlib import Path
from typing import Any

import yaml

_DEFAULT = Path(__file__).with_name("default.yaml")
CTDG_FAMILIES = {"tgn", "jodie", "dyrep", "tgat", "apan"}
REQUIRED_PATHS = ("model.family", "model.hidden_dim", "data.name", "train.batch_size", "runtime.device",
                  "sampling.neighbor_limit", "sampling.history", "sampling.strategy")


def _merge(base: dict, over: dict) -> dict:
    out = copy.deepcopy(base)
    for k, v in (over or {}).items():
        if isinstance(v, dict) and isinstance(out.get(k), dict):
            out[k] = _merge(out[k], v)
        else:
            out[k] = copy.deepcopy(v)
    return out


def load_config(config_or_path: str | Path | dict[str, Any], overrides: dict[str, Any] | None = None) -> dict:
    with open(_DEFAULT) as f:
        base = yaml.safe_load(f)
    if isinstance(config_or_path, dict):
        user = config_or_path
    else:
        with open(config_or_path) as f:
            user = yaml.safe_load(f) or {}
    cfg = _merge(base, user)
    if overrides:
        cfg = _merge(cfg, overrides)
    cfg.setdefault("data", {}).setdefault("graph_mode", detect_graph_mode(cfg))
    return cfg


def detect_graph_mode(cfg: dict) -> str:
    mode = cfg.get("data", {}).get("graph_mode")
    if mode:
        return str(mode)
    fam = str(cfg.get("model", {}).get("family", "")).lower()
    return "ctdg" if fam in CTDG_FAMILIES else "dtdg"


def _get(cfg: dict, path: str):
    cur: Any = cfg
    for part in path.split("."):
        if not isinstance(cur, dict) or part not in cur:
            raise KeyError(path)
        cur = cur[part]
    return cur


def validate_config(cfg: dict) -> list[str]:
    """Raises on missing required keys; returns warnings."""
    for p in REQUIRED_PATHS:
        _get(cfg, p)
    warnings = []
    if detect_graph_mode(cfg) != "ctdg":
        raise ValueError("this build implements the CTDG (continuous-time) path only")
    if str(cfg.get("ctdg", {}).get("pipeline", "online")) != "online":
        warnings.append("ctdg.pipeline is not 'online'; the online pipeline is used")
    if int(cfg.get("dist", {}).get("world_size", 1)) != 1:
        warnings.append("dist.world_size > 1 is not built; running on one GPU")
    return warnings
