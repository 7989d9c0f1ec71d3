"""SchedulerSession -- the reference's session API (session.py:25-439), CTDG
(``graph_mode == "ctdg"``, ``ctdg.pipeline: online``) path.

Lifecycle: ``from_config`` -> ``prepare_data`` -> ``build_runtime`` ->
``run_epoch("train")`` / ``run_epoch("val")`` / ``evaluate`` / ``predict`` ->
``save_checkpoint`` / ``load_checkpoint``. The snapshot (DTDG) and chunk
backends of the reference are not part of this build.
"""
from __future__ import annotations

import time
from pathlib import Path
from typing import Any

from starry_unigraph.backends.ctdg.preprocess import CTDGPreprocessor, load_prepared_from_disk
from starry_unigraph.backends.ctdg.runtime.session import CTDGSession
from starry_unigraph.config.schema import detect_graph_mode, load_config, validate_config
from starry_unigraph.types import (DistributedContext, PredictionResult, PreparedArtifacts, RuntimeBundle,
                                   SessionContext)


def build_distributed_context(config: dict) -> DistributedContext:
    d = config.get("dist", {})
    return DistributedContext(backend=str(d.get("backend", "nccl")), world_size=int(d.get("world_size", 1)),
                              rank=int(d.get("rank", 0)), local_rank=int(d.get("local_rank", 0)),
                              local_world_size=int(d.get("local_world_size", 1)),
                              master_addr=str(d.get("master_addr", "127.0.0.1")),
                              master_port=int(d.get("master_port", 29500)))


class SchedulerSession:
    def __init__(self, session_ctx: SessionContext, model_spec: Any = None, task_adapter: Any = None):
        self.ctx = session_ctx
        self.model_spec = model_spec
        self.task_adapter = task_adapter
        self.current_epoch = 0
        self.global_step = 0
        self.runtime = RuntimeBundle()
        self.ctdg_session: CTDGSession | None = None
        self.prepared: PreparedArtifacts | None = None
        self._events = None

    @classmethod
    def from_config(cls, config_or_path: str | Path | dict[str, Any], dataset_path: str | Path | None = None,
                    overrides: dict[str, Any] | None = None) -> "SchedulerSession":
        config = load_config(config_or_path, overrides=overrides)
        warnings = validate_config(config)
        ctx = SessionContext(config=config, project_root=Path.cwd(),
                             dataset_path=Path(dataset_path).expanduser().resolve() if dataset_path else None,
                             artifact_root=(Path("artifacts") / config["data"]["name"]).resolve(),
                             dist=build_distributed_context(config), warnings=warnings)
        return cls(session_ctx=ctx)

    def with_events(self, events) -> "SchedulerSession":
        """Use an in-memory RawTemporalEvents instead of loading from disk."""
        self._events = events
        return self

    def prepare_data(self) -> PreparedArtifacts:
        if detect_graph_mode(self.ctx.config) != "ctdg":
            raise ValueError("this build implements graph_mode 'ctdg' only")
        self.prepared = CTDGPreprocessor().run(self.ctx)
        self.ctx.prepared_artifacts = self.prepared
        return self.prepared

    def build_runtime(self) -> RuntimeBundle:
        if self.prepared is None:
            try:
                self.prepared = load_prepared_from_disk(self.ctx.artifact_root)
            except FileNotFoundError:
                self.prepared = self.prepare_data()
        self.ctx.prepared_artifacts = self.prepared
        if self.prepared.provider_meta.get("graph_mode") != "ctdg":
            raise ValueError(f"Unknown graph_mode: {self.prepared.provider_meta.get('graph_mode')}")
        self.ctdg_session = CTDGSession()
        self.ctdg_session.prepared = self.prepared
        self.ctdg_session.build_runtime(self.ctx, events=self._events)
        self.runtime = self.ctdg_session._runtime
        return self.runtime

    def run_epoch(self, split: str = "train") -> dict[str, Any]:
        """session.py:223-269 (CTDG branch)."""
        assert self.ctdg_session is not None, "Call build_runtime() first"
        it = self.ctdg_session.iter_train(self.ctx) if split == "train" else self.ctdg_session.iter_eval(self.ctx,
                                                                                                         split)
        t0 = time.perf_counter()
        outputs = []
        for batch in it:
            if split == "train":
                outputs.append(self.ctdg_session.train_step(batch))
                self.global_step += 1
            else:
                outputs.append(self.ctdg_session.eval_step(batch))
        elapsed = time.perf_counter() - t0
        self.ctdg_session.online_runtime.check_sync()
        if split == "train":
            self.current_epoch += 1
        losses = [float(o["loss"]) for o in outputs if "loss" in o]
        acc: dict[str, list[float]] = {}
        for o in outputs:
            for k, v in o.get("meta", {}).get("metrics", {}).items():
                acc.setdefault(k, []).append(float(v))
        steps = len(losses) if split != "train" else len(outputs)
        loss_sum = float(sum(losses))
        return {"split": split, "steps": steps, "local_steps": steps, "loss": loss_sum / steps if steps else 0.0,
                "local_loss": loss_sum / steps if steps else 0.0,
                "metrics": {k: float(sum(v) / len(v)) for k, v in acc.items() if v},
                "elapsed_s": elapsed, "local_elapsed_s": elapsed, "outputs": outputs}

    def run_task(self) -> dict[str, Any]:
        self.build_runtime()
        train, evals = [], []
        t0 = time.perf_counter()
        for epoch in range(int(self.ctx.config["train"]["epochs"])):
            train.append(self.run_epoch("train"))
            if (epoch + 1) % int(self.ctx.config["train"].get("eval_interval", 1)) == 0:
                evals.append(self.run_epoch("val"))
        return {"epochs": self.current_epoch, "train": train, "eval": evals,
                "train_total_s": sum(t["elapsed_s"] for t in train),
                "train_total_local_s": sum(t["local_elapsed_s"] for t in train),
                "run_task_total_s": time.perf_counter() - t0, "warnings": self.ctx.warnings}

    def evaluate(self, split: str = "test") -> dict[str, Any]:
        return self.run_epoch(split=split)

    def predict(self, split: str = "test") -> PredictionResult:
        assert self.ctdg_session is not None, "Call build_runtime() first"
        preds, targets = [], []
        for batch in self.ctdg_session.iter_predict(self.ctx, split=split):
            out = self.ctdg_session.predict_step(batch)
            preds.extend(out.get("predictions", []))
            targets.extend(out.get("targets", []) or [])
        return PredictionResult(predictions=preds, targets=targets or None,
                                meta={"split": split, "graph_mode": "ctdg"})

    def save_checkpoint(self, path: str | Path) -> Path:
        assert self.ctdg_session is not None, "Call build_runtime() first"
        self.ctdg_session.save_checkpoint(path)
        return Path(path)

    def load_checkpoint(self, path: str | Path) -> dict[str, Any]:
        assert self.ctdg_session is not None, "Call build_runtime() first"
        self.ctdg_session.load_checkpoint(path)
        return {}
