"""Thin CTDG session (backends/ctdg/runtime/session.py:16-93 in the reference)."""
from __future__ import annotations

from pathlib import Path
from typing import Any

import torch

from starry_unigraph.backends.ctdg.preprocess import CTDGPreprocessor
from starry_unigraph.types import PreparedArtifacts, RuntimeBundle, SessionContext

from .factory import build_ctdg_runtime
from .runtime import CTDGOnlineRuntime


class CTDGSession:
    def __init__(self) -> None:
        self.online_runtime: CTDGOnlineRuntime | None = None
        self.prepared: PreparedArtifacts | None = None
        self._runtime: RuntimeBundle = RuntimeBundle()

    def prepare_data(self, session_ctx: SessionContext) -> PreparedArtifacts:
        self.prepared = CTDGPreprocessor().run(session_ctx)
        session_ctx.prepared_artifacts = self.prepared
        return self.prepared

    def build_runtime(self, session_ctx: SessionContext, events=None) -> None:
        if self.prepared is not None:
            session_ctx.prepared_artifacts = self.prepared
        self.online_runtime, self._runtime = build_ctdg_runtime(session_ctx, events=events)

    def _iter(self, session_ctx: SessionContext, split: str):
        assert self.online_runtime is not None
        yield from self.online_runtime.iter_batches(split=split,
                                                    batch_size=int(session_ctx.config["train"]["batch_size"]))

    def iter_train(self, session_ctx: SessionContext):
        yield from self._iter(session_ctx, "train")

    def iter_eval(self, session_ctx: SessionContext, split: str = "val"):
        yield from self._iter(session_ctx, split)

    def iter_predict(self, session_ctx: SessionContext, split: str = "test"):
        yield from self._iter(session_ctx, split)

    def train_step(self, batch: Any) -> dict[str, Any]:
        assert self.online_runtime is not None
        return self.online_runtime.train_step(batch)

    def eval_step(self, batch: Any) -> dict[str, Any]:
        assert self.online_runtime is not None
        return self.online_runtime.eval_step(batch, split=batch.split)

    def predict_step(self, batch: Any) -> dict[str, Any]:
        assert self.online_runtime is not None
        return self.online_runtime.predict_step(batch)

    def save_checkpoint(self, path: str | Path) -> None:
        """session.py:78-85: model and updater state dicts."""
        assert self.online_runtime is not None
        model = self.online_runtime.model
        ckpt: dict[str, Any] = {"model": (model.module if hasattr(model, "module") else model).state_dict()}
        if self.online_runtime.memory_updater is not None:
            ckpt["memory_updater"] = self.online_runtime.memory_updater.state_dict()
        torch.save(ckpt, str(path))

    def load_checkpoint(self, path: str | Path) -> None:
        assert self.online_runtime is not None
        ckpt = torch.load(str(path), map_location="cpu", weights_only=True)
        model = self.online_runtime.model
        core = model.module if hasattr(model, "module") else model
        with torch.no_grad():
            for name, t in ckpt["model"].items():
                core.state_dict()[name].copy_(t)        # in place: parameters are views of the optimizer's buffer
            if self.online_runtime.memory_updater is not None and "memory_updater" in ckpt:
                self.online_runtime.memory_updater.load_state_dict(ckpt["memory_updater"])
                self.online_runtime.memory_updater.kernel_weights()   # refresh bf16 copies in place
