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
        """session.py:87-93: strict state-dict loads of the model and the
        updater. The model's tensors are copied in place (its parameters are
        views of the fused optimizer's flat buffer); the next step is ordered
        after the copies."""
        rt = self.online_runtime
        assert rt is not None
        ckpt = torch.load(str(path), map_location="cpu", weights_only=True)
        model = rt.model
        core = model.module if hasattr(model, "module") else model
        _check_state_keys(type(core).__name__, core.state_dict(), ckpt["model"])
        with torch.no_grad():
            own = core.state_dict()
            for name, t in ckpt["model"].items():
                own[name].copy_(t)
            if rt.memory_updater is not None and "memory_updater" in ckpt:
                rt.memory_updater.load_state_dict(ckpt["memory_updater"])
                rt.memory_updater.kernel_weights()   # refresh bf16 copies in place
        rt.params_changed()   # the attention's bf16 weight copies, before the next step
        rt.fence()


def _check_state_keys(owner: str, own: dict, loaded: dict) -> None:
    """The strict checks of nn.Module.load_state_dict (same message form):
    missing and unexpected keys and shape mismatches raise RuntimeError."""
    missing = [k for k in own if k not in loaded]
    unexpected = [k for k in loaded if k not in own]
    errs = []
    if unexpected:
        errs.append("Unexpected key(s) in state_dict: " + ", ".join(f'"{k}"' for k in unexpected) + ". ")
    if missing:
        errs.append("Missing key(s) in state_dict: " + ", ".join(f'"{k}"' for k in missing) + ". ")
    for k, t in loaded.items():
        if k in own and tuple(own[k].shape) != tuple(t.shape):
            errs.append(f"size mismatch for {k}: copying a param with shape {tuple(t.shape)} from checkpoint, "
                        f"the shape in current model is {tuple(own[k].shape)}.")
    if errs:
        raise RuntimeError(f"Error(s) in loading state_dict for {owner}:\n\t" + "\n\t".join(errs))
