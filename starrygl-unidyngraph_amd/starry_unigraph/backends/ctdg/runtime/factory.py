"""Build a CTDGOnlineRuntime from a session config (backends/ctdg/runtime/factory.py:20-178
in the reference). Construction order is the reference's -- dataset, sampler,
memory bank, model, memory updater -- so a seeded run draws the same initial
weights. The optimizer is a fused HIP Adam over the trainable parameters."""
from __future__ import annotations

from pathlib import Path

import torch

from starry_unigraph.native.step import FusedAdam
from starry_unigraph.types import RuntimeBundle, SessionContext

from .data import TGTemporalDataset
from .memory import CTDGMemoryBank
from .models import CTDGMemoryUpdater, build_ctdg_model
from .runtime import CTDGOnlineRuntime
from .sampler import NativeTemporalSampler


class _SingleRankRoute:
    """The reference's CTDGFeatureRoute is multi-rank only; one GPU needs none."""

    def __init__(self, route_type: str, world_size: int):
        self.route_type, self.world_size = route_type, world_size

    def describe(self) -> dict:
        return {"route_type": self.route_type, "world_size": self.world_size}


def build_ctdg_runtime(session_ctx: SessionContext, events=None) -> tuple[CTDGOnlineRuntime, RuntimeBundle]:
    cfg = session_ctx.config
    root = session_ctx.dataset_path or Path(cfg["data"]["root"]).expanduser().resolve()
    dataset = TGTemporalDataset(root, cfg["data"]["name"], split_ratio=cfg.get("data", {}).get("split_ratio"),
                                config=cfg, events=events)
    device = str(cfg["runtime"]["device"])
    hidden_dim = int(cfg["model"]["hidden_dim"])
    c = cfg.get("ctdg", {})
    mailbox_slots = int(c.get("mailbox_slots", 4))
    dim_time = int(c.get("dim_time", 100))
    num_head = int(c.get("num_head", 2))
    dropout = float(c.get("dropout", 0.1))
    att_dropout = float(c.get("att_dropout", 0.1))
    sampler = NativeTemporalSampler(dataset=dataset, fanout=list(cfg["sampling"]["neighbor_limit"]),
                                    history=int(cfg["sampling"]["history"]),
                                    strategy=str(cfg["sampling"]["strategy"]),
                                    workers=max(1, min(4, session_ctx.dist.local_world_size or 1)))
    edge_feat_dim = max(1, dataset.edge_feat_dim)
    dataset.configure_partition(node_parts=None, edge_parts=None, rank=session_ctx.dist.rank,
                                world_size=session_ctx.dist.world_size)
    memory = CTDGMemoryBank(num_nodes=dataset.num_nodes, hidden_dim=hidden_dim, device=device,
                            mailbox_slots=mailbox_slots, edge_feat_dim=edge_feat_dim)
    embedding = str(c.get("embedding", "attention"))
    shift, scale = dataset.inter_event_stats("train") if embedding == "time_projection" else (0.0, 1.0)
    model = build_ctdg_model(str(cfg["model"]["family"]), num_nodes=dataset.num_nodes, hidden_dim=hidden_dim,
                             edge_feat_dim=edge_feat_dim, dim_time=dim_time, num_head=num_head, dropout=dropout,
                             att_dropout=att_dropout, embedding=embedding, time_shift=shift,
                             time_scale=scale,
                             attention_gemm_dtype=str(c.get("attention_gemm_dtype", "fp32"))).to(device)
    memory_updater = CTDGMemoryUpdater(hidden_dim=hidden_dim, mailbox_slot_dim=2 * hidden_dim + edge_feat_dim,
                                       mailbox_slots=mailbox_slots,
                                       gemm_dtype=str(c.get("memory_gemm_dtype", "fp32"))).to(device)
    optimizer = make_optimizer(model, lr=float(cfg.get("train", {}).get("lr", 1e-3)))
    runtime = CTDGOnlineRuntime(dataset=dataset, sampler=sampler, memory=memory, model=model, optimizer=optimizer,
                                route=_SingleRankRoute(str(cfg["graph"]["route"]), session_ctx.dist.world_size),
                                device=device, dist_ctx=session_ctx.dist, memory_updater=memory_updater,
                                max_batch=int(cfg["train"]["batch_size"]))
    if getattr(model, "conv", None) is not None:
        optimizer.gate_fn = lambda: runtime.step.buf.any_edges
    optimizer.inner  # re-seat the parameters in the optimizer's flat buffers before any forward
    bundle = RuntimeBundle(model=model, optimizer=optimizer,
                           state={"pipeline": "ctdg_online_native", "dataset": dataset.describe(),
                                  "memory_state": memory.describe(), "route_state": runtime.route.describe()})
    return runtime, bundle


def make_optimizer(model: torch.nn.Module, lr: float) -> "GatedAdam":
    return GatedAdam(model, lr)


class GatedAdam:
    """Adam over the link predictor's parameters (factory.py:122-128), in
    three segments: the embedding module's first parameter (the model's
    first parameter), the rest of the embedding (the attention, or the time
    projection) and the edge predictor. The first two are gated by the
    step's "block has edges" flag (when it is 0 those parameters have no
    gradient in the reference, and Adam skips them). The first parameter has
    a segment of its own because the reference's empty-batch step
    (runtime.py:248-253) gives it, alone among the model's parameters, a zero
    gradient and an Adam step (its step count and moments advance).

    The memory updater gets no gradients in the reference (runtime.py:279)
    and is not optimised here. Its first parameter's zero-gradient steps on
    empty batches (runtime.py:111-116) leave its values unchanged: its
    moments start at zero and stay there, so each update is 0 / (0 + eps)."""

    def __init__(self, model: torch.nn.Module, lr: float):
        self.model = model
        self.lr = lr
        self._inner: FusedAdam | None = None
        self.gate_fn = None

    def _build(self) -> FusedAdam:
        core = self.model.module if hasattr(self.model, "module") else self.model
        emb = list(core.embedding_module().parameters())
        first = next(core.parameters())
        if emb[0] is not first:
            raise RuntimeError("GatedAdam: the model's first parameter must open its embedding module")
        emb_ids = {id(p) for p in emb}
        rest = [p for p in core.parameters() if id(p) not in emb_ids]
        return FusedAdam([emb[:1], emb[1:], rest], lr=self.lr)

    @property
    def inner(self) -> FusedAdam:
        if self._inner is None:
            self._inner = self._build()
        return self._inner

    def zero_grad(self, set_to_none: bool = False) -> None:
        self.inner.zero_grad()

    def step(self) -> None:
        gate = self.gate_fn() if self.gate_fn is not None else None
        self.inner.step([gate, gate, None])

    def empty_step(self) -> None:
        """The reference's step on an empty batch (runtime.py:248-253): the
        model's first parameter takes an Adam step with a zero gradient;
        every other parameter is untouched."""
        inner = self.inner
        start, n, _ = inner.segments[0]
        inner.flat_grad[start:start + n].zero_()
        inner.step([None], only=[0])

    def state_dict(self) -> dict:
        return self.inner.state_dict()

    def load_state_dict(self, sd: dict) -> None:
        self.inner.load_state_dict(sd)
