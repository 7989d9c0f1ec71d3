"""Per-node memory and K-slot mailbox in HBM (backends/ctdg/runtime/memory.py:43-574
in the reference, single rank).

The state is a ``NodeState`` (starry_unigraph.native.step); the training step
updates it with fused kernels (sgl_memory_update / sgl_memory_commit). The
methods below keep the reference's public API for callers outside the fused
step (gather, read_mailbox, write_mailbox, _apply_memory_update, the sync
entry points) and run as GPU tensor ops with the reference's semantics: the
mailbox write keeps, per node and pass, the last event in stable timestamp
order and advances the slot pointer by the occurrence count.

Multi-rank exchange (all_to_all of memory and mail, memory.py:300-553) is not
part of this single-GPU build; with world_size 1 the sync calls reduce to what
the reference's single-rank fallbacks do.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch

from starry_unigraph.lib import _capi
from starry_unigraph.native.step import NodeState


@dataclass
class CTDGMemoryBank:
    num_nodes: int
    hidden_dim: int
    device: str
    mailbox_slots: int = 1
    edge_feat_dim: int = 0
    rank: int = 0
    world_size: int = 1
    async_sync: bool = True
    node_parts: torch.Tensor | None = None

    def __post_init__(self) -> None:
        if self.world_size != 1:
            raise NotImplementedError("CTDGMemoryBank: this build runs one GPU (world_size 1)")
        dev = _capi.require_gpu(self.device)
        self._storage_device = dev
        E = max(0, self.edge_feat_dim)
        self.slot_width = 2 * self.hidden_dim + E
        self.state = NodeState(self.num_nodes, self.hidden_dim, self.mailbox_slots, E, dev)
        self.num_local_nodes = self.num_nodes
        self.memory_version = 0
        self.mailbox_version = 0
        self.historical_cache = None
        self.last_memory_sync = None
        self.last_mail_sync = None

    # reference attribute names
    @property
    def memory(self) -> torch.Tensor:
        return self.state.memory

    @property
    def mailbox(self) -> torch.Tensor:
        return self.state.mailbox

    @property
    def mailbox_ts(self) -> torch.Tensor:
        return self.state.mailbox_ts

    @property
    def memory_ts(self) -> torch.Tensor:
        return self.state.memory_ts

    @property
    def next_mail_pos(self) -> torch.Tensor:
        return self.state.next_mail_pos

    @property
    def last_update(self) -> torch.Tensor:
        return self.state.memory_ts

    def _ids(self, node_ids: torch.Tensor) -> torch.Tensor:
        return node_ids.to(self._storage_device, torch.long)

    def gather(self, node_ids: torch.Tensor) -> torch.Tensor:
        return self.state.memory[self._ids(node_ids)]

    def read_mailbox(self, node_ids: torch.Tensor) -> torch.Tensor:
        return self.state.mailbox[self._ids(node_ids)]

    def gather_mailbox(self, node_ids: torch.Tensor) -> torch.Tensor:
        return self.read_mailbox(node_ids)[:, 0, :]

    def read_mailbox_ts(self, node_ids: torch.Tensor) -> torch.Tensor:
        return self.state.mailbox_ts[self._ids(node_ids)]

    def write_mailbox(self, src_ids, dst_ids, src_mem, dst_mem, edge_feat, timestamps) -> None:
        """memory.py:183-222: [self | other | edge_feat] messages, src pass then dst pass."""
        dev = self._storage_device
        E = self.slot_width - 2 * self.hidden_dim
        ef = edge_feat.to(dev).float()
        ef = ef[..., :E] if ef.size(-1) >= E else torch.cat(
            [ef, torch.zeros(*ef.shape[:-1], E - ef.size(-1), device=dev)], dim=-1)
        smem, dmem = src_mem.to(dev).float(), dst_mem.to(dev).float()
        ts = timestamps.to(dev).float()
        self._write_slots(self._ids(src_ids), torch.cat([smem, dmem, ef], -1), ts)
        self._write_slots(self._ids(dst_ids), torch.cat([dmem, smem, ef], -1), ts)
        self.mailbox_version += 1

    def _write_slots(self, ids: torch.Tensor, vals: torch.Tensor, ts: torch.Tensor) -> None:
        if ids.numel() == 0:
            return
        self.state.touched()
        K = self.mailbox_slots
        order = torch.argsort(ts, stable=True)
        ids_o, vals_o, ts_o = ids[order], vals[order], ts[order]
        uniq, inv, counts = torch.unique(ids_o, return_inverse=True, return_counts=True)
        last = torch.full((uniq.numel(),), -1, dtype=torch.long, device=ids.device)
        last.scatter_reduce_(0, inv, torch.arange(ids_o.numel(), device=ids.device), "amax", include_self=True)
        pos = self.state.next_mail_pos[uniq].long()
        self.state.mailbox[uniq, pos] = vals_o[last]
        self.state.mailbox_ts[uniq, pos] = ts_o[last]
        self.state.next_mail_pos[uniq] = ((pos + counts) % K).to(torch.int32)

    def _apply_memory_update(self, node_ids: torch.Tensor, values: torch.Tensor, timestamps: torch.Tensor) -> None:
        """memory.py:254-269 (ids unique, latest timestamp written last)."""
        if node_ids.numel() == 0:
            return
        ids = self._ids(node_ids)
        self.state.touched()
        ts = timestamps.to(ids.device).float()
        order = torch.argsort(ts, stable=True)
        self.state.memory[ids[order]] = values.to(ids.device).float()[order]
        self.state.memory_ts[ids[order]] = ts[order]
        self.memory_version += 1

    _apply_updates = _apply_memory_update

    def submit_async_memory_sync(self, ctx, node_ids, values, timestamps) -> None:
        # single rank: the reference re-applies the rows (memory.py:348-350)
        self._apply_memory_update(node_ids, values.detach(), timestamps.detach())

    def submit_async_mail_sync(self, ctx, node_ids, mail_slots, mail_ts) -> None:
        return None

    def wait_pending_syncs(self) -> None:
        return None

    def sync_updates(self, ctx, node_ids, values, timestamps) -> None:
        self.submit_async_memory_sync(ctx, node_ids, values, timestamps)

    def reset(self) -> None:
        self.state.reset()
        self.memory_version = 0
        self.mailbox_version = 0

    def describe(self) -> dict[str, Any]:
        return {"num_nodes": self.num_nodes, "num_local_nodes": self.num_local_nodes, "hidden_dim": self.hidden_dim,
                "mailbox_slots": self.mailbox_slots, "memory_version": self.memory_version,
                "storage_device": str(self._storage_device)}
