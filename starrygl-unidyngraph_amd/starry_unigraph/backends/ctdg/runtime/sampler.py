"""Native temporal sampler for CTDG (backends/ctdg/runtime/sampler.py:18-128 in
the reference): one sampler per split, built lazily from
``TGTemporalDataset.sampler_graph(split)`` through the drop-in binding
(starry_unigraph.native). The graph lives in HBM; ``device_sampler(split)``
hands the runtime the device CSR for its fused step."""
from __future__ import annotations

from dataclasses import dataclass

import torch

from starry_unigraph.native import BTSNativeSampler, build_temporal_neighbor_block, is_bts_sampler_available
from starry_unigraph.native.tcsr import RecentSampler

from .data import TGTemporalDataset


@dataclass
class CTDGSampleOutput:
    split: str
    root_nodes: torch.Tensor
    timestamps: torch.Tensor
    sampled_nodes: torch.Tensor
    sampled_eids: torch.Tensor
    blocks: list[object]

    def describe(self) -> dict[str, int]:
        return {"root_count": int(self.root_nodes.numel()), "sampled_node_count": int(self.sampled_nodes.numel()),
                "sampled_edge_count": int(self.sampled_eids.numel()), "num_layers": len(self.blocks)}


class NativeTemporalSampler:
    def __init__(self, dataset: TGTemporalDataset, fanout: list[int], history: int, strategy: str, workers: int = 1):
        self.dataset = dataset
        self.fanout = list(fanout)
        self.history = int(history)
        self.strategy = str(strategy)
        self.workers = int(workers)
        self._samplers: dict[str, BTSNativeSampler] = {}
        self._device: dict[str, RecentSampler] = {}

    def _build_sampler(self, split: str) -> BTSNativeSampler:
        graph = self.dataset.sampler_graph(split)
        tnb = build_temporal_neighbor_block(graph_name=f"{self.dataset.root.name}_{split}", row=graph["row"],
                                            col=graph["col"], num_nodes=self.dataset.num_nodes, eid=graph["eid"],
                                            timestamp=graph["ts"])
        return BTSNativeSampler(tnb=tnb, num_nodes=self.dataset.num_nodes, num_edges=graph["eid"].numel(),
                                num_layers=self.history, fanout=self.fanout, workers=self.workers,
                                policy=self.strategy,
                                edge_part=torch.zeros(graph["eid"].numel(), dtype=torch.int32),
                                node_part=torch.zeros(self.dataset.num_nodes, dtype=torch.int32))

    def _get(self, split: str) -> BTSNativeSampler:
        s = self._samplers.get(split)
        if s is None:
            s = self._samplers[split] = self._build_sampler(split)
        return s

    def device_sampler(self, split: str) -> RecentSampler:
        if self.strategy != "recent":
            raise RuntimeError(f'sampling strategy "{self.strategy}" is not implemented on the MI355X path '
                               '(the CTDG configs use "recent")')
        r = self._device.get(split)
        if r is None:
            r = self._device[split] = RecentSampler.for_graph(self._get(split).tnb.graph)
        return r

    def sample(self, split: str, root_nodes: torch.Tensor, timestamps: torch.Tensor) -> CTDGSampleOutput:
        """sampler.py:93-128 (query times go through float32 as there)."""
        if not is_bts_sampler_available():
            raise RuntimeError("Native BTS sampler is not available")
        blocks = self._get(split).sample_from_nodes(root_nodes.long(), timestamps.float())
        nodes = [b.sample_nodes().long() for b in blocks]
        eids = [b.eid().long() for b in blocks]
        dev = nodes[0].device if nodes else root_nodes.device
        merged_nodes = torch.unique(torch.cat([root_nodes.long().to(dev), *nodes]))
        merged_eids = torch.unique(torch.cat(eids)) if eids else torch.empty(0, dtype=torch.long)
        return CTDGSampleOutput(split=split, root_nodes=root_nodes.long(), timestamps=timestamps.float(),
                                sampled_nodes=merged_nodes, sampled_eids=merged_eids, blocks=list(blocks))
