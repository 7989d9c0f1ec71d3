"""CTDG model components backed by the MI355X kernels.

Module structure, parameter names and construction order follow the
reference (backends/ctdg/runtime/models.py), so state dicts are
interchangeable and a seeded construction draws the same initial weights:

* ``TemporalTransformerConv`` (models.py:35-137): TimeEncode, w_q, w_k, w_v,
  w_out, LayerNorm. Its forward runs the fused HIP attention kernels over a
  device block (the padded hop-0 sample of the step's roots) instead of a
  DGL block; backward is the matching HIP kernel plus weight-gradient GEMMs.
* ``CTDGMemoryUpdater`` (models.py:214-254): nn.GRU(2D+F -> D) over the K
  mailbox slots, then nn.GRUCell(D, D). Evaluated by the fused GRU kernel;
  it never receives gradients in the reference (its output is detached,
  runtime.py:279), so it is forward-only here.
* ``CTDGLinkPredictor`` (models.py:261-324) and ``build_ctdg_model``
  (models.py:327-386). The runtime's step evaluates the edge predictor and
  the BCE loss with the sgl_predictor kernel; the module's forward (torch)
  serves callers outside the step.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from starry_unigraph.lib import _capi
from starry_unigraph.native.step import ConvFunction, DeviceStep
from starry_unigraph.runtime.modules import TimeEncode


class TemporalTransformerConv(nn.Module):
    """Single-layer temporal multi-head attention (models.py:35-137)."""

    def __init__(self, dim_node: int, dim_edge: int, dim_time: int, num_head: int, dim_out: int,
                 dropout: float = 0.1, att_dropout: float = 0.1) -> None:
        super().__init__()
        if dim_time <= 0:
            raise ValueError("TemporalTransformerConv: the MI355X kernels need dim_time > 0")
        if dim_out != dim_node:
            raise ValueError("TemporalTransformerConv: dim_out must equal dim_node (the CTDG path uses hidden_dim)")
        if dim_out % num_head:
            raise ValueError("TemporalTransformerConv: dim_out must be divisible by num_head")
        self.num_head = num_head
        self.dim_node = dim_node
        self.dim_edge = dim_edge
        self.dim_time = dim_time
        self.dim_out = dim_out
        self.time_enc = TimeEncode(dim_time)
        self.w_q = nn.Linear(dim_node + dim_time, dim_out)
        self.w_k = nn.Linear(dim_node + dim_edge + dim_time, dim_out)
        self.w_v = nn.Linear(dim_node + dim_edge + dim_time, dim_out)
        self.w_out = nn.Linear(dim_node + dim_out, dim_out)
        self.dropout = nn.Dropout(dropout)
        self.att_dropout = nn.Dropout(att_dropout)
        self.att_act = nn.LeakyReLU(0.2)
        self.layer_norm = nn.LayerNorm(dim_out)
        # dropout masks come from a counter-based generator keyed by this seed
        # and the step buffers' counter (torch's generators are not consumed)
        self.dropout_seed = int(torch.initial_seed()) & 0xFFFFFFFFFFFFFFFF
        # "bf16": the fused step runs the attention and edge-predictor
        # products on bf16 weight copies (fp32 accumulation)
        self.gemm_dtype = "fp32"

    def set_gemm_dtype(self, dtype: str) -> None:
        if dtype not in ("fp32", "bf16"):
            raise ValueError(f"attention GEMM dtype {dtype!r}: expected 'fp32' or 'bf16'")
        if dtype == "bf16" and (self.dropout.p != 0 or self.att_dropout.p != 0):
            raise ValueError("the bf16 attention products run without dropout (set dropout and att_dropout to 0)")
        self.gemm_dtype = dtype

    def kernel_params(self) -> list[torch.Tensor]:
        return [self.time_enc.w.weight, self.time_enc.w.bias, self.w_q.weight, self.w_q.bias, self.w_k.weight,
                self.w_k.bias, self.w_v.weight, self.w_v.bias, self.w_out.weight, self.w_out.bias,
                self.layer_norm.weight, self.layer_norm.bias]

    def drop_args(self):
        """(p_att, p_out, seed) of the attention kernels in training, or None
        when both dropouts are off (or in eval mode)."""
        if not self.training or (self.dropout.p == 0 and self.att_dropout.p == 0):
            return None
        return float(self.att_dropout.p), float(self.dropout.p), self.dropout_seed

    def forward(self, step: DeviceStep, edge_feat_all: torch.Tensor) -> torch.Tensor:
        """Embeddings [capacity, D] of the step's roots (rows >= the live root
        count are zero). In training with dropout each call draws fresh masks
        (the step buffers' counter advances)."""
        drop = self.drop_args()
        if drop is not None:
            step.buf.rng_step.add_(1)
        return ConvFunction.apply(step, edge_feat_all, drop, *self.kernel_params())


@dataclass
class CTDGModelOutput:
    pos_logits: torch.Tensor
    neg_logits: torch.Tensor


class CTDGMemoryUpdater(nn.Module):
    """GRU over the K-slot mailbox, then GRUCell with the memory (models.py:214-254)."""

    _MATRICES = ("w_ih", "w_hh", "wc_ih", "wc_hh")

    def __init__(self, hidden_dim: int, mailbox_slot_dim: int, mailbox_slots: int, gemm_dtype: str = "fp32") -> None:
        super().__init__()
        if gemm_dtype not in ("fp32", "bf16"):
            raise ValueError(f"memory updater GEMM dtype {gemm_dtype!r}: expected 'fp32' or 'bf16'")
        self.hidden_dim = hidden_dim
        self.mailbox_slots = mailbox_slots
        self.gemm_dtype = gemm_dtype
        self.mail_aggregator = nn.GRU(input_size=mailbox_slot_dim, hidden_size=hidden_dim, batch_first=True)
        self.memory_cell = nn.GRUCell(hidden_dim, hidden_dim)
        self._bf16: dict[str, torch.Tensor] = {}
        self._bf16_versions: tuple = ()

    def kernel_weights(self) -> dict[str, torch.Tensor]:
        """The fused kernel's operands. With bf16 GEMMs the four weight
        matrices are bf16 copies (round to nearest even) held in persistent
        buffers: the weights never train (the update is detached,
        runtime.py:279), and a changed weight (a loaded checkpoint) is copied
        into the same buffers, so recorded launch plans stay valid."""
        g, c = self.mail_aggregator, self.memory_cell
        w = {"w_ih": g.weight_ih_l0.detach(), "w_hh": g.weight_hh_l0.detach(), "b_ih": g.bias_ih_l0.detach(),
             "b_hh": g.bias_hh_l0.detach(), "wc_ih": c.weight_ih.detach(), "wc_hh": c.weight_hh.detach(),
             "bc_ih": c.bias_ih.detach(), "bc_hh": c.bias_hh.detach()}
        if self.gemm_dtype == "fp32":
            return w
        params = (g.weight_ih_l0, g.weight_hh_l0, c.weight_ih, c.weight_hh)
        versions = tuple((p.data_ptr(), p._version) for p in params)
        if versions != self._bf16_versions:
            for name in self._MATRICES:
                if name in self._bf16 and self._bf16[name].shape == w[name].shape:
                    self._bf16[name].copy_(w[name])
                else:
                    self._bf16[name] = w[name].to(torch.bfloat16).contiguous()
            # the wide-tile kernel's fragment-order copy of the four matrices
            D = self.hidden_dim
            F = int(w["w_ih"].shape[1]) - 2 * D
            n = int(_capi.lib().sgl_gru_packed_elems(D, F))
            pk = self._bf16.get("packed")
            if pk is None or pk.numel() != n or pk.device != w["w_ih"].device:
                pk = self._bf16["packed"] = torch.empty(n, dtype=torch.bfloat16, device=w["w_ih"].device)
            P = _capi.ptr
            _capi.check(_capi.lib().sgl_gru_pack_bf16(
                D, F, P(self._bf16["w_ih"]), P(self._bf16["w_hh"]), P(self._bf16["wc_ih"]), P(self._bf16["wc_hh"]),
                P(pk), _capi.stream_of(pk.device)), "sgl_gru_pack_bf16")
            self._bf16_versions = versions
        w.update(self._bf16)
        return w

    @torch.no_grad()
    def forward(self, mailbox_history: torch.Tensor, current_memory: torch.Tensor) -> torch.Tensor:
        """mailbox_history [M, K, S], current_memory [M, D] -> [M, D], through
        the fused GRU kernel (rows addressed by an identity root list)."""
        M = mailbox_history.size(0)
        if M == 0:
            return current_memory.clone()
        dev = _capi.require_gpu(current_memory.device)
        D = self.hidden_dim
        K = mailbox_history.size(1)
        S = mailbox_history.size(2)
        Fd = S - 2 * D
        mail = mailbox_history.to(dev, torch.float32).contiguous()
        mem = current_memory.to(dev, torch.float32).contiguous()
        cap = (M + 15) // 16 * 16
        roots = torch.arange(M, dtype=torch.int64, device=dev)
        n = torch.tensor([M], dtype=torch.int32, device=dev)
        zeros_i = torch.zeros(cap, dtype=torch.int32, device=dev)
        zeros_k = torch.zeros(cap, dtype=torch.int64, device=dev)
        out = torch.empty(cap, D, dtype=torch.float32, device=dev)
        w = self.kernel_weights()
        P = _capi.ptr
        dummy_i64 = torch.zeros(1, dtype=torch.int64, device=dev)
        dummy_f = torch.zeros(max(Fd, 1), dtype=torch.float32, device=dev)
        mts = torch.zeros(M, K, dtype=torch.float32, device=dev)
        nmp = torch.zeros(M, dtype=torch.int32, device=dev)
        name = "sgl_memory_update_bf16" if self.gemm_dtype == "bf16" else "sgl_memory_update"
        _capi.check(getattr(_capi.lib(), name)(
            D, K, Fd, cap, P(n), P(roots), P(mem), P(mail), P(mts), P(nmp), P(w["w_ih"]), P(w["w_hh"]),
            P(w["b_ih"]), P(w["b_hh"]), P(w["wc_ih"]), P(w["wc_hh"]), P(w["bc_ih"]), P(w["bc_hh"]), P(dummy_i64),
            P(dummy_i64), P(dummy_f), P(dummy_f), None, P(zeros_k), P(zeros_k), P(zeros_i), P(zeros_i), P(out),
            *([P(w["packed"])] if self.gemm_dtype == "bf16" else []), _capi.stream_of(dev)), name)
        return out[:M]


class CTDGLinkPredictor(nn.Module):
    """Temporal attention + edge predictor (models.py:261-324)."""

    def __init__(self, num_nodes: int, hidden_dim: int, edge_feat_dim: int, dim_time: int = 100, num_head: int = 2,
                 dropout: float = 0.1, att_dropout: float = 0.1) -> None:
        super().__init__()
        self.hidden_dim = hidden_dim
        self.conv = TemporalTransformerConv(dim_node=hidden_dim, dim_edge=edge_feat_dim, dim_time=dim_time,
                                            num_head=num_head, dim_out=hidden_dim, dropout=dropout,
                                            att_dropout=att_dropout)
        self.src_fc = nn.Linear(hidden_dim, hidden_dim)
        self.dst_fc = nn.Linear(hidden_dim, hidden_dim)
        self.out_fc = nn.Linear(hidden_dim, 1)

    def embedding_module(self) -> nn.Module:
        """The module that embeds the roots (its parameters are the
        optimizer's first segment)."""
        return self.conv

    def forward(self, src_conv: torch.Tensor, dst_conv: torch.Tensor, neg_conv: torch.Tensor) -> CTDGModelOutput:
        h_src = self.src_fc(src_conv)
        h_dst = self.dst_fc(dst_conv)
        h_neg = self.dst_fc(neg_conv)
        pos_logits = self.out_fc(F.relu(h_src + h_dst)).squeeze(-1)
        neg_logits = self.out_fc(F.relu(h_src + h_neg)).squeeze(-1)
        return CTDGModelOutput(pos_logits=pos_logits, neg_logits=neg_logits)


class TimeProjection(nn.Module):
    """JODIE's time projection (Kumar, Zhang, Leskovec, KDD 2019, eq. 3):
    h * (1 + proj(x)) with proj = nn.Linear(1, D) and x the time since the
    node's previous memory update, normalised as (dt - shift) * scale
    (shift / scale: the mean and the inverse spread of the training
    split's per-node inter-event times). Evaluated by
    sgl_time_projection_forward / _backward on the step's roots."""

    def __init__(self, dim: int, shift: float = 0.0, scale: float = 1.0) -> None:
        super().__init__()
        self.proj = nn.Linear(1, dim)
        nn.init.normal_(self.proj.weight, 0.0, 0.1)
        nn.init.zeros_(self.proj.bias)
        self.shift, self.scale = float(shift), float(scale)


class CTDGTimeProjectionPredictor(nn.Module):
    """Config 2's JODIE model: the node memory (GRU updater) embedded by a
    time projection instead of the temporal attention, then the same edge
    predictor (src_fc, dst_fc, out_fc; models.py:313-324). The reference has
    no such embedding (its "jodie" builds CTDGLinkPredictor,
    models.py:337-338); select it with ctdg.embedding = time_projection."""

    def __init__(self, num_nodes: int, hidden_dim: int, time_shift: float = 0.0, time_scale: float = 1.0,
                 **_unused) -> None:
        super().__init__()
        self.hidden_dim = hidden_dim
        self.conv = None
        self.time_proj = TimeProjection(hidden_dim, time_shift, time_scale)
        self.src_fc = nn.Linear(hidden_dim, hidden_dim)
        self.dst_fc = nn.Linear(hidden_dim, hidden_dim)
        self.out_fc = nn.Linear(hidden_dim, 1)

    def embedding_module(self) -> nn.Module:
        return self.time_proj

    def forward(self, src_emb: torch.Tensor, dst_emb: torch.Tensor, neg_emb: torch.Tensor) -> CTDGModelOutput:
        h_src = self.src_fc(src_emb)
        pos_logits = self.out_fc(F.relu(h_src + self.dst_fc(dst_emb))).squeeze(-1)
        neg_logits = self.out_fc(F.relu(h_src + self.dst_fc(neg_emb))).squeeze(-1)
        return CTDGModelOutput(pos_logits=pos_logits, neg_logits=neg_logits)


@dataclass(frozen=True)
class CTDGModelSpec:
    model_cls: type[nn.Module]


# One implementation serves the CTDG families the reference registers (models.py:332-342).
CTDG_MODEL_SPECS: dict[str, CTDGModelSpec] = {
    name: CTDGModelSpec(CTDGLinkPredictor) for name in ("tgn", "jodie", "dyrep", "tgat", "apan")
}


def build_ctdg_model(model_family: str, *, num_nodes: int, hidden_dim: int, edge_feat_dim: int, dim_time: int = 100,
                     num_head: int = 2, dropout: float = 0.1, att_dropout: float = 0.1,
                     embedding: str = "attention", time_shift: float = 0.0, time_scale: float = 1.0,
                     attention_gemm_dtype: str = "fp32") -> nn.Module:
    """models.py:345-386. ``embedding`` "attention" (the reference's model for
    every family) or "time_projection" (config 2's JODIE embedding);
    ``attention_gemm_dtype`` "bf16": the attention and edge-predictor products
    on bf16 weight copies (benchmark configurations 4 and 5)."""
    spec = CTDG_MODEL_SPECS.get(model_family.lower())
    if spec is None:
        raise KeyError(f"Unsupported CTDG model family: {model_family}")
    if embedding == "time_projection":
        return CTDGTimeProjectionPredictor(num_nodes=num_nodes, hidden_dim=hidden_dim, time_shift=time_shift,
                                           time_scale=time_scale)
    if embedding != "attention":
        raise KeyError(f"unknown ctdg.embedding {embedding!r}: expected 'attention' or 'time_projection'")
    model = spec.model_cls(num_nodes=num_nodes, hidden_dim=hidden_dim, edge_feat_dim=edge_feat_dim,
                           dim_time=dim_time, num_head=num_head, dropout=dropout, att_dropout=att_dropout)
    if getattr(model, "conv", None) is not None:
        model.conv.set_gemm_dtype(attention_gemm_dtype)
    elif attention_gemm_dtype != "fp32":
        raise ValueError(f"model family {model_family!r} has no attention for ctdg.attention_gemm_dtype")
    return model
