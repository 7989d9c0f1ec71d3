"""TEST INFRASTRUCTURE ONLY -- torch-CPU restatement of the reference's CTDG
training step (the part after sampling). Only tests/, ``smoke()`` and
bench.py's ``cpu_baseline`` leg may import it, and only as the checker or the
timed CPU baseline; the product path never imports it.

Follows, function by function:
  TimeEncodeO            runtime/modules/time_encode.py:41-58 (argument rounded
                         as fl(fl(t*w) + b): the GEMM-with-bias-epilogue result)
  TemporalConvO.forward  backends/ctdg/runtime/models.py:77-137 with
                         build_dgl_block models.py:144-197 (DGL edge_softmax
                         restated as a per-destination max-subtracted softmax,
                         update_all(copy_e, sum) as index_add)
  LinkPredictorO         models.py:261-324
  MemoryUpdaterO         models.py:214-254 (torch.nn.GRU + GRUCell, as there)
  build_models           factory.py:96-112 (construction order fixes init RNG)
  MemoryO                backends/ctdg/runtime/memory.py:43-269 (1 rank)
  negative_sample        backends/ctdg/runtime/runtime.py:124-136
  prepare_roots          runtime.py:138-144
  conv_output/_select    runtime.py:146-183
  train_step             runtime.py:225-328 (dropout as explicit masks: the
                         GPU kernels' masks are replayed, torch's own draws
                         cannot be matched)
  empty_train_step       runtime.py:248-253 with runtime.py:111-116, pinned
                         by Adam's closed form with a zero gradient
  ProjectionPredictorO   config 2's JODIE time projection (the build's own
                         definition: the reference has none), pinned by a
                         closed form
  philox4x32_10          the counter-based generator of the kernels' dropout
                         masks (Salmon et al., SC 2011), pinned by the
                         published known-answer vectors

Parity pins (tests/test_oracle_step.py): GRU/GRUCell against hand-written
gate equations; the conv against a per-root brute-force attention loop and
invariants (single neighbour, no neighbour, empty block, permutation of a
root's neighbours); mailbox writes against a serial loop of the A10 rules.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F
from torch import nn


# --------------------------------------------------------------------------- models
class TimeEncodeO(nn.Module):
    """time_encode.py:41-58: cos(w t + b), w = 10^-linspace(0, 9, T), b = 0."""

    def __init__(self, dim: int):
        super().__init__()
        self.dim = dim
        self.w = nn.Linear(1, dim)                       # draws init RNG, then replaced
        self.w.bias = nn.Parameter(torch.zeros(dim))
        self.w.weight = nn.Parameter((1.0 / 10 ** torch.linspace(0, 9, dim)).reshape(dim, 1))

    # float64 copies only: keep the float32 rounding of the argument (its
    # value), with the exact derivative of t*w + b (tests that compare float32
    # gradients against float64 sums of the same float32 algorithm)
    round_arg_f32 = False

    def forward(self, t: torch.Tensor) -> torch.Tensor:
        # The reference evaluates nn.Linear(1, T); a GPU GEMM with a bias
        # epilogue rounds the product, then adds the bias. CPU BLAS picks a fused
        # multiply-add for some shapes and not others, so the oracle states the
        # two-rounding form elementwise. (t.float() in the reference; the
        # parameter dtype here so that a float64 copy can be checked in float64.)
        tt = t.to(self.w.weight.dtype).reshape(-1, 1)
        arg = tt * self.w.weight.reshape(1, -1) + self.w.bias
        if self.round_arg_f32 and arg.dtype == torch.float64:
            with torch.no_grad():
                a32 = (tt.float() * self.w.weight.float().reshape(1, -1)) + self.w.bias.float()
            arg = arg + (a32.double() - arg).detach()
        return torch.cos(arg).reshape(*t.shape, self.dim)


class TemporalConvO(nn.Module):
    """models.py:35-137 (TemporalTransformerConv) without DGL."""

    def __init__(self, dim_node, dim_edge, dim_time, num_head, dim_out, dropout=0.0, att_dropout=0.0):
        super().__init__()
        self.num_head = num_head
        self.dim_node, self.dim_edge, self.dim_time, self.dim_out = dim_node, dim_edge, dim_time, dim_out
        if dim_time > 0:
            self.time_enc = TimeEncodeO(dim_time)
        self.w_q = nn.Linear(dim_node + dim_time, dim_out)
        self.w_k = nn.Linear(dim_node + dim_edge + dim_time, dim_out)
        self.w_v = nn.Linear(dim_node + dim_edge + dim_time, dim_out)
        self.w_out = nn.Linear(dim_node + dim_out, dim_out)
        self.dropout = nn.Dropout(dropout)
        self.att_dropout = nn.Dropout(att_dropout)
        self.att_act = nn.LeakyReLU(0.2)
        self.layer_norm = nn.LayerNorm(dim_out)

    def forward(self, h_dst, h_nbr, ef, dt, edge_dst, att_mask=None, out_mask=None):
        """h_dst [R,D] (memory of roots), h_nbr [E,D] (memory of sampled
        neighbours), ef [E,F], dt [E] float32, edge_dst [E] in [0,R).
        att_mask [E,H] / out_mask [R,D] (values 0 or 1/(1-p)) replace the
        dropout modules' own draws (models.py:127,136) when given."""
        n_dst = h_dst.shape[0]
        if edge_dst.numel() == 0:                                  # models.py:88-89
            return torch.zeros(n_dst, self.dim_out, dtype=h_dst.dtype)
        if self.dim_time > 0:
            time_feat = self.time_enc(dt)
            zero_time = self.time_enc(torch.zeros(n_dst, dtype=h_dst.dtype))
            q_in = torch.cat([h_dst, zero_time], dim=1)
            k_in = torch.cat([h_nbr, ef, time_feat], dim=1)
        else:
            q_in = h_dst
            k_in = torch.cat([h_nbr, ef], dim=1)
        H = self.num_head
        Q = self.w_q(q_in)[edge_dst].reshape(-1, H, self.dim_out // H)
        K = self.w_k(k_in).reshape(-1, H, self.dim_out // H)
        V = self.w_v(k_in).reshape(-1, H, self.dim_out // H)
        att_raw = self.att_act((Q * K).sum(dim=2))                 # [E,H]
        att = segment_softmax(att_raw, edge_dst, n_dst)
        att = att * att_mask.to(att.dtype) if att_mask is not None else self.att_dropout(att)
        vw = (V * att.unsqueeze(-1)).reshape(V.shape[0], -1)
        agg = torch.zeros(n_dst, self.dim_out, dtype=vw.dtype).index_add(0, edge_dst, vw)
        rst = self.w_out(torch.cat([agg, h_dst], dim=1))
        rst = rst * out_mask.to(rst.dtype) if out_mask is not None else self.dropout(rst)
        return self.layer_norm(F.relu(rst))


def segment_softmax(x: torch.Tensor, seg: torch.Tensor, n: int) -> torch.Tensor:
    """DGL edge_softmax on a block: softmax of x [E,H] over edges sharing seg."""
    idx = seg.unsqueeze(1).expand_as(x)
    mx = torch.full((n, x.shape[1]), -math.inf, dtype=x.dtype).scatter_reduce(0, idx, x, "amax",
                                                                              include_self=True)
    e = torch.exp(x - mx[seg])
    s = torch.zeros(n, x.shape[1], dtype=x.dtype).index_add(0, seg, e)
    return e / s[seg]


class LinkPredictorO(nn.Module):
    """models.py:261-324."""

    def __init__(self, hidden_dim, edge_feat_dim, dim_time=100, num_head=2, dropout=0.0, att_dropout=0.0):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.conv = TemporalConvO(hidden_dim, edge_feat_dim, dim_time, num_head, hidden_dim, dropout, att_dropout)
        self.src_fc = nn.Linear(hidden_dim, hidden_dim)
        self.dst_fc = nn.Linear(hidden_dim, hidden_dim)
        self.out_fc = nn.Linear(hidden_dim, 1)

    def forward(self, src_conv, dst_conv, neg_conv):
        h_src = self.src_fc(src_conv)
        h_dst = self.dst_fc(dst_conv)
        h_neg = self.dst_fc(neg_conv)
        pos = self.out_fc(F.relu(h_src + h_dst)).squeeze(-1)
        neg = self.out_fc(F.relu(h_src + h_neg)).squeeze(-1)
        return pos, neg


class ProjectionPredictorO(nn.Module):
    """Config 2's JODIE model (no reference counterpart: the reference's
    "jodie" is its TGN model, models.py:337-338): the updated memory h of a
    root embedded as h * (1 + proj(x)), proj = nn.Linear(1, D), x = (dt -
    shift) * scale with dt the time since the root's previous memory update
    (JODIE, KDD 2019, eq. 3), then the edge predictor of LinkPredictorO."""

    def __init__(self, hidden_dim, shift=0.0, scale=1.0):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.time_proj = nn.Module()
        self.time_proj.proj = nn.Linear(1, hidden_dim)
        nn.init.normal_(self.time_proj.proj.weight, 0.0, 0.1)
        nn.init.zeros_(self.time_proj.proj.bias)
        self.shift, self.scale = float(shift), float(scale)
        self.src_fc = nn.Linear(hidden_dim, hidden_dim)
        self.dst_fc = nn.Linear(hidden_dim, hidden_dim)
        self.out_fc = nn.Linear(hidden_dim, 1)

    def embed(self, h, dt):
        """h [R, D] updated memory, dt [R] float32 time since the previous update."""
        x = (dt - torch.tensor(self.shift, dtype=dt.dtype)) * torch.tensor(self.scale, dtype=dt.dtype)
        lin = x.to(h.dtype).unsqueeze(1) * self.time_proj.proj.weight.reshape(1, -1) + self.time_proj.proj.bias
        return h * (1.0 + lin)

    forward = LinkPredictorO.forward


class MemoryUpdaterO(nn.Module):
    """models.py:214-254."""

    def __init__(self, hidden_dim, slot_dim, slots):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.mailbox_slots = slots
        self.mail_aggregator = nn.GRU(input_size=slot_dim, hidden_size=hidden_dim, batch_first=True)
        self.memory_cell = nn.GRUCell(hidden_dim, hidden_dim)

    def forward(self, mail, mem):
        if mail.size(0) == 0:
            return mem.clone()
        _, agg = self.mail_aggregator(mail)
        return self.memory_cell(agg.squeeze(0), mem)


def build_models(hidden_dim, edge_feat_dim, dim_time, num_head, slots, seed=0, dropout=0.0, att_dropout=0.0):
    """factory.py:96-112 order: predictor (TimeEncode, w_q, w_k, w_v, w_out,
    LayerNorm, src_fc, dst_fc, out_fc), then the updater (GRU, GRUCell)."""
    torch.manual_seed(seed)
    f = max(1, edge_feat_dim)
    model = LinkPredictorO(hidden_dim, f, dim_time, num_head, dropout, att_dropout)
    updater = MemoryUpdaterO(hidden_dim, 2 * hidden_dim + f, slots)
    return model, updater


def philox4x32_10(ctr, key):
    """Philox4x32-10 on uint32 numpy arrays: ctr [..., 4], key [..., 2]."""
    c = [np.asarray(ctr[..., i], dtype=np.uint64) for i in range(4)]
    k0 = np.asarray(key[..., 0], dtype=np.uint64)
    k1 = np.asarray(key[..., 1], dtype=np.uint64)
    m32 = np.uint64(0xFFFFFFFF)
    for _ in range(10):
        p0 = np.uint64(0xD2511F53) * c[0]
        p1 = np.uint64(0xCD9E8D57) * c[2]
        c = [((p1 >> np.uint64(32)) ^ c[1] ^ k0) & m32, p1 & m32, ((p0 >> np.uint64(32)) ^ c[3] ^ k1) & m32,
             p0 & m32]
        k0 = (k0 + np.uint64(0x9E3779B9)) & m32
        k1 = (k1 + np.uint64(0xBB67AE85)) & m32
    return np.stack(c, axis=-1).astype(np.uint32)


def dropout_masks(seed, step, pass_, rows, fanout, H, D, p_att, p_out):
    """The kernels' mask definition restated: attention [rows, fanout, H]
    from counter (row, slot, 2 pass, step) lanes 0..H-1, output [rows, D]
    from (row, col // 4, 2 pass + 1, step) lane col % 4, key (seed low,
    seed high ^ step high); keep when (u >> 8) / 2^24 >= p, kept = 1/(1-p)."""
    key = np.array([seed & 0xFFFFFFFF, ((seed >> 32) ^ (step >> 32)) & 0xFFFFFFFF], dtype=np.uint32)

    def keep(u, p):
        return np.where((u >> np.uint32(8)).astype(np.float64) * 2.0 ** -24 >= p, 1.0 / (1.0 - p), 0.0).astype(
            np.float32)

    r, e = np.meshgrid(np.arange(rows), np.arange(fanout), indexing="ij")
    ctr = np.stack([r, e, np.full_like(r, 2 * pass_), np.full_like(r, step & 0xFFFFFFFF)], -1).astype(np.uint32)
    att = keep(philox4x32_10(ctr, np.broadcast_to(key, ctr.shape[:-1] + (2,)))[..., :H], p_att)
    g4 = (D + 3) // 4
    r, cg = np.meshgrid(np.arange(rows), np.arange(g4), indexing="ij")
    ctr = np.stack([r, cg, np.full_like(r, 2 * pass_ + 1), np.full_like(r, step & 0xFFFFFFFF)], -1).astype(np.uint32)
    out = keep(philox4x32_10(ctr, np.broadcast_to(key, ctr.shape[:-1] + (2,))), p_out).reshape(rows, g4 * 4)[:, :D]
    return att, np.ascontiguousarray(out)


# --------------------------------------------------------------------------- memory bank
class MemoryO:
    """memory.py:43-269 restated for one rank (identity global->local map)."""

    def __init__(self, num_nodes, hidden_dim, slots, edge_feat_dim):
        self.N, self.D, self.K = num_nodes, hidden_dim, slots
        self.F = max(0, edge_feat_dim)
        self.S = 2 * hidden_dim + self.F
        self.memory = torch.zeros(num_nodes, hidden_dim)
        self.mailbox = torch.zeros(num_nodes, slots, self.S)
        self.mailbox_ts = torch.zeros(num_nodes, slots)
        self.memory_ts = torch.full((num_nodes,), -1.0)
        self.next_mail_pos = torch.zeros(num_nodes, dtype=torch.long)

    def clone(self) -> "MemoryO":
        m = MemoryO.__new__(MemoryO)
        m.N, m.D, m.K, m.F, m.S = self.N, self.D, self.K, self.F, self.S
        for a in ("memory", "mailbox", "mailbox_ts", "memory_ts", "next_mail_pos"):
            setattr(m, a, getattr(self, a).clone())
        return m

    def write_mailbox(self, src, dst, src_mem, dst_mem, edge_feat, ts):
        """memory.py:183-222: src pass, then dst pass."""
        F_ = self.F
        ef = edge_feat.float()
        ef = ef[..., :F_] if ef.size(-1) >= F_ else torch.cat(
            [ef, torch.zeros(*ef.shape[:-1], F_ - ef.size(-1))], dim=-1)
        src_slot = torch.cat([src_mem, dst_mem, ef], dim=-1)
        dst_slot = torch.cat([dst_mem, src_mem, ef], dim=-1)
        self._write_slots(src.long(), src_slot, ts.float())
        self._write_slots(dst.long(), dst_slot, ts.float())

    def _write_slots(self, ids, vals, ts):
        """memory.py:224-248. Duplicates within a pass all target the slot read
        once (pos = next_mail_pos[id]); the surviving value is the LAST event in
        stable ts order (the build's definition of the reference's unstable
        argsort + index_put); the slot pointer advances by the occurrence count."""
        K = self.K
        order = torch.argsort(ts, stable=True)
        ids_o, vals_o, ts_o = ids[order], vals[order], ts[order]
        uniq, inv, counts = torch.unique(ids_o, return_inverse=True, return_counts=True)
        last = torch.full((uniq.numel(),), -1, dtype=torch.long)
        last.scatter_reduce_(0, inv, torch.arange(ids_o.numel()), "amax", include_self=True)
        pos = self.next_mail_pos[uniq]
        self.mailbox[uniq, pos] = vals_o[last]
        self.mailbox_ts[uniq, pos] = ts_o[last]
        self.next_mail_pos[uniq] = (pos + counts) % K

    def apply_memory_update(self, ids, vals, ts):
        """memory.py:254-269 (ids unique): ``ts`` one time per row, or one
        for all rows (the training step's batch maximum)."""
        self.memory[ids] = vals.float()
        self.memory_ts[ids] = torch.as_tensor(ts, dtype=torch.float32)


def write_slots_serial(mem: MemoryO, ids, vals, ts):
    """The A10 rules as a serial loop (small inputs; pins MemoryO._write_slots)."""
    K = mem.K
    order = sorted(range(len(ids)), key=lambda i: (float(ts[i]), i))
    pos0 = {int(i): int(mem.next_mail_pos[int(i)]) for i in ids}
    cnt: dict[int, int] = {}
    for i in order:
        n = int(ids[i])
        mem.mailbox[n, pos0[n]] = vals[i]
        mem.mailbox_ts[n, pos0[n]] = float(ts[i])
        cnt[n] = cnt.get(n, 0) + 1
    for n, c in cnt.items():
        mem.next_mail_pos[n] = (pos0[n] + c) % K


# --------------------------------------------------------------------------- step
def negative_sample(pool_sorted: torch.Tensor, dst: torch.Tensor, generator=None) -> torch.Tensor:
    """runtime.py:124-136 (torch.randint on the given/global CPU generator)."""
    idx = torch.randint(low=0, high=pool_sorted.numel(), size=dst.shape, dtype=torch.long, generator=generator)
    neg = pool_sorted[idx]
    col = neg.eq(dst)
    if col.any():
        idx[col] = (idx[col] + 1) % pool_sorted.numel()
        neg = pool_sorted[idx]
    return neg


def prepare_roots(src, dst, ts):
    """runtime.py:138-144 + sampler.py:113 + bts_sampler.py:81: roots sorted
    unique; query time = int64(float32(int64(max ts))) = floor(max ts) here."""
    roots = torch.unique(torch.cat([src, dst])).long()
    t = int(ts.max().item())
    tq = torch.full((roots.numel(),), t, dtype=torch.long).float().to(torch.int64)
    return roots, tq


@dataclass
class Block:
    """A hop-0 block in the reference's concatenated layout."""
    src_index: torch.Tensor   # int64 [E]
    nbr: torch.Tensor         # int64 [E]
    eid: torch.Tensor         # int64 [E]
    delta_ts: torch.Tensor    # int64 [E]


def conv_all(model: LinkPredictorO, memory: torch.Tensor, roots, blk: Block, edge_feat_all,
             masks=None) -> torch.Tensor:
    """runtime.py:158-174 + build_dgl_block (models.py:170-195); ``masks`` =
    (att_mask [E,H], out_mask [R,D]) for this call's dropout."""
    if blk.nbr.numel() == 0:
        return torch.zeros(roots.numel(), model.hidden_dim)
    h_dst = memory[roots].detach()
    h_nbr = memory[blk.nbr].detach()
    ef = edge_feat_all[blk.eid].float()
    dt = blk.delta_ts.float()
    am, om = masks if masks is not None else (None, None)
    return model.conv(h_dst, h_nbr, ef, dt, blk.src_index.long(), am, om)


def select_rows(conv: torch.Tensor, roots: torch.Tensor, nodes: torch.Tensor) -> torch.Tensor:
    """runtime.py:176-183: searchsorted selection; non-roots get zeros."""
    idx = torch.searchsorted(roots, nodes).clamp(0, conv.size(0) - 1)
    valid = roots[idx] == nodes
    out = conv[idx]
    out = out * valid.unsqueeze(1).to(out.dtype)
    return out


def memory_phase(mem: MemoryO, updater: MemoryUpdaterO, src, dst, ts, edge_feat):
    """runtime.py:268-282: prev gathers, GRU over unique nodes, scatter, mailbox."""
    src_prev = mem.memory[src].clone()
    dst_prev = mem.memory[dst].clone()
    all_nodes = torch.unique(torch.cat([src, dst]))
    with torch.no_grad():
        mail = mem.mailbox[all_nodes]
        cur = mem.memory[all_nodes]
        upd = updater(mail, cur)
    mem.apply_memory_update(all_nodes, upd.detach(), float(ts.max().item()))
    mem.write_mailbox(src, dst, src_prev, dst_prev, edge_feat, ts)
    return all_nodes, upd


def loss_from_logits(pos, neg):
    return (F.binary_cross_entropy_with_logits(pos, torch.ones_like(pos))
            + F.binary_cross_entropy_with_logits(neg, torch.zeros_like(neg)))


def train_step(model, updater, optimizer, mem: MemoryO, sample_fn, src, dst, ts, edge_feat, neg, edge_feat_all,
               train=True, after_memory=None, masks=None):
    """runtime.py:225-297 for one batch (1 rank). ``sample_fn(roots, tq)``
    returns the hop-0 Block. ``after_memory(mem)`` (tests) runs between the
    memory phase and the attention, e.g. to hand the attention another
    implementation's updated memory. Without ``masks`` the attention runs
    once (dropout 0: the reference's three calls are identical); with
    ``masks`` = three (att_mask, out_mask) pairs it runs three times, for
    the src, dst and negative rows in that order (runtime.py:193-195).
    Returns a dict of the step's tensors."""
    roots, tq = prepare_roots(src, dst, ts)
    blk = sample_fn(roots, tq)
    mts_prev = mem.memory_ts.clone()
    if updater is not None:   # runtime.py:283-285: without one, memory and mailbox stay as they are
        memory_phase(mem, updater, src, dst, ts, edge_feat)
    if after_memory is not None:
        after_memory(mem)
    if train:
        model.train()
    else:
        model.eval()
    with torch.set_grad_enabled(train):
        if isinstance(model, ProjectionPredictorO):
            # time since the previous update: batch max time - memory_ts before the update (float32)
            dt = torch.tensor(float(ts.max().item()), dtype=torch.float32) - mts_prev[roots]
            conv = model.embed(mem.memory[roots].detach(), dt)
            convs = (conv, conv, conv)
        elif masks is None:
            conv = conv_all(model, mem.memory, roots, blk, edge_feat_all)
            convs = (conv, conv, conv)
        else:
            convs = tuple(conv_all(model, mem.memory, roots, blk, edge_feat_all, m) for m in masks)
            conv = convs[0]
        e_s = select_rows(convs[0], roots, src)
        e_d = select_rows(convs[1], roots, dst)
        e_n = select_rows(convs[2], roots, neg)
        pos, negl = model(e_s, e_d, e_n)
        loss = loss_from_logits(pos, negl)
    if train:
        optimizer.zero_grad(set_to_none=True)
        loss.backward()
        optimizer.step()
    return {"loss": loss.detach(), "pos": pos.detach(), "neg": negl.detach(), "conv": conv.detach(),
            "convs": tuple(c.detach() for c in convs), "roots": roots, "block": blk}


def empty_train_step(model, updater, optimizer):
    """runtime.py:248-253 with runtime.py:111-116: on an empty batch the
    backward of 0 * (sum of the model's first parameter) + 0 * (sum of the
    updater's first parameter), then an optimizer step; those two
    parameters alone have (zero) gradients."""
    model.train()
    zero = next(model.parameters()).sum() * 0.0
    if updater is not None:
        zero = zero + next(updater.parameters()).sum() * 0.0
    optimizer.zero_grad(set_to_none=True)
    zero.backward()
    optimizer.step()


def metric_dict(pos_logits, neg_logits):
    """runtime.py:202-214 (sklearn AP/AUC, pairwise 'mrr')."""
    from sklearn.metrics import average_precision_score, roc_auc_score
    pp = torch.sigmoid(pos_logits).cpu()
    pn = torch.sigmoid(neg_logits).cpu()
    scores = torch.cat([pp, pn]).numpy()
    labels = torch.cat([torch.ones_like(pp), torch.zeros_like(pn)]).numpy()
    return {"ap": float(average_precision_score(labels, scores)), "auc": float(roc_auc_score(labels, scores)),
            "mrr": float((pp.unsqueeze(1) > pn.unsqueeze(0)).float().mean().item())}


def block_from_oracle_sampler(g, roots, tq, fanout):
    """Hop 0 of the C sampler oracle as a Block."""
    import sampler_oracle as so
    out = so.sample_layer(g, roots.numpy(), tq.numpy(), fanout)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    return Block(t(out["src_index"]), t(out["sample_nodes"]), t(out["eid"]), t(out["delta_ts"]))
