"""Pins the parts of the step oracle (oracle/ctdg_oracle.py) that the GPU
parity tests rely on and that no library routine fixes by itself:

* edge predictor + root selection + BCE (LinkPredictorO, select_rows,
  loss_from_logits) against a float64 per-event loop written from
  models.py:313-324 and runtime.py:176-183,290-292: a node that is not a root
  gets a zero embedding, negatives go through dst_fc, the loss is the sum of
  the two mean BCE terms;
* the ordering of one training step (train_step, memory_phase, conv_all,
  MemoryO.write_mailbox) on a 3-event batch whose expected memory, mailbox,
  slot pointers and attention inputs are worked out by hand in the comments:
  messages carry the memory from BEFORE the update (runtime.py:270-271), the
  attention reads the memory AFTER it (runtime.py:172 after :279), the src
  pass precedes the dst pass (memory.py:220-221), tied timestamps keep the
  last event in stable order, slot pointers advance by the occurrence count
  (memory.py:245-248);
* the metric dict (metric_dict, runtime.py:202-214) against AP / AUC / "mrr"
  from their definitions.

Each pin is also run against planted mistakes in the oracle (monkeypatched
variants below) and must fail on every one of them."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import ctdg_oracle as co


# --------------------------------------------------------------------------- predictor
def _softplus(x: float) -> float:
    return max(x, 0.0) + math.log1p(math.exp(-abs(x)))


def _brute_predictor(P, roots, conv, src, dst, neg):
    """Per event, in float64: e(x) = conv row of x if x is a root else 0;
    pos = w_o relu(W_s e_s + b_s + W_d e_d + b_d) + b_o, neg the same with
    e_n through W_d; loss = mean softplus(-pos) + mean softplus(neg)."""
    row = {int(r): i for i, r in enumerate(roots)}
    D = conv.shape[1]

    def emb(x):
        return conv[row[x]] if x in row else np.zeros(D)

    pos, ngl = [], []
    for s, d, n in zip(src.tolist(), dst.tolist(), neg.tolist()):
        hs = P["src_fc.weight"] @ emb(s) + P["src_fc.bias"]
        hd = P["dst_fc.weight"] @ emb(d) + P["dst_fc.bias"]
        hn = P["dst_fc.weight"] @ emb(n) + P["dst_fc.bias"]
        pos.append(float(P["out_fc.weight"][0] @ np.maximum(hs + hd, 0.0) + P["out_fc.bias"][0]))
        ngl.append(float(P["out_fc.weight"][0] @ np.maximum(hs + hn, 0.0) + P["out_fc.bias"][0]))
    loss = np.mean([_softplus(-p) for p in pos]) + np.mean([_softplus(q) for q in ngl])
    return np.array(pos), np.array(ngl), float(loss)


def _predictor_case(seed):
    torch.manual_seed(seed)
    rng = np.random.default_rng(seed)
    D = 9
    model = co.LinkPredictorO(D, 3, 4, 1).double()
    roots = torch.tensor(sorted(rng.choice(np.arange(5, 60), 12, replace=False).tolist()))
    conv = torch.randn(roots.numel(), D, dtype=torch.float64)
    B = 40
    src = roots[torch.as_tensor(rng.integers(0, roots.numel(), B))]
    dst = roots[torch.as_tensor(rng.integers(0, roots.numel(), B))]
    # negatives: roots, non-roots between roots, below the smallest and above
    # the largest root (searchsorted lands on 0 / R there), the largest root
    neg = torch.as_tensor(rng.integers(0, 70, B))
    neg[:4] = torch.tensor([0, 69, int(roots[-1]), int(roots[0])])
    return model, roots, conv, src, dst, neg


def _oracle_predictor(model, roots, conv, src, dst, neg):
    e_s = co.select_rows(conv, roots, src)
    e_d = co.select_rows(conv, roots, dst)
    e_n = co.select_rows(conv, roots, neg)
    pos, ngl = model(e_s, e_d, e_n)
    return pos.detach().numpy(), ngl.detach().numpy(), float(co.loss_from_logits(pos, ngl).detach())


def _check_predictor(seed):
    model, roots, conv, src, dst, neg = _predictor_case(seed)
    assert int((~torch.isin(neg, roots)).sum()) >= 5 and int(torch.isin(neg, roots).sum()) >= 5
    P = {n: p.detach().numpy() for n, p in model.named_parameters()}
    want = _brute_predictor(P, roots.numpy(), conv.numpy(), src, dst, neg)
    got = _oracle_predictor(model, roots, conv, src, dst, neg)
    np.testing.assert_allclose(got[0], want[0], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(got[1], want[1], rtol=1e-12, atol=1e-12)
    assert abs(got[2] - want[2]) <= 1e-12 * abs(want[2])


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_predictor_selection_bce_match_brute_force(seed):
    _check_predictor(seed)


def _sel_no_zero(conv, roots, nodes):
    idx = torch.searchsorted(roots, nodes).clamp(0, conv.size(0) - 1)
    return conv[idx]


def _fwd_neg_src_fc(self, src_conv, dst_conv, neg_conv):
    h_src = self.src_fc(src_conv)
    pos = self.out_fc(F.relu(h_src + self.dst_fc(dst_conv))).squeeze(-1)
    neg = self.out_fc(F.relu(h_src + self.src_fc(neg_conv))).squeeze(-1)
    return pos, neg


def _fwd_no_relu(self, src_conv, dst_conv, neg_conv):
    h_src = self.src_fc(src_conv)
    pos = self.out_fc(h_src + self.dst_fc(dst_conv)).squeeze(-1)
    neg = self.out_fc(h_src + self.dst_fc(neg_conv)).squeeze(-1)
    return pos, neg


def _loss_neg_label_one(pos, neg):
    return (F.binary_cross_entropy_with_logits(pos, torch.ones_like(pos))
            + F.binary_cross_entropy_with_logits(neg, torch.ones_like(neg)))


def _loss_sum(pos, neg):
    return (F.binary_cross_entropy_with_logits(pos, torch.ones_like(pos), reduction="sum")
            + F.binary_cross_entropy_with_logits(neg, torch.zeros_like(neg), reduction="sum"))


@pytest.mark.parametrize("plant", ["non-root not zeroed", "negatives through src_fc", "no relu",
                                   "negative label 1", "summed BCE"])
def test_predictor_pin_catches_planted_mistakes(monkeypatch, plant):
    patch = {"non-root not zeroed": (co, "select_rows", _sel_no_zero),
             "negatives through src_fc": (co.LinkPredictorO, "forward", _fwd_neg_src_fc),
             "no relu": (co.LinkPredictorO, "forward", _fwd_no_relu),
             "negative label 1": (co, "loss_from_logits", _loss_neg_label_one),
             "summed BCE": (co, "loss_from_logits", _loss_sum)}[plant]
    monkeypatch.setattr(*patch)
    with pytest.raises(AssertionError):
        _check_predictor(0)


# --------------------------------------------------------------------------- one hand-worked step
def _hand_step():
    """5 nodes, D = 2, F = 1, K = 2 slots, T = 2, one head.

    Initial memory[n] = [n+1, -(n+1)], next_mail_pos = [0, 1, 0, 0, 0], mailbox 0.
    Events (src -> dst, ts, edge feature):
      e0: 0 -> 1, 10.0, 0.5
      e1: 2 -> 1, 10.0, 0.25   (ties e0's time; node 1 is dst twice)
      e2: 1 -> 3, 12.7, 0.125
    negatives [4, 1, 4]: node 4 is no root, node 1 is.
    Roots = [0, 1, 2, 3]; query time = floor(12.7) = 12 for each.
    The updater's weights are zero and its biases zero, so every gate is
    sigmoid(0) = 1/2 and every candidate tanh(0) = 0: the mailbox GRU gives 0
    and the GRUCell gives 1/2 * memory. Updated memory of the roots:
      0: [0.5,-0.5]  1: [1,-1]  2: [1.5,-1.5]  3: [2,-2]; node 4 stays [5,-5];
    memory_ts of the roots = float32(12.7), node 4 keeps -1.
    Mailbox, messages [self_prev | other_prev | feat] from the memory BEFORE
    the update:
      src pass (pointers read once: 0->0, 2->0, 1->1):
        node 0 slot 0 = [1,-1, 2,-2, .5] ts 10;   pointer 0 -> 1
        node 2 slot 0 = [3,-3, 2,-2, .25] ts 10;  pointer 0 -> 1
        node 1 slot 1 = [2,-2, 4,-4, .125] ts 12.7; pointer 1 -> 0
      dst pass (node 1 now at pointer 0; e0, e1 tie at ts 10: e1 is last
      in stable order and wins; node 1 occurs twice):
        node 1 slot 0 = [2,-2, 3,-3, .25] ts 10;  pointer 0 -> (0+2) % 2 = 0
        node 3 slot 0 = [4,-4, 2,-2, .125] ts 12.7; pointer 0 -> 1
    The attention block (handed in): root 1 has neighbours 0 (eid 0) and 2
    (eid 1), both dt 2; root 3 has neighbour 1 (eid 2), dt 0. It reads the
    memory AFTER the update: h_dst = the updated rows above, h_nbr =
    [[.5,-.5], [1.5,-1.5], [1,-1]]."""
    torch.manual_seed(0)
    model, updater = co.build_models(2, 1, 2, 1, 2, seed=0)
    with torch.no_grad():
        for p in updater.parameters():
            p.zero_()
    mem = co.MemoryO(5, 2, 2, 1)
    mem.memory = torch.tensor([[1.0, -1.0], [2.0, -2.0], [3.0, -3.0], [4.0, -4.0], [5.0, -5.0]])
    mem.next_mail_pos = torch.tensor([0, 1, 0, 0, 0])
    src, dst = torch.tensor([0, 2, 1]), torch.tensor([1, 1, 3])
    ts = torch.tensor([10.0, 10.0, 12.7])
    ef = torch.tensor([[0.5], [0.25], [0.125]])
    neg = torch.tensor([4, 1, 4])
    edge_feat_all = torch.tensor([[0.5], [0.25], [0.125], [7.0]])
    seen = {}

    def sample_fn(roots, tq):
        seen["roots"], seen["tq"] = roots.clone(), tq.clone()
        return co.Block(src_index=torch.tensor([1, 1, 3]), nbr=torch.tensor([0, 2, 1]), eid=torch.tensor([0, 1, 2]),
                        delta_ts=torch.tensor([2, 2, 0]))

    conv_fwd, model_fwd = model.conv.forward, model.forward

    def conv_rec(h_dst, h_nbr, ef_, dt, edge_dst, *masks):
        seen["conv_in"] = (h_dst.detach().clone(), h_nbr.detach().clone(), ef_.clone(), dt.clone(), edge_dst.clone())
        out = conv_fwd(h_dst, h_nbr, ef_, dt, edge_dst, *masks)
        seen["conv_out"] = out.detach().clone()
        return out

    def model_rec(e_s, e_d, e_n):
        seen["emb"] = (e_s.detach().clone(), e_d.detach().clone(), e_n.detach().clone())
        return model_fwd(e_s, e_d, e_n)

    model.conv.forward = conv_rec
    model.forward = model_rec
    opt = torch.optim.Adam(list(model.parameters()) + list(updater.parameters()), lr=1e-3)
    co.train_step(model, updater, opt, mem, sample_fn, src, dst, ts, ef, neg, edge_feat_all)
    return mem, seen


def _check_hand_step():
    mem, seen = _hand_step()
    assert seen["roots"].tolist() == [0, 1, 2, 3] and seen["tq"].tolist() == [12] * 4
    t127 = float(np.float32(12.7))
    assert mem.memory.tolist() == [[0.5, -0.5], [1.0, -1.0], [1.5, -1.5], [2.0, -2.0], [5.0, -5.0]]
    assert mem.memory_ts.tolist() == [t127] * 4 + [-1.0]
    want_box = torch.zeros(5, 2, 5)
    want_ts = torch.zeros(5, 2)
    for n, slot, row, t in ((0, 0, [1, -1, 2, -2, .5], 10.0), (2, 0, [3, -3, 2, -2, .25], 10.0),
                            (1, 1, [2, -2, 4, -4, .125], t127), (1, 0, [2, -2, 3, -3, .25], 10.0),
                            (3, 0, [4, -4, 2, -2, .125], t127)):
        want_box[n, slot] = torch.tensor(row, dtype=torch.float32)
        want_ts[n, slot] = t
    assert torch.equal(mem.mailbox, want_box)
    assert torch.equal(mem.mailbox_ts, want_ts)
    assert mem.next_mail_pos.tolist() == [1, 0, 1, 1, 0]
    h_dst, h_nbr, ef_, dt, edge_dst = seen["conv_in"]
    assert h_dst.tolist() == [[0.5, -0.5], [1.0, -1.0], [1.5, -1.5], [2.0, -2.0]]
    assert h_nbr.tolist() == [[0.5, -0.5], [1.5, -1.5], [1.0, -1.0]]
    assert ef_.tolist() == [[0.5], [0.25], [0.125]]
    assert dt.tolist() == [2.0, 2.0, 0.0] and dt.dtype == torch.float32
    assert edge_dst.tolist() == [1, 1, 3]
    conv = seen["conv_out"]
    e_s, e_d, e_n = seen["emb"]
    assert torch.equal(e_s, conv[[0, 2, 1]]) and torch.equal(e_d, conv[[1, 1, 3]])
    assert torch.equal(e_n[1], conv[1]) and not bool(e_n[0].any()) and not bool(e_n[2].any())


def test_hand_worked_step():
    _check_hand_step()


def _plant_messages_post_update(monkeypatch):
    orig = co.MemoryO.apply_memory_update

    def memory_phase(mem, updater, src, dst, ts, edge_feat):
        all_nodes = torch.unique(torch.cat([src, dst]))
        with torch.no_grad():
            upd = updater(mem.mailbox[all_nodes], mem.memory[all_nodes])
        orig(mem, all_nodes, upd.detach(), float(ts.max().item()))
        mem.write_mailbox(src, dst, mem.memory[src].clone(), mem.memory[dst].clone(), edge_feat, ts)
        return all_nodes, upd
    monkeypatch.setattr(co, "memory_phase", memory_phase)


def _plant_conv_pre_update(monkeypatch):
    phase, conv_all = co.memory_phase, co.conv_all
    snap = {}

    def memory_phase(mem, *a):
        snap["m"] = mem.memory.clone()
        return phase(mem, *a)

    monkeypatch.setattr(co, "memory_phase", memory_phase)
    monkeypatch.setattr(co, "conv_all", lambda model, memory, *a: conv_all(model, snap["m"], *a))


def _plant_dst_pass_first(monkeypatch):
    def write_mailbox(self, src, dst, src_mem, dst_mem, edge_feat, ts):
        ef = edge_feat.float()[..., :self.F]
        self._write_slots(dst.long(), torch.cat([dst_mem, src_mem, ef], -1), ts.float())
        self._write_slots(src.long(), torch.cat([src_mem, dst_mem, ef], -1), ts.float())
    monkeypatch.setattr(co.MemoryO, "write_mailbox", write_mailbox)


def _plant_first_writer(monkeypatch):
    orig = co.MemoryO._write_slots

    def write_slots(self, ids, vals, ts):   # the reverse order keeps the first event of a tie
        rev = torch.arange(ids.numel() - 1, -1, -1)
        orig(self, ids[rev], vals[rev], ts[rev])
    monkeypatch.setattr(co.MemoryO, "_write_slots", write_slots)


def _plant_advance_by_one(monkeypatch):
    orig = co.MemoryO._write_slots

    def write_slots(self, ids, vals, ts):
        uniq = torch.unique(ids)
        pos = self.next_mail_pos[uniq].clone()
        orig(self, ids, vals, ts)
        self.next_mail_pos[uniq] = (pos + 1) % self.K
    monkeypatch.setattr(co.MemoryO, "_write_slots", write_slots)


def _plant_query_time_ceil(monkeypatch):
    orig = co.prepare_roots

    def prepare_roots(src, dst, ts):
        roots, tq = orig(src, dst, ts)
        return roots, torch.full_like(tq, int(math.ceil(float(ts.max()))))
    monkeypatch.setattr(co, "prepare_roots", prepare_roots)


@pytest.mark.parametrize("plant", [_plant_messages_post_update, _plant_conv_pre_update, _plant_dst_pass_first,
                                   _plant_first_writer, _plant_advance_by_one, _plant_query_time_ceil],
                         ids=lambda f: f.__name__[len("_plant_"):])
def test_hand_step_catches_planted_mistakes(monkeypatch, plant):
    plant(monkeypatch)
    with pytest.raises(AssertionError):
        _check_hand_step()


# --------------------------------------------------------------------------- metrics
def _brute_metrics(pos_logits, neg_logits):
    """AP = sum over descending distinct score thresholds of (recall step) x
    precision; AUC = P(score_pos > score_neg) + P(tie) / 2 over all pairs;
    "mrr" = mean over pairs of [pos > neg] (runtime.py:211)."""
    sp = 1.0 / (1.0 + np.exp(-pos_logits.astype(np.float64)))
    sn = 1.0 / (1.0 + np.exp(-neg_logits.astype(np.float64)))
    sp, sn = sp.astype(np.float32).astype(np.float64), sn.astype(np.float32).astype(np.float64)
    scores = np.concatenate([sp, sn])
    labels = np.concatenate([np.ones(sp.size), np.zeros(sn.size)])
    ap, prev_r = 0.0, 0.0
    for thr in sorted(set(scores.tolist()), reverse=True):
        sel = scores >= thr
        tp = labels[sel].sum()
        r = tp / labels.sum()
        ap += (r - prev_r) * (tp / sel.sum())
        prev_r = r
    gt = (sp[:, None] > sn[None, :]).mean()
    eq = (sp[:, None] == sn[None, :]).mean()
    return {"ap": ap, "auc": gt + 0.5 * eq, "mrr": gt}


@pytest.mark.parametrize("seed", [0, 1])
def test_metric_dict_matches_definitions(seed):
    rng = np.random.default_rng(seed)
    pos = rng.normal(0.5, 1.0, 300).astype(np.float32)
    neg = rng.normal(-0.2, 1.0, 300).astype(np.float32)
    pos[:20] = neg[:20]            # ties across the classes
    pos[20:40] = 30.0              # saturated: sigmoid ties at 1.0
    got = co.metric_dict(torch.from_numpy(pos), torch.from_numpy(neg))
    want = _brute_metrics(pos, neg)
    for k, tol in (("ap", 1e-9), ("auc", 1e-9), ("mrr", 1e-6)):   # "mrr" is a float32 mean
        assert abs(got[k] - want[k]) <= tol, (k, got[k], want[k])


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_product_metrics_match_sklearn(seed):
    """The runtime's metric dict (metrics.link_metrics, sorts on the logits'
    device; here the CPU) against the oracle's scikit-learn metric_dict,
    with ties within and across the classes."""
    from starry_unigraph.backends.ctdg.runtime.metrics import link_metrics
    rng = np.random.default_rng(seed)
    pos = torch.from_numpy(rng.normal(0.3, 1.0, 257).astype(np.float32))
    neg = torch.from_numpy(rng.normal(-0.1, 1.0, 257).astype(np.float32))
    pos[:30] = neg[:30]
    neg[30:40] = neg[40]
    pos[50:60] = 40.0
    got = link_metrics(pos, neg)
    want = co.metric_dict(pos, neg)
    for k, tol in (("ap", 1e-9), ("auc", 1e-9), ("mrr", 1e-6)):   # the reference's "mrr" is a float32 mean
        assert abs(got[k] - want[k]) <= tol, (k, got[k], want[k])


def test_philox_known_answers():
    """The oracle's Philox4x32-10 (the dropout masks' generator) against the
    known-answer vectors published with Random123 (Salmon et al., SC 2011)."""
    kat = [((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
           ((0xffffffff,) * 4, (0xffffffff, 0xffffffff), (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
           ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
            (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1))]
    for ctr, key, want in kat:
        got = co.philox4x32_10(np.array(ctr, dtype=np.uint32), np.array(key, dtype=np.uint32))
        assert got.tolist() == list(want)


def test_oracle_dropout_masks_scale_and_rate():
    """Mask values are 0 or 1/(1-p); p = 0 keeps everything."""
    att, out = co.dropout_masks(3, 7, 1, 500, 20, 4, 64, 0.2, 0.0)
    assert set(np.unique(att).tolist()) == {0.0, np.float32(1 / 0.8)}
    assert abs(float((att > 0).mean()) - 0.8) < 0.01
    assert bool((out == 1.0).all())


def test_time_projection_closed_form():
    """Config 2's JODIE embedding in the oracle: y = h * (1 + w x + b) with
    x = (dt - shift) * scale, written out for two roots."""
    m = co.ProjectionPredictorO(3, shift=10.0, scale=0.5)
    with torch.no_grad():
        m.time_proj.proj.weight.copy_(torch.tensor([[1.0], [-2.0], [0.5]]))
        m.time_proj.proj.bias.copy_(torch.tensor([0.0, 1.0, -1.0]))
    h = torch.tensor([[1.0, 2.0, 3.0], [4.0, -1.0, 2.0]])
    dt = torch.tensor([14.0, 10.0])   # x = 2, 0
    y = m.embed(h, dt)
    # root 0: 1+w*2+b = [3, -2, 1]; root 1: 1+b = [1, 2, 0]
    assert y.tolist() == [[3.0, -4.0, 3.0], [4.0, -2.0, 0.0]]
