"""Dropout in the attention kernels (models.py:127 att_dropout, models.py:136
output dropout; the reference's default config sets both to 0.1):

* the device masks (sgl_dropout_masks, the kernels' Philox4x32-10 draws)
  equal the oracle's restatement, whose generator is pinned by the published
  known-answer vectors (tests/test_oracle_pins.py);
* keep rates and the 1/(1-p) scale hold statistically, passes and steps
  draw independent masks;
* one attention pass with dropout (forward and all 12 parameter gradients)
  equals torch autograd through the oracle with the same masks replayed;
* teacher-forced training steps with dropout (three passes with their own
  masks for the src, dst and negative rows, runtime.py:193-195) match the
  oracle step replaying the three passes' masks: loss and logits within
  rtol 1e-3, gradients against the same step in float64.
With dropout 0 the kernels are the dropout-free instances (every other GPU
test)."""
import copy

import numpy as np
import pytest
import torch

import ctdg_oracle as co
import sampler_oracle as so

pytestmark = pytest.mark.gpu


def _masks(rows, fanout, H, D, pa, po, seed, step, pas, gpu):
    from starry_unigraph.lib import _capi
    att = torch.full((rows, fanout, H), -1.0, device=gpu)
    out = torch.full((rows, D), -1.0, device=gpu)
    st = torch.tensor([step], dtype=torch.int64, device=gpu)
    P = _capi.ptr
    _capi.check(_capi.lib().sgl_dropout_masks(rows, fanout, H, D, pa, po, seed, P(st), pas, P(att), P(out),
                                              _capi.stream_of(gpu)), "sgl_dropout_masks")
    torch.cuda.synchronize()
    return att.cpu(), out.cpu()


@pytest.mark.parametrize("seed,step,pas,pa,po", [(0, 1, 0, 0.1, 0.1), (123456789012345, 2 ** 33 + 7, 2, 0.5, 0.25),
                                                 (7, 99, 1, 0.0, 0.3)])
def test_device_masks_match_oracle(gpu, seed, step, pas, pa, po):
    att, out = _masks(300, 13, 4, 37, pa, po, seed, step, pas, gpu)
    wa, wo = co.dropout_masks(seed, step, pas, 300, 13, 4, 37, pa, po)
    assert torch.equal(att, torch.from_numpy(wa))
    assert torch.equal(out, torch.from_numpy(wo))


def test_mask_statistics(gpu):
    """Keep rates within 6 standard deviations of 1 - p over ~10^6 entries;
    kept entries are exactly 1/(1-p); other passes / steps / seeds give
    masks that agree only at the rate of independent draws."""
    p = 0.1
    att, out = _masks(20000, 20, 4, 100, p, p, 5, 10, 0, gpu)
    for m in (att.flatten(), out.flatten()):
        kept = m != 0
        n = m.numel()
        rate = float(kept.double().mean())
        assert abs(rate - (1 - p)) < 6 * (p * (1 - p) / n) ** 0.5, rate
        assert bool((m[kept] == np.float32(1 / (1 - p))).all())
    base = att != 0
    for other in (_masks(20000, 20, 4, 100, p, p, 5, 10, 1, gpu)[0], _masks(20000, 20, 4, 100, p, p, 5, 11, 0, gpu)[0],
                  _masks(20000, 20, 4, 100, p, p, 6, 10, 0, gpu)[0]):
        agree = float((base == (other != 0)).double().mean())
        want = (1 - p) ** 2 + p ** 2
        assert abs(agree - want) < 0.005, agree


class _Wrap:
    def __init__(self, conv):
        self.conv = conv
        self.hidden_dim = conv.dim_out


@pytest.mark.parametrize("H,k,D,F,T,pa,po", [(2, 10, 32, 6, 16, 0.1, 0.1), (4, 20, 32, 6, 16, 0.3, 0.0),
                                              (2, 10, 100, 16, 100, 0.0, 0.2), (2, 10, 100, 172, 100, 0.25, 0.25)])
def test_attention_pass_with_dropout_matches_autograd(gpu, H, k, D, F, T, pa, po):
    """One attention pass with dropout (the module's forward: pass 0, fresh
    masks per call) against the oracle conv with the same masks: embeddings
    and the 12 parameter gradients (torch autograd through the masked
    softmax and the masked output projection)."""
    from starry_unigraph.backends.ctdg.runtime.models import TemporalTransformerConv
    from starry_unigraph.native.step import ConvDims, DeviceStep, NodeState
    from starry_unigraph.native.tcsr import RecentSampler, build_tcsr
    rng = np.random.default_rng(H + k)
    N, E, R = 400, 3000, 150
    row, col = rng.integers(0, N, E), np.minimum(rng.zipf(1.3, E) - 1, N - 1)
    ts = np.sort(rng.integers(0, 10 ** 6, E))
    roots = np.sort(rng.choice(N, R, replace=False))
    tq = np.full(R, 10 ** 6 // 2, dtype=np.int64)
    mem, ef = torch.randn(N, D), torch.randn(E, F)
    torch.manual_seed(1)
    conv = TemporalTransformerConv(D, F, T, H, D, dropout=po, att_dropout=pa).to(gpu)
    with torch.no_grad():
        conv.time_enc.w.bias.uniform_(-1, 1)
        conv.w_v.bias.uniform_(-1, 1)      # the value bias enters with the kept-weight sums
        conv.layer_norm.weight.uniform_(0.5, 1.5)
    conv.train()
    ref = co.TemporalConvO(D, F, T, H, D)
    ref.load_state_dict({kk: v.cpu() for kk, v in conv.state_dict().items()})
    st = NodeState(N, D, 1, F, gpu)
    st.memory.copy_(mem)
    step = DeviceStep(st, ConvDims(D, F, T, H, k), R)
    b = step.buf
    b.roots[:R] = torch.as_tensor(roots, device=gpu)
    b.root_ts[:R] = torch.as_tensor(tq, device=gpu)
    b.num_roots.fill_(R)
    b.num_roots64.fill_(R)
    b.new_mem[:R] = mem[roots].to(gpu)
    g = build_tcsr(N, torch.as_tensor(row), torch.as_tensor(col), None, torch.as_tensor(ts))
    step.sample(RecentSampler(g))
    b.any_edges.fill_(1)
    y = conv(step, ef.to(gpu))
    gy = torch.randn(R, D)
    (y[:R] * gy.to(gpu)).sum().backward()
    # the masks this call drew (the module advanced the buffers' step counter to 1)
    assert int(b.rng_step.item()) == 1
    att, out = _masks(R, k, H, D, pa, po, conv.dropout_seed, 1, 0, gpu)
    cnt = b.hop.cnt[:R].long().cpu()
    live = torch.arange(k)[None, :] < cnt[:, None]
    og = so.build_tcsr(N, row, col, np.arange(E), ts)
    blk = co.block_from_oracle_sampler(og, torch.as_tensor(roots), torch.as_tensor(tq), k)
    assert blk.nbr.numel() == int(live.sum())
    yr = co.conv_all(_Wrap(ref), mem, torch.as_tensor(roots), blk, ef, masks=(att[live], out))
    (yr * gy).sum().backward()
    torch.testing.assert_close(y[:R].cpu().double(), yr.double(), rtol=1e-3, atol=2e-4)
    if pa > 0 or po > 0:
        assert float((att[live] == 0).float().mean() + (out == 0).float().mean()) > 0   # something was dropped
    for (name, p), (_, pr) in zip(conv.named_parameters(), ref.named_parameters()):
        scale = float(pr.grad.abs().max()) + 1e-6
        torch.testing.assert_close(p.grad.cpu().double(), pr.grad.double(), rtol=2e-3, atol=2e-4 * scale,
                                   msg=lambda m: f"grad {name}: {m}")


def test_train_steps_with_dropout_match_oracle(gpu):
    """The reference's default dropout (0.1 / 0.1) in training steps at the
    cfg4 dimensions (D = T = 100, F = 16, H = 2, k = 10, B = 600 on a reduced
    stream of the cfg4 generator): three attention passes with independent
    masks, teacher-forced against the oracle replaying each pass's masks."""
    from starry_unigraph import SchedulerSession, synth
    from starry_unigraph.data import from_stream
    s = synth.unipartite_stream(num_nodes=30000, num_events=120000, seed=0)
    D, T, H, k, K, B, F = 100, 100, 2, 10, 1, 600, 16
    cfg = {"model": {"family": "tgn", "hidden_dim": D}, "data": {"name": "drop", "format": "synthetic"},
           "train": {"batch_size": B, "lr": 1e-3}, "runtime": {"device": "cuda"},
           "ctdg": {"mailbox_slots": K, "dim_time": T, "num_head": H, "dropout": 0.1, "att_dropout": 0.1},
           "sampling": {"neighbor_limit": [k], "history": 1, "strategy": "recent"}}
    torch.manual_seed(0)
    sess = SchedulerSession.from_config(cfg).with_events(from_stream(s))
    sess.build_runtime()
    rt = sess.ctdg_session.online_runtime
    assert rt.step.buf.passes == 3
    conv = rt.model.conv
    model, upd = co.build_models(D, F, T, H, K, seed=0)
    model.load_state_dict({kk: v.cpu() for kk, v in rt.model.state_dict().items()})
    upd.load_state_dict({kk: v.cpu() for kk, v in rt.memory_updater.state_dict().items()})
    opt = torch.optim.Adam(list(model.parameters()) + list(upd.parameters()), lr=1e-3)
    g = torch.Generator().manual_seed(1)
    N = rt.dataset.num_nodes
    mem = co.MemoryO(N, D, K, F)
    mem.memory = torch.rand(N, D, generator=g) * 2 - 1
    mem.mailbox = torch.randn(N, K, 2 * D + F, generator=g) * 0.5
    gr = rt.dataset.sampler_graph("train")
    og = so.build_tcsr(N, gr["row"].numpy(), gr["col"].numpy(), gr["eid"].numpy(), gr["ts"].numpy())
    pool = rt.dataset.dst.unique()
    gen = torch.Generator().manual_seed(5)
    batches = list(rt.iter_batches("train", B))
    for i in (60, 61, 62):
        batch = batches[i]
        neg = co.negative_sample(pool, batch.dst, gen)
        with torch.no_grad():
            for p, q in zip(rt.model.parameters(), model.parameters()):
                p.copy_(q)
        st = rt.memory.state
        for name in ("memory", "mailbox", "mailbox_ts", "memory_ts"):
            getattr(st, name).copy_(getattr(mem, name))
        st.next_mail_pos.copy_(mem.next_mail_pos.to(torch.int32))
        st.touched()
        rt._neg_queue["train"] = (neg.to(gpu), 0)
        out = rt.train_step(batch)
        buf = rt.step.buf
        U = int(buf.num_roots.item())
        step_no = int(buf.rng_step.item())
        cnt = buf.hop.cnt[:U].long().cpu()
        live = torch.arange(k)[None, :] < cnt[:, None]
        masks = []
        for pas in range(3):
            a, o = _masks(U, k, H, D, 0.1, 0.1, conv.dropout_seed, step_no, pas, gpu)
            masks.append((a[live], o))
        model64 = copy.deepcopy(model).double()
        ref = co.train_step(model, upd, opt, mem, lambda r, t: co.block_from_oracle_sampler(og, r, t, k),
                            batch.src, batch.dst, batch.ts, batch.edge_feat, neg, rt.dataset.edge_feat, masks=masks)
        rl = float(ref["loss"])
        assert abs(out["loss"] - rl) <= 1e-3 * abs(rl) + 1e-6, (i, out["loss"], rl)
        np.testing.assert_allclose(out["predictions"], torch.sigmoid(ref["pos"]).numpy(), rtol=1e-3, atol=1e-5)
        torch.testing.assert_close(buf.neg[:batch.size].cpu(), ref["neg"], rtol=1e-3,
                                   atol=1e-3 * float(ref["neg"].abs().max()))
        # the three passes' embeddings differ (independent masks)
        y = buf.y.view(3, buf.y_rows, D)[:, :U].cpu()
        assert not torch.equal(y[0], y[1]) and not torch.equal(y[1], y[2])
        for pas in range(3):
            torch.testing.assert_close(y[pas], ref["convs"][pas], rtol=1e-3, atol=2e-4)
        # gradients against the same step in float64 (time arguments rounded as in float32)
        model64.conv.time_enc.round_arg_f32 = True
        blk, roots = ref["block"], ref["roots"]
        m = mem.memory.double()
        convs = [model64.conv(m[roots], m[blk.nbr], rt.dataset.edge_feat[blk.eid].double(), blk.delta_ts.float(),
                              blk.src_index.long(), *mk) for mk in masks]
        pos, ngl = model64(co.select_rows(convs[0], roots, batch.src), co.select_rows(convs[1], roots, batch.dst),
                           co.select_rows(convs[2], roots, neg))
        co.loss_from_logits(pos, ngl).backward()
        for (pn, p), q in zip(rt.model.named_parameters(), model64.parameters()):
            scale = float(q.grad.abs().max()) + 1e-12
            torch.testing.assert_close(p.grad.cpu().double(), q.grad, rtol=2e-3, atol=1e-3 * scale,
                                       msg=lambda msg: f"grad {pn} batch {i}: {msg}")
