"""Pins the torch-CPU step oracle (oracle/ctdg_oracle.py) against
independent statements: textbook GRU gate equations in float64, a per-root
brute-force attention loop, invariants of the attention, and a serial loop of
the mailbox write rules."""
import math

import numpy as np
import pytest
import torch

import ctdg_oracle as co


def _sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def _gru_cell_np(x, h, w_ih, w_hh, b_ih, b_hh):
    """PyTorch GRU gate order (r, z, n): n = tanh(W_in x + b_in + r*(W_hn h + b_hn))."""
    D = h.shape[-1]
    gi = x @ w_ih.T + b_ih
    gh = h @ w_hh.T + b_hh
    r = _sig(gi[:, :D] + gh[:, :D])
    z = _sig(gi[:, D:2 * D] + gh[:, D:2 * D])
    n = np.tanh(gi[:, 2 * D:] + r * gh[:, 2 * D:])
    return (1 - z) * n + z * h


@pytest.mark.parametrize("K", [1, 3])
def test_memory_updater_matches_gate_equations(K):
    torch.manual_seed(0)
    D, S, M = 12, 31, 9
    up = co.MemoryUpdaterO(D, S, K).double()
    mail = torch.randn(M, K, S, dtype=torch.float64)
    mem = torch.randn(M, D, dtype=torch.float64)
    got = up(mail, mem).detach().numpy()
    g, c = up.mail_aggregator, up.memory_cell
    p = lambda t: t.detach().numpy()
    h = np.zeros((M, D))
    for k in range(K):                                   # slot index order, h0 = 0
        h = _gru_cell_np(mail[:, k].numpy(), h, p(g.weight_ih_l0), p(g.weight_hh_l0), p(g.bias_ih_l0),
                         p(g.bias_hh_l0))
    want = _gru_cell_np(h, mem.numpy(), p(c.weight_ih), p(c.weight_hh), p(c.bias_ih), p(c.bias_hh))
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_time_encode_closed_form():
    te = co.TimeEncodeO(7)
    w = 1.0 / 10 ** np.linspace(0, 9, 7)
    assert np.allclose(te.w.weight.detach().numpy()[:, 0], w, rtol=1e-6)
    assert np.all(te.w.bias.detach().numpy() == 0)
    t = torch.tensor([0.0, 1.5, 1e6, 2e8])
    # the argument is the float32 product (Linear in fp32), cos taken of that value
    arg = (t.numpy()[:, None] * te.w.weight.detach().numpy()[:, 0][None, :]).astype(np.float32)
    np.testing.assert_allclose(te(t).detach().numpy(), np.cos(arg.astype(np.float64)), rtol=1e-5, atol=1e-6)


def _brute_conv(conv, h_dst, h_nbr, ef, dt, edge_dst):
    """Per root, per head: explicit scores, softmax, weighted sum (float64)."""
    P = {n: p.detach().double().numpy() for n, p in conv.named_parameters()}
    R, D = h_dst.shape
    H = conv.num_head
    dh = D // H
    w, b = P["time_enc.w.weight"][:, 0], P["time_enc.w.bias"]
    out = np.zeros((R, D))
    for r in range(R):
        q_in = np.concatenate([h_dst[r], np.cos(b)])
        q = P["w_q.weight"] @ q_in + P["w_q.bias"]
        es = [e for e in range(len(edge_dst)) if edge_dst[e] == r]
        agg = np.zeros(D)
        for hh in range(H):
            sl = slice(hh * dh, (hh + 1) * dh)
            scores, vals = [], []
            for e in es:
                k_in = np.concatenate([h_nbr[e], ef[e], np.cos(w * dt[e] + b)])
                k = P["w_k.weight"] @ k_in + P["w_k.bias"]
                v = P["w_v.weight"] @ k_in + P["w_v.bias"]
                s = float(q[sl] @ k[sl])
                scores.append(s if s > 0 else 0.2 * s)
                vals.append(v[sl])
            if es:
                m = max(scores)
                ex = [math.exp(s - m) for s in scores]
                tot = sum(ex)
                agg[sl] = sum(x / tot * v for x, v in zip(ex, vals))
        z = P["w_out.weight"] @ np.concatenate([agg, h_dst[r]]) + P["w_out.bias"]
        z = np.maximum(z, 0)
        mu, var = z.mean(), z.var()
        out[r] = (z - mu) / np.sqrt(var + 1e-5) * P["layer_norm.weight"] + P["layer_norm.bias"]
    return out


def _random_block(seed, R=6, E=17, D=8, F=5):
    rng = np.random.default_rng(seed)
    edge_dst = np.sort(rng.integers(0, R - 1, E))        # root R-1 has no edges
    return (rng.standard_normal((R, D)), rng.standard_normal((E, D)), rng.standard_normal((E, F)),
            rng.uniform(0, 1e4, E).astype(np.float32), edge_dst)


def test_conv_matches_brute_force():
    torch.manual_seed(1)
    conv = co.TemporalConvO(8, 5, 6, 2, 8).double()
    with torch.no_grad():
        conv.time_enc.w.bias.uniform_(-1, 1)
        conv.layer_norm.weight.uniform_(0.5, 1.5)
        conv.layer_norm.bias.uniform_(-0.5, 0.5)
    h_dst, h_nbr, ef, dt, ed = _random_block(3)
    t = torch.from_numpy
    got = conv(t(h_dst), t(h_nbr), t(ef), t(dt).double(), t(ed)).detach().numpy()
    want = _brute_conv(conv, h_dst, h_nbr, ef, dt.astype(np.float64), ed)
    np.testing.assert_allclose(got, want, rtol=1e-9, atol=1e-9)


def test_conv_invariants():
    torch.manual_seed(2)
    conv = co.TemporalConvO(8, 5, 6, 2, 8).double()
    h_dst, h_nbr, ef, dt, ed = _random_block(4)
    t = torch.from_numpy
    base = conv(t(h_dst), t(h_nbr), t(ef), t(dt).double(), t(ed))
    # permuting the edges (and their owners) leaves every root's output unchanged
    perm = np.random.default_rng(0).permutation(len(ed))
    pb = conv(t(h_dst), t(h_nbr[perm]), t(ef[perm]), t(dt[perm]).double(), t(ed[perm]))
    torch.testing.assert_close(pb, base)
    # a block without edges gives zeros (models.py:88-89)
    z = conv(t(h_dst), t(h_nbr[:0]), t(ef[:0]), t(dt[:0]).double(), t(ed[:0]))
    assert torch.count_nonzero(z) == 0
    # a root whose neighbours are all identical attends with weight 1 to that V
    one = np.zeros(3, dtype=np.int64)
    hn = np.repeat(h_nbr[:1], 3, 0)
    efr = np.repeat(ef[:1], 3, 0)
    dtr = np.repeat(dt[:1], 3, 0)
    a = conv(t(h_dst[:1]), t(hn), t(efr), t(dtr).double(), t(one))
    b = conv(t(h_dst[:1]), t(hn[:1]), t(efr[:1]), t(dtr[:1]).double(), t(one[:1]))
    torch.testing.assert_close(a, b)


@pytest.mark.parametrize("K", [1, 2, 4])
def test_mailbox_write_matches_serial_rules(K):
    rng = np.random.default_rng(K)
    N, D, F, B = 15, 3, 2, 40
    m1 = co.MemoryO(N, D, K, F)
    m1.memory = torch.randn(N, D)
    m1.next_mail_pos = torch.from_numpy(rng.integers(0, K, N))
    m2 = m1.clone()
    for _ in range(3):
        src = torch.from_numpy(rng.integers(0, N, B))
        dst = torch.from_numpy(rng.integers(0, N, B))
        ts = torch.from_numpy(np.sort(rng.integers(0, 5, B)).astype(np.float32))   # ties
        ef = torch.randn(B, F)
        sp, dp = m1.memory[src].clone(), m1.memory[dst].clone()
        m1.write_mailbox(src, dst, sp, dp, ef, ts)
        co.write_slots_serial(m2, src, torch.cat([sp, dp, ef], 1), ts)
        co.write_slots_serial(m2, dst, torch.cat([dp, sp, ef], 1), ts)
        assert torch.equal(m1.mailbox, m2.mailbox)
        assert torch.equal(m1.mailbox_ts, m2.mailbox_ts)
        assert torch.equal(m1.next_mail_pos, m2.next_mail_pos)


def test_mailbox_dst_role_wins_with_one_slot():
    m = co.MemoryO(4, 2, 1, 1)
    m.memory = torch.arange(8, dtype=torch.float32).view(4, 2)
    src, dst = torch.tensor([1, 2]), torch.tensor([2, 3])
    m.write_mailbox(src, dst, m.memory[src], m.memory[dst], torch.tensor([[9.0], [7.0]]), torch.tensor([1.0, 2.0]))
    # node 2 is src of event 1 and dst of event 0: the dst pass (event 0) wins
    assert m.mailbox[2, 0].tolist() == [4.0, 5.0, 2.0, 3.0, 9.0]
    assert m.mailbox_ts[2, 0].item() == 1.0


def test_negative_sample_collision_bump():
    pool = torch.tensor([3, 5, 8])
    g = torch.Generator().manual_seed(0)
    dst = torch.tensor([5] * 50)
    neg = co.negative_sample(pool, dst, g)
    assert not bool((neg == dst).any())
    g2 = torch.Generator().manual_seed(0)
    idx = torch.randint(0, 3, (50,), generator=g2)
    want = pool[torch.where(pool[idx] == 5, (idx + 1) % 3, idx)]
    assert torch.equal(neg, want)


def test_prepare_roots_floor_time():
    src, dst = torch.tensor([4, 2, 4]), torch.tensor([7, 2, 1])
    roots, tq = co.prepare_roots(src, dst, torch.tensor([1.0, 5.75, 3.0]))
    assert roots.tolist() == [1, 2, 4, 7] and tq.tolist() == [5] * 4


def test_empty_train_step_closed_form():
    """The oracle's empty-batch step (runtime.py:248-253): the model's first
    parameter moves by Adam's closed form with a zero gradient (moments
    decay by beta1 and beta2, bias corrections at the advanced step count);
    the updater's first parameter gets a step count and stays put; every
    other parameter has neither gradient nor state."""
    model, updater = co.build_models(8, 4, 6, 2, 2, seed=3)
    params = list(model.parameters()) + list(updater.parameters())
    lr, b1, b2, eps = 2e-3, 0.9, 0.999, 1e-8
    opt = torch.optim.Adam(params, lr=lr, betas=(b1, b2), eps=eps)
    first, ufirst = next(model.parameters()), next(updater.parameters())
    gen = torch.Generator().manual_seed(5)
    m0 = torch.randn(first.shape, generator=gen) * 1e-3
    v0 = torch.rand(first.shape, generator=gen) * 1e-5 + 1e-7
    t0 = 5
    opt.state[first] = {"step": torch.tensor(float(t0)), "exp_avg": m0.clone(), "exp_avg_sq": v0.clone()}
    before = [p.detach().clone() for p in params]
    co.empty_train_step(model, updater, opt)
    t = t0 + 1
    m, v = b1 * m0.double(), b2 * v0.double()
    want = (before[0].double() - lr / (1 - b1 ** t) * m / (v.sqrt() / math.sqrt(1 - b2 ** t) + eps)).float()
    torch.testing.assert_close(first.detach(), want, rtol=1e-6, atol=1e-9)
    assert not torch.equal(first.detach(), before[0])
    st = opt.state[first]
    assert float(st["step"]) == t
    torch.testing.assert_close(st["exp_avg"], m.float(), rtol=1e-6, atol=0)
    torch.testing.assert_close(st["exp_avg_sq"], v.float(), rtol=1e-6, atol=0)
    assert float(opt.state[ufirst]["step"]) == 1
    assert torch.equal(opt.state[ufirst]["exp_avg"], torch.zeros_like(ufirst))
    for p, b in zip(params[1:], before[1:]):
        assert torch.equal(p.detach(), b)
        if p is not ufirst:
            assert p.grad is None and p not in opt.state
