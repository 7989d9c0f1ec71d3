"""Session-level behaviour on the GPU: the checkpoint round trip of
CTDGSession (backends/ctdg/runtime/session.py:78-93: model + updater state
dicts, strict loading), a load queued between asynchronous steps, and the
step's metric dict computed on the device against scikit-learn."""
import math

import numpy as np
import pytest
import torch

import ctdg_oracle as co

pytestmark = pytest.mark.gpu


def _session(seed, B=200):
    from starry_unigraph import SchedulerSession, synth
    from starry_unigraph.data import from_stream
    s = synth.bipartite_stream(num_src=300, num_dst=60, num_events=6000, edge_dim=16, seed=3)
    cfg = {"model": {"family": "tgn", "hidden_dim": 32}, "data": {"name": "ckpt", "format": "synthetic"},
           "train": {"batch_size": B, "lr": 1e-3}, "runtime": {"device": "cuda"},
           "ctdg": {"mailbox_slots": 2, "dim_time": 16, "num_head": 2, "dropout": 0.0, "att_dropout": 0.0},
           "sampling": {"neighbor_limit": [10], "history": 1, "strategy": "recent"}}
    torch.manual_seed(seed)
    sess = SchedulerSession.from_config(cfg).with_events(from_stream(s))
    sess.build_runtime()
    return sess.ctdg_session


def test_checkpoint_round_trip(gpu, tmp_path):
    """Save after training steps; a session built with other initial weights
    loads it and then has bit-identical model and updater weights, and from
    the same node state and negatives its next eval step is bit-identical."""
    a, b = _session(0), _session(99)
    rta, rtb = a.online_runtime, b.online_runtime
    for batch in list(rta.iter_batches("train", 200))[:4]:
        a.train_step(batch)
    path = tmp_path / "ck.pt"
    a.save_checkpoint(path)
    b.load_checkpoint(path)
    for (n, p), (_, q) in zip(rta.model.state_dict().items(), rtb.model.state_dict().items()):
        assert torch.equal(p, q), n
    for (n, p), (_, q) in zip(rta.memory_updater.state_dict().items(), rtb.memory_updater.state_dict().items()):
        assert torch.equal(p, q), n
    sa, sb = rta.memory.state, rtb.memory.state
    for name in ("memory", "mailbox", "mailbox_ts", "memory_ts", "next_mail_pos"):
        getattr(sb, name).copy_(getattr(sa, name))
    sb.touched()
    batch = list(rta.iter_batches("val", 200))[2]
    neg = co.negative_sample(rta.dataset.dst.unique(), batch.dst, torch.Generator().manual_seed(4)).to(gpu)
    outs = []
    for rt in (rta, rtb):
        rt._neg_queue["val"] = (neg, 0)
        outs.append(rt.eval_step(batch, "val"))
    assert outs[0]["loss"] == outs[1]["loss"]
    assert outs[0]["predictions"] == outs[1]["predictions"]
    assert outs[0]["meta"]["metrics"] == outs[1]["meta"]["metrics"]


def test_checkpoint_loading_is_strict(gpu, tmp_path):
    """Missing keys, unexpected keys and shape mismatches raise, as
    nn.Module.load_state_dict does; the weights stay untouched."""
    a = _session(0)
    rt = a.online_runtime
    path = tmp_path / "ck.pt"
    a.save_checkpoint(path)
    ck = torch.load(path, weights_only=True)
    before = [p.clone() for p in rt.model.parameters()]
    bad = []
    m = dict(ck["model"])
    m.pop("src_fc.bias")
    bad.append(("Missing key", m))
    m = dict(ck["model"], extra=torch.zeros(1))
    bad.append(("Unexpected key", m))
    m = dict(ck["model"])
    m["out_fc.weight"] = torch.zeros(2, 32)
    bad.append(("size mismatch", m))
    for what, m in bad:
        p = tmp_path / "bad.pt"
        torch.save({"model": m, "memory_updater": ck["memory_updater"]}, p)
        with pytest.raises(RuntimeError, match=what):
            a.load_checkpoint(p)
        for x, y in zip(before, rt.model.parameters()):
            assert torch.equal(x, y)


def test_load_between_async_steps_is_ordered(gpu, tmp_path):
    """A checkpoint loaded right after asynchronous (pipelined) steps, with no
    synchronisation, takes effect exactly as if the device had been
    synchronised first: two identical runs end bit-identical."""
    src = _session(5)
    for batch in list(src.online_runtime.iter_batches("train", 200))[:3]:
        src.train_step(batch)
    path = tmp_path / "w.pt"
    src.save_checkpoint(path)
    runs = []
    for sync_first in (False, True):
        s = _session(0)
        rt = s.online_runtime
        rt.collect_results = False
        batches = list(rt.iter_batches("train", 200))
        torch.manual_seed(8)
        for batch in batches[:3]:
            rt.train_step(batch)
        if sync_first:
            torch.cuda.synchronize()
        s.load_checkpoint(path)
        for batch in batches[3:6]:
            rt.train_step(batch)
        torch.cuda.synchronize()
        rt.check_sync()
        runs.append([t.detach().clone() for t in (rt.optimizer.inner.flat, rt.memory.state.memory,
                                                   rt.memory.state.mailbox)])
    for x, y in zip(*runs):
        assert torch.equal(x, y)


def test_device_metrics_match_sklearn(gpu):
    from starry_unigraph.backends.ctdg.runtime.metrics import link_metrics
    rng = np.random.default_rng(3)
    pos = torch.from_numpy(rng.normal(0.2, 1.5, 4000).astype(np.float32))
    neg = torch.from_numpy(rng.normal(-0.2, 1.5, 4000).astype(np.float32))
    pos[:500] = neg[:500]
    got = link_metrics(pos.to(gpu), neg.to(gpu))
    want = co.metric_dict(pos, neg)
    for k, tol in (("ap", 1e-9), ("auc", 1e-9), ("mrr", 1e-6)):
        assert abs(got[k] - want[k]) <= tol, (k, got[k], want[k])


@pytest.mark.parametrize("P,N,ties", [(600, 600, "dup"), (4000, 4000, "dup"), (4000, 4000, "sat"), (3, 5000, "dup"),
                                       (1000, 1, "none"), (1, 1, "none"), (600, 600, "all"), (2048, 2000, "dup"),
                                       (2049, 150, "dup"), (600, 600, "narrow"), (3000, 1000, "tiny"),
                                       (0, 10, "none"), (10, 0, "none")])
def test_link_metrics_kernel_matches_sklearn(gpu, P, N, ties):
    """sgl_link_metrics (per positive, counts of the scores below, equal and
    above it over slices of the staged scores; a fixed-order sum of the
    workgroups' partials) against scikit-learn's metrics
    (runtime.py:202-214): AP and AUC to 1e-9, "mrr" to 1e-6; with tied
    scores (logits on a coarse grid, as the non-root negatives' shared zero
    embedding ties them; saturated logits whose sigmoids are all 1; every
    score equal), distinct scores packed close together (near 1, and below
    2^-24), unbalanced sizes, single elements and an empty side (every
    metric NaN). The loss is copied through, and the ring takes consecutive
    calls in order."""
    from starry_unigraph.lib import _capi
    rng = np.random.default_rng(P + N)
    if ties == "none":
        pos = torch.from_numpy(rng.normal(0.2, 1.5, P).astype(np.float32))
        neg = torch.from_numpy(rng.normal(-0.2, 1.5, N).astype(np.float32))
    else:
        # logits on a 1/64 grid: many exact ties, and distinct logits' sigmoids
        # far apart (a sigmoid that differs from the host's in the last bit
        # cannot tie or untie two of them)
        pos = torch.from_numpy((rng.integers(-180, 220, P) / 64).astype(np.float32))
        neg = torch.from_numpy((rng.integers(-220, 180, N) / 64).astype(np.float32))
    if ties == "narrow":   # sigmoids in (0.99995, 0.999994): one bucket, distinct values
        pos = torch.from_numpy(rng.uniform(10.0, 12.0, P).astype(np.float32))
        neg = torch.from_numpy(rng.uniform(10.0, 12.0, N).astype(np.float32))
    elif ties == "tiny":   # sigmoids below 2^-24: one bucket, distinct values
        pos = torch.from_numpy(rng.uniform(-30.0, -20.0, P).astype(np.float32))
        neg = torch.from_numpy(rng.uniform(-31.0, -21.0, N).astype(np.float32))
    if ties == "sat":   # sigmoid(x) rounds to exactly 1 for x >= 20
        pos[: P // 4] = torch.from_numpy(rng.uniform(20.0, 40.0, P // 4).astype(np.float32))
        neg[: N // 8] = torch.from_numpy(rng.uniform(20.0, 40.0, N // 8).astype(np.float32))
    elif ties == "all":
        pos.fill_(0.25)
        neg.fill_(0.25)
    loss = torch.tensor([1.25], device=gpu)
    out = torch.zeros(4, dtype=torch.float64, device=gpu)
    ring = torch.full((3, 4), -1.0, dtype=torch.float64, device=gpu)
    seq = torch.zeros(1, dtype=torch.int64, device=gpu)
    P_ = _capi.ptr
    pg, ng = pos.to(gpu), neg.to(gpu)
    work = torch.zeros(int(_capi.lib().sgl_link_metrics_work_doubles(P)), dtype=torch.float64, device=gpu)
    done = torch.zeros(1, dtype=torch.int32, device=gpu)
    for _ in range(4):   # ring slots 0, 1, 2, 0
        _capi.check(_capi.lib().sgl_link_metrics(P, N, P_(pg), P_(ng), P_(loss), P_(seq), P_(ring), 3, P_(out),
                                                  P_(work), P_(done), _capi.stream_of(gpu)), "sgl_link_metrics")
    torch.cuda.synchronize()
    if P == 0 or N == 0:
        got = out.cpu().tolist()
        assert got[0] == 1.25 and all(math.isnan(x) for x in got[1:]), got
        assert int(seq.item()) == 4
        return
    # the reference's scores: torch.sigmoid of the float32 logits on the device
    # (runtime.py:203-204; torch's CPU sigmoid can give one logit two values,
    # its vector and scalar paths rounding differently, which unties scores)
    from sklearn.metrics import average_precision_score, roc_auc_score
    sp, sn = torch.sigmoid(pg).cpu(), torch.sigmoid(ng).cpu()
    scores = torch.cat([sp, sn]).numpy()
    labels = np.concatenate([np.ones(P), np.zeros(N)])
    want = {"ap": float(average_precision_score(labels, scores)), "auc": float(roc_auc_score(labels, scores)),
            "mrr": float((sp.unsqueeze(1) > sn.unsqueeze(0)).float().mean().item())}
    got = out.cpu().tolist()
    assert got[0] == 1.25
    for k, i, tol in (("ap", 1, 1e-9), ("auc", 2, 1e-9), ("mrr", 3, 1e-6)):
        assert abs(got[i] - want[k]) <= tol, (k, got[i], want[k])
    assert int(seq.item()) == 4 and int(done.item()) == 0
    assert torch.equal(ring.cpu(), out.cpu().unsqueeze(0).expand(3, 4))


def test_fixed_point_range_is_reported(gpu):
    """A term outside the predictor's fixed-point range (forced from the host:
    out_fc weights of 1e10 make the per-event loss and hidden-layer gradient
    terms exceed 2^23) sets the range flag, check_sync raises and clears it;
    ordinary steps leave it clear."""
    cs = _session(0)
    rt = cs.online_runtime
    batches = list(rt.iter_batches("train", 200))
    cs.train_step(batches[0])
    rt.check_sync()
    with torch.no_grad():
        rt._core().out_fc.weight.fill_(1e10)
    rt.fence()
    cs.train_step(batches[1])
    with pytest.raises(RuntimeError, match="fixed-point range"):
        rt.check_sync()
    rt.check_sync()
