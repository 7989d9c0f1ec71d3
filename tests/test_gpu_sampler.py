"""GPU parity of the HIP temporal CSR + recent-k sampler (bit-exact).

Checked against (a) the golden fixtures written by the reference's own C++
sampler, through the drop-in API (starry_unigraph.native), and (b) the C oracle
on seeded graphs at sizes the oracle finishes in seconds; the config-3 sized
run is checked through size-independent properties plus an oracle subset.
"""
import glob
import os

import numpy as np
import pytest
import torch

import sampler_oracle as so

pytestmark = pytest.mark.gpu

FIELDS = ("src_index", "sample_nodes", "sample_nodes_ts", "eid", "delta_ts", "sample_weight")
GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "sampler_*.npz")))


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_dropin_api_matches_reference_golden(gpu, path):
    from starry_unigraph.native import BTSNativeSampler, build_temporal_neighbor_block
    z = np.load(path)
    t = lambda a: torch.as_tensor(a)
    name = "golden_gpu_" + os.path.basename(path)
    tnb = build_temporal_neighbor_block(name, t(z["row"]), t(z["col"]), int(z["num_nodes"]), t(z["eid"]),
                                        timestamp=t(z["ts"]))
    np.testing.assert_array_equal(tnb.deg.cpu().numpy(), z["deg"])
    fan = [int(f) for f in z["fanouts"]]
    s = BTSNativeSampler(tnb=tnb, num_nodes=int(z["num_nodes"]), num_edges=len(z["row"]), num_layers=len(fan),
                         fanout=fan, policy="recent")
    blocks = s.sample_from_nodes(t(z["nodes"]), t(z["q_ts"]))
    assert len(blocks) == len(fan)
    for h, b in enumerate(blocks):
        got = {f: getattr(b, f)().cpu().numpy() for f in FIELDS}
        for f in FIELDS:
            np.testing.assert_array_equal(got[f], z[f"{f}_{h}"], err_msg=f"hop {h} {f}")
        np.testing.assert_array_equal(b.dt_f32().cpu().numpy(), z[f"delta_ts_{h}"].astype(np.float32))


def _random_stream(seed, n, e, tmax=10 ** 6, zipf=1.3):
    rng = np.random.default_rng(seed)
    col = np.minimum(rng.zipf(zipf, e) - 1, n - 1)
    row = rng.integers(0, n, e)
    ts = np.sort(rng.integers(0, tmax, e))
    return rng, row, col, ts


@pytest.mark.parametrize("seed,n,e,nq,k", [(0, 1000, 20000, 5000, 10), (1, 50000, 400000, 100000, 20),
                                            (2, 7, 3000, 999, 64), (3, 100000, 1000, 4000, 1),
                                            (4, 2000, 200000, 70000, 0)])
def test_recent_matches_oracle(gpu, seed, n, e, nq, k):
    from starry_unigraph.native.tcsr import RecentSampler, build_tcsr
    rng, row, col, ts = _random_stream(seed, n, e)
    eid = rng.permutation(e)
    g = build_tcsr(n, torch.as_tensor(row), torch.as_tensor(col), torch.as_tensor(eid), torch.as_tensor(ts))
    og = so.build_tcsr(n, row, col, eid, ts)
    np.testing.assert_array_equal(g.indptr.cpu().numpy(), og.indptr)
    np.testing.assert_array_equal(g.nbr.cpu().numpy(), og.nbr)
    np.testing.assert_array_equal(g.eid.cpu().numpy(), og.eid)
    np.testing.assert_array_equal(g.ts.cpu().numpy(), og.ts)
    nodes = rng.integers(0, n, nq)
    qt = rng.integers(-5, 10 ** 6 + 5, nq)
    s = RecentSampler(g)
    padded = s.sample(torch.as_tensor(nodes).cuda(), torch.as_tensor(qt).cuda(), k, want_ts=True)
    hop = s.compact(padded)
    want = so.sample_layer(og, nodes, qt, k)
    m = int(want["ptr"][-1])
    np.testing.assert_array_equal(padded.cnt.cpu().numpy(), np.diff(want["ptr"]))
    np.testing.assert_array_equal(hop.ptr.cpu().numpy(), want["ptr"])
    np.testing.assert_array_equal(hop.nbr[:m].cpu().numpy(), want["sample_nodes"])
    np.testing.assert_array_equal(hop.eid[:m].cpu().numpy(), want["eid"])
    np.testing.assert_array_equal(hop.ts[:m].cpu().numpy(), want["sample_nodes_ts"])
    np.testing.assert_array_equal(hop.dt[:m].cpu().numpy(), want["delta_ts"].astype(np.float32))


def test_dt_rounding_large_values(gpu):
    """int64 -> float32 rounding of t - ts for differences above 2^24 and 2^53."""
    from starry_unigraph.native.tcsr import RecentSampler, build_tcsr
    rng = np.random.default_rng(5)
    e = 4096
    ts = np.sort(rng.integers(-(2 ** 62), 2 ** 40, e))
    col = rng.integers(0, 3, e)
    row = rng.integers(0, 3, e)
    g = build_tcsr(3, torch.as_tensor(row), torch.as_tensor(col), None, torch.as_tensor(ts))
    q = rng.integers(0, 3, 500)
    qt = np.full(500, 2 ** 62, dtype=np.int64)
    s = RecentSampler(g)
    hop = s.compact(s.sample(torch.as_tensor(q).cuda(), torch.as_tensor(qt).cuda(), 30, want_ts=True))
    og = so.build_tcsr(3, row, col, np.arange(e), ts)
    want = so.sample_layer(og, q, qt, 30)
    m = int(want["ptr"][-1])
    np.testing.assert_array_equal(hop.dt[:m].cpu().numpy(), want["delta_ts"].astype(np.float32))


def test_multi_hop_matches_oracle(gpu):
    from starry_unigraph.native.tcsr import RecentSampler, build_tcsr
    rng, row, col, ts = _random_stream(9, 3000, 60000)
    g = build_tcsr(3000, torch.as_tensor(row), torch.as_tensor(col), None, torch.as_tensor(ts))
    og = so.build_tcsr(3000, row, col, np.arange(60000), ts)
    nodes = rng.integers(0, 3000, 2000)
    qt = rng.integers(0, 10 ** 6, 2000)
    s = RecentSampler(g)
    nd, td = torch.as_tensor(nodes).cuda(), torch.as_tensor(qt).cuda()
    hops = s.sample_hops(nd, td, [10, 5, 3], want_last_ts=True)
    want = so.sample_recent(og, nodes, qt, [10, 5, 3])
    for h, w in zip(hops, want):
        m = int(w["ptr"][-1])
        assert h.count() == m
        np.testing.assert_array_equal(h.ptr.cpu().numpy(), w["ptr"])
        np.testing.assert_array_equal(h.nbr.cpu().numpy(), w["sample_nodes"])
        np.testing.assert_array_equal(h.eid.cpu().numpy(), w["eid"])
        np.testing.assert_array_equal(h.ts.cpu().numpy(), w["sample_nodes_ts"])
        np.testing.assert_array_equal(h.dt.cpu().numpy(), w["delta_ts"].astype(np.float32))
    # the padded, sync-free multi-hop path holds the same entries in the same order
    for ph, w in zip(s.sample_padded_hops(nd, td, [10, 5, 3], want_last_ts=True), want):
        c = s.compact(ph)
        np.testing.assert_array_equal(c.nbr.cpu().numpy(), w["sample_nodes"])
        np.testing.assert_array_equal(c.eid.cpu().numpy(), w["eid"])
        np.testing.assert_array_equal(c.ts.cpu().numpy(), w["sample_nodes_ts"])
        np.testing.assert_array_equal(c.dt.cpu().numpy(), w["delta_ts"].astype(np.float32))


def test_out_of_range_ids_raise(gpu):
    from starry_unigraph.native.tcsr import RecentSampler, build_tcsr
    with pytest.raises(RuntimeError, match="out of range"):
        build_tcsr(4, torch.tensor([0, 9]), torch.tensor([1, 1]), None, torch.tensor([1, 2]))
    with pytest.raises(RuntimeError, match="out of range"):
        build_tcsr(4, torch.tensor([0, 1]), torch.tensor([1, 4]), None, torch.tensor([1, 2]))
    g = build_tcsr(4, torch.tensor([0, 1]), torch.tensor([1, 1]), None, torch.tensor([1, 2]))
    s = RecentSampler(g)
    s.err.reset()
    hop = s.sample(torch.tensor([1, 7, -1, 1]).cuda(), torch.tensor([5, 5, 5, 5]).cuda(), 3)
    with pytest.raises(RuntimeError, match="node id out of range"):
        s.err.raise_if_set("sample")
    assert hop.cnt.cpu().tolist() == [2, 0, 0, 2]   # invalid queries yield empty windows


def test_policy_errors(gpu):
    from starry_unigraph.native import BTSNativeSampler, build_temporal_neighbor_block
    tnb = build_temporal_neighbor_block("policy_err", torch.tensor([0, 1]), torch.tensor([1, 1]), 3,
                                        torch.tensor([0, 1]), timestamp=torch.tensor([1, 2]))
    s = BTSNativeSampler(tnb=tnb, num_nodes=3, num_edges=2, num_layers=1, fanout=[2], policy="bogus")
    with pytest.raises(RuntimeError, match="is not exit"):
        s.sample_from_nodes(torch.tensor([1]), torch.tensor([5]))


def test_config3_scale_properties(gpu):
    """Config-3 sized graph (1e7 nodes, 1e8 edges), 4e6 degree-weighted queries:
    size-independent checks on all outputs plus bit-exact oracle checks on a subset."""
    from starry_unigraph import synth
    from starry_unigraph.native.tcsr import RecentSampler, build_tcsr
    g_np = synth.powerlaw_sampler_graph(seed=0)
    nodes, qt = synth.degree_weighted_queries(g_np, seed=1)
    g = build_tcsr(g_np.num_nodes, torch.from_numpy(g_np.row), torch.from_numpy(g_np.col), None,
                   torch.from_numpy(g_np.ts))
    deg = g.deg
    assert int(g.indptr[-1]) == g_np.num_edges
    assert torch.equal(deg.cpu(), torch.from_numpy(np.bincount(g_np.col, minlength=g_np.num_nodes)))
    # the CSR is a stable counting sort of the stream: entry j of node n is an
    # event with col == n, and the event ids (= positions) increase along a list
    e_all = g.eid.long()
    node_of = torch.repeat_interleave(torch.arange(g_np.num_nodes, device="cuda"), deg, output_size=g_np.num_edges)
    assert torch.equal(torch.from_numpy(g_np.col).cuda()[e_all], node_of)
    assert torch.equal(torch.from_numpy(g_np.row).cuda()[e_all], g.nbr.long())
    assert torch.equal(torch.from_numpy(g_np.ts).cuda()[e_all], g.ts)
    same_node = node_of[1:] == node_of[:-1]
    assert bool((e_all[1:][same_node] > e_all[:-1][same_node]).all())
    del e_all, node_of, same_node
    s = RecentSampler(g)
    nd, td = torch.from_numpy(nodes).cuda(), torch.from_numpy(qt).cuda()
    for k in (10, 20):
        hop = s.compact(s.sample(nd, td, k, want_ts=True))
        m = hop.count()
        cnt = hop.ptr[1:] - hop.ptr[:-1]
        assert int(cnt.min()) >= 0 and int(cnt.max()) <= k
        qi = torch.repeat_interleave(torch.arange(len(nodes), device="cuda"), cnt, output_size=m)
        ets = hop.ts[:m]
        assert bool((ets < td[qi]).all())                           # strictly earlier
        same = qi[1:] == qi[:-1]
        assert bool((ets[1:][same] >= ets[:-1][same]).all())        # oldest -> newest
        assert torch.equal((td[qi] - ets).float(), hop.dt[:m])
        # exact check of a random subset of queries against the oracle run on
        # the same CSR lists
        sub = np.sort(np.random.default_rng(k).choice(len(nodes), 2000, replace=False))
        want = _subset_oracle(g, nodes[sub], qt[sub], k)
        ptr = hop.ptr.cpu().numpy()
        np.testing.assert_array_equal(np.diff(ptr)[sub], np.diff(want["ptr"]))
        sel = np.concatenate([np.arange(ptr[i], ptr[i + 1]) for i in sub])
        sel_t = torch.from_numpy(sel).cuda()
        np.testing.assert_array_equal(hop.nbr[sel_t].cpu().numpy(), want["sample_nodes"])
        np.testing.assert_array_equal(hop.eid[sel_t].cpu().numpy(), want["eid"])
        np.testing.assert_array_equal(hop.dt[sel_t].cpu().numpy(), want["delta_ts"].astype(np.float32))
        del hop, qi, ets, same
    # 2 hops (sampler.h:393-399): hop-2 queries are every hop-1 entry (its
    # node at its timestamp), in the padded layout (k = 20: 80M queries,
    # 1.6e9 slots)
    for k in (10, 20):
        h1, h2 = s.sample_padded_hops(nd, td, [k, k])
        q2 = h2.num_queries
        assert q2 == len(nodes) * k
        live1 = (torch.arange(k, device="cuda")[None, :] < h1.cnt[:, None]).reshape(-1)
        assert torch.equal(h2.cnt[~live1], torch.zeros_like(h2.cnt[~live1]))   # padding slots: no query
        assert int(h2.cnt.max()) <= k and int(h2.cnt.min()) >= 0
        assert int(h2.cnt.sum()) > 0
        step = 8_000_000
        for a in range(0, q2, step):   # every live hop-2 entry is strictly before its query time
            b = min(q2, a + step)
            live2 = torch.arange(k, device="cuda")[None, :] < h2.cnt[a:b, None]
            dt = h2.dt[a * k:b * k].view(b - a, k)
            assert bool((dt[live2] >= 1.0).all()), a
        # exact check of random live hop-2 queries against the oracle
        live_idx = torch.nonzero(live1).flatten()
        draw = torch.randint(0, live_idx.numel(), (2000,), generator=torch.Generator().manual_seed(k))
        pick = live_idx[torch.unique(draw).to(live_idx.device)]
        qn, qtt = h1.nbr[pick].long().cpu().numpy(), h1.ts[pick].cpu().numpy()
        want = _subset_oracle(g, qn, qtt, k)
        cnt = h2.cnt[pick].cpu().numpy()
        np.testing.assert_array_equal(cnt, np.diff(want["ptr"]))
        rows = pick.cpu().numpy()[:, None] * k + np.arange(k)[None, :]
        live = np.arange(k)[None, :] < cnt[:, None]
        sel = torch.from_numpy(rows[live]).cuda()
        np.testing.assert_array_equal(h2.nbr[sel].cpu().numpy(), want["sample_nodes"])
        np.testing.assert_array_equal(h2.eid[sel].cpu().numpy(), want["eid"])
        np.testing.assert_array_equal(h2.dt[sel].cpu().numpy(), want["delta_ts"].astype(np.float32))
        del h1, h2, live1, live_idx


def _subset_oracle(g, nodes, qt, k):
    """The oracle's search/fill over the queried nodes' own CSR lists (exact, small)."""
    ip = g.indptr.cpu().numpy()
    uniq = np.unique(nodes)
    starts, ends = ip[uniq], ip[uniq + 1]
    idx = torch.from_numpy(np.concatenate([np.arange(a, b) for a, b in zip(starts, ends)])).cuda()
    sub = so.OracleTCSR(num_nodes=len(uniq),
                        indptr=np.concatenate([[0], np.cumsum(ends - starts)]).astype(np.int64),
                        nbr=g.nbr[idx].long().cpu().numpy(), eid=g.eid[idx].long().cpu().numpy(),
                        ts=g.ts[idx].cpu().numpy())
    return so.sample_layer(sub, np.searchsorted(uniq, nodes), qt, k)


@pytest.mark.parametrize("nq", [2000, 100_000])
def test_int32_timestamps_match_int64(gpu, nq):
    """The packed sampler (sgl_recent_sample_packed: int32 timestamps and
    interleaved ids, chosen when every timestamp fits in int32) gives
    bit-identical windows to the int64 one, in
    both kernel modes (one wave per query up to 32768 queries, one lane per
    query above), with negative times and query times beyond int32's range;
    a graph whose timestamps do not fit keeps the int64 path."""
    from starry_unigraph.native.tcsr import RecentSampler, build_tcsr
    rng = np.random.default_rng(nq)
    N, E = 3000, 80_000
    row, col = rng.integers(0, N, E), rng.integers(0, N, E)
    ts = np.sort(rng.integers(-2 ** 31, 2 ** 31, E))
    g = build_tcsr(N, torch.as_tensor(row), torch.as_tensor(col), None, torch.as_tensor(ts))
    narrow, wide = RecentSampler(g), RecentSampler(g, narrow_ts=False)
    assert narrow.ts32 is not None and wide.ts32 is None
    nodes = torch.as_tensor(rng.integers(0, N, nq)).cuda()
    qt = torch.as_tensor(rng.integers(-2 ** 32, 2 ** 32, nq)).cuda()
    a = narrow.sample(nodes, qt, 10, want_ts=True)
    b = wide.sample(nodes, qt, 10, want_ts=True)
    assert torch.equal(a.cnt, b.cnt)
    assert int(a.cnt.sum().item()) > 0
    live = (torch.arange(10, device=a.cnt.device)[None, :] < a.cnt.long()[:, None]).reshape(-1)
    for f in ("nbr", "eid", "dt", "ts"):
        assert torch.equal(getattr(a, f)[live], getattr(b, f)[live]), f
    assert narrow.fence is not None   # sorted lists: the fence search runs in the one-lane-per-query mode
    g2 = build_tcsr(4, torch.tensor([0, 1]), torch.tensor([1, 1]), None, torch.tensor([1, 2 ** 31]))
    assert RecentSampler(g2).ts32 is None


def test_unsorted_lists_skip_the_fences(gpu):
    """Lists whose times are not sorted (event order is not time order) keep
    std::lower_bound's probe sequence: no fences, and the packed sampler
    equals the int64 one and the oracle."""
    from starry_unigraph.native.tcsr import RecentSampler, build_tcsr
    rng = np.random.default_rng(5)
    N, E, nq = 500, 60_000, 50_000
    row, col = rng.integers(0, N, E), rng.integers(0, N, E)
    ts = rng.integers(0, 10 ** 6, E)          # unsorted
    g = build_tcsr(N, torch.as_tensor(row), torch.as_tensor(col), None, torch.as_tensor(ts))
    narrow, wide = RecentSampler(g), RecentSampler(g, narrow_ts=False)
    assert narrow.ts32 is not None and narrow.fence is None
    nodes, qt = rng.integers(0, N, nq), rng.integers(0, 10 ** 6, nq)
    a = narrow.sample(torch.as_tensor(nodes).cuda(), torch.as_tensor(qt).cuda(), 7)
    b = wide.sample(torch.as_tensor(nodes).cuda(), torch.as_tensor(qt).cuda(), 7)
    assert torch.equal(a.cnt, b.cnt)
    live = (torch.arange(7, device=a.cnt.device)[None, :] < a.cnt.long()[:, None]).reshape(-1)
    for f in ("nbr", "eid", "dt"):
        assert torch.equal(getattr(a, f)[live], getattr(b, f)[live]), f
    og = so.build_tcsr(N, row, col, np.arange(E), ts)
    want = so.sample_recent(og, nodes[:2000], qt[:2000], [7])[0]
    got = narrow.compact(narrow.sample(torch.as_tensor(nodes[:2000]).cuda(), torch.as_tensor(qt[:2000]).cuda(), 7))
    np.testing.assert_array_equal(got.nbr.cpu().numpy(), want["sample_nodes"])
    np.testing.assert_array_equal(got.eid.cpu().numpy(), want["eid"])


def test_fence_search_matches_int64_and_oracle(gpu):
    """The fence search of the one-lane-per-query mode (> 32768 queries on a
    time-sorted packed CSR): lists of 65-5000 entries at unaligned offsets,
    runs of tied timestamps across fence lines, and
    query times equal to fence values, equal to list entries, below a list's
    first entry and above its last. Windows equal the int64 sampler's and
    the oracle's."""
    from starry_unigraph.native.tcsr import RecentSampler, build_tcsr
    rng = np.random.default_rng(17)
    N = 400
    deg = rng.integers(65, 5001, N)
    deg[deg % 32 == 0] += 1                          # list boundaries drift off the 32-entry lines
    col = np.repeat(np.arange(N), deg)
    E = col.size
    # few distinct times: long tied runs within and across 32-entry lines
    ts_per = [np.sort(rng.integers(0, max(2, d // 40), d)) * 1000 for d in deg]
    ts = np.concatenate(ts_per)
    row = rng.integers(0, N, E)
    # event order = the lists' order (a stable sort by dst keeps it), so every list is time-sorted
    g = build_tcsr(N, torch.as_tensor(row), torch.as_tensor(col), None, torch.as_tensor(ts))
    narrow, wide = RecentSampler(g), RecentSampler(g, narrow_ts=False)
    assert narrow.ts32 is not None and narrow.fence is not None
    nq = 60_000
    nodes = rng.integers(0, N, nq)
    ip = g.indptr.cpu().numpy()
    gts = g.ts.cpu().numpy()
    kind = rng.integers(0, 5, nq)
    qt = np.empty(nq, dtype=np.int64)
    for i, (n, k) in enumerate(zip(nodes, kind)):
        a, b = ip[n], ip[n + 1]
        if k == 0:      # a fence value inside the list (every 32nd global entry)
            f = np.arange((a + 31) // 32 * 32, b, 32)
            qt[i] = gts[f[rng.integers(0, f.size)]] if f.size else gts[a]
        elif k == 1:    # an entry of the list
            qt[i] = gts[rng.integers(a, b)]
        elif k == 2:    # below the first entry
            qt[i] = gts[a] - rng.integers(0, 2)
        elif k == 3:    # above the last entry
            qt[i] = gts[b - 1] + rng.integers(0, 2)
        else:
            qt[i] = rng.integers(-5, int(gts[b - 1]) + 5)
    for fan in (10, 25):
        tn, tq = torch.as_tensor(nodes).cuda(), torch.as_tensor(qt).cuda()
        a = narrow.sample(tn, tq, fan, want_ts=True)
        b = wide.sample(tn, tq, fan, want_ts=True)
        assert torch.equal(a.cnt, b.cnt), fan
        live = (torch.arange(fan, device=a.cnt.device)[None, :] < a.cnt.long()[:, None]).reshape(-1)
        for f in ("nbr", "eid", "dt", "ts"):
            assert torch.equal(getattr(a, f)[live], getattr(b, f)[live]), (f, fan)
        og = so.build_tcsr(N, row, col, np.arange(E), ts)
        want = so.sample_recent(og, nodes, qt, [fan])[0]
        got = narrow.compact(a)
        np.testing.assert_array_equal(got.ptr.cpu().numpy(), want["ptr"])
        np.testing.assert_array_equal(got.nbr.cpu().numpy(), want["sample_nodes"])
        np.testing.assert_array_equal(got.eid.cpu().numpy(), want["eid"])
        np.testing.assert_array_equal(got.dt.cpu().numpy(), want["delta_ts"].astype(np.float32))
