"""sgl_recent_compact_noalloc (the compaction whose scratch is a static device
array) against sgl_recent_compact (the workspace entry point): bit-identical
outputs on two calls in a row, the second with fewer queries (the scratch
keeps the first call's tile sums); a call above the limit is refused on the
host."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _padded(seed, nq, k):
    from starry_unigraph.native.tcsr import RecentSampler, build_tcsr
    rng = np.random.default_rng(seed)
    n, e = 5000, 300_000
    row, col = rng.integers(0, n, e), np.minimum(rng.zipf(1.3, e) - 1, n - 1)
    ts = np.sort(rng.integers(0, 10 ** 6, e))
    g = build_tcsr(n, torch.as_tensor(row), torch.as_tensor(col), None, torch.as_tensor(ts))
    s = RecentSampler(g)
    nodes = torch.as_tensor(rng.integers(0, n, nq)).cuda()
    qt = torch.as_tensor(rng.integers(0, 10 ** 6, nq)).cuda()
    return s, s.sample(nodes, qt, k, want_ts=True)


def _noalloc(hop, m):
    from starry_unigraph.lib import _capi
    dev = hop.cnt.device
    nq = hop.num_queries
    ptr = torch.full((nq + 1,), -7, dtype=torch.int64, device=dev)
    mm = max(m, 1)
    nbr = torch.full((mm,), -7, dtype=torch.int32, device=dev)
    eid = torch.full((mm,), -7, dtype=torch.int32, device=dev)
    dt = torch.full((mm,), -7.0, dtype=torch.float32, device=dev)
    ts = torch.full((mm,), -7, dtype=torch.int64, device=dev)
    P = _capi.ptr
    with torch.cuda.device(dev):
        _capi.check(_capi.lib().sgl_recent_compact_noalloc(
            nq, hop.fanout, P(hop.cnt), P(hop.nbr), P(hop.eid), P(hop.dt), P(hop.ts), P(ptr), P(nbr), P(eid),
            P(dt), P(ts), _capi.stream_of(dev)), "sgl_recent_compact_noalloc")
    return ptr, nbr[:m], eid[:m], dt[:m], ts[:m]


def test_noalloc_compact_matches_workspace_compact(gpu):
    for seed, nq, k in ((0, 1_000_000, 20), (1, 70_001, 10)):   # the second call is smaller
        s, hop = _padded(seed, nq, k)
        want = s.compact(hop)                                   # sgl_recent_compact
        m = int(want.ptr[-1].item())
        got = _noalloc(hop, m)
        torch.cuda.synchronize()
        assert m > 0
        assert torch.equal(got[0], want.ptr), seed
        for a, b, name in zip(got[1:], (want.nbr, want.eid, want.dt, want.ts), ("nbr", "eid", "dt", "ts")):
            assert torch.equal(a, b), (seed, name)


def test_noalloc_compact_limit_and_empty(gpu):
    from starry_unigraph.lib import _capi
    L = _capi.lib()
    big = _capi.SGL_COMPACT_NOALLOC_MAX_QUERIES + 1
    rc = L.sgl_recent_compact_noalloc(big, 4, None, None, None, None, None, None, None, None, None, None, None)
    assert rc == 1 and b"static scratch limit" in L.sgl_last_error()
    ptr = torch.full((1,), 5, dtype=torch.int64, device=gpu)
    assert L.sgl_recent_compact_noalloc(0, 4, None, None, None, None, None, _capi.ptr(ptr), None, None, None, None,
                                        _capi.stream_of(gpu)) == 0
    torch.cuda.synchronize()
    assert int(ptr.item()) == 0
