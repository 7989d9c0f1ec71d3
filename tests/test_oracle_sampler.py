"""Pins the C sampler oracle (oracle/sampler_oracle.c) before anything is
checked against it:

* golden fixtures written by the reference's own C++ sampler compiled from
  its sources (tests/golden/make_sampler_golden.py);
* a brute-force statement of the recent policy on many random tiny graphs;
* closed-form properties (window size, strict ``ts < t``, ordering).
"""
import glob
import os

import numpy as np
import pytest

import sampler_oracle as so

FIELDS = ("src_index", "sample_nodes", "sample_nodes_ts", "eid", "delta_ts", "sample_weight")


def _golden_cases(golden_dir):
    return sorted(glob.glob(os.path.join(golden_dir, "sampler_*.npz")))


def test_golden_fixtures_exist(golden_dir):
    assert len(_golden_cases(golden_dir)) >= 8


@pytest.mark.parametrize("case", [os.path.basename(p) for p in
                                  sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "sampler_*.npz")))])
def test_oracle_matches_reference_golden(golden_dir, case):
    z = np.load(os.path.join(golden_dir, case))
    g = so.build_tcsr(int(z["num_nodes"]), z["row"], z["col"], z["eid"], z["ts"])
    np.testing.assert_array_equal(g.deg, z["deg"])
    blocks = so.sample_recent(g, z["nodes"], z["q_ts"], list(z["fanouts"]))
    for h, b in enumerate(blocks):
        for f in FIELDS:
            np.testing.assert_array_equal(b[f], z[f"{f}_{h}"], err_msg=f"{case} hop {h} {f}")
            assert b[f].dtype == z[f"{f}_{h}"].dtype


@pytest.mark.parametrize("seed", range(40))
def test_oracle_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 12))
    e = int(rng.integers(0, 60))
    row = rng.integers(0, n, e)
    col = rng.integers(0, n, e)
    ts = np.sort(rng.integers(0, 30, e))          # time-sorted stream, with ties
    eid = rng.permutation(e) + 1000
    nodes = rng.integers(0, n, 25)
    q_ts = rng.integers(-2, 35, 25)
    k = int(rng.integers(0, 8))
    g = so.build_tcsr(n, row, col, eid, ts)
    got = so.sample_layer(g, nodes, q_ts, k)
    want = so.brute_force_layer(n, row, col, eid, ts, nodes, q_ts, k)
    for f in FIELDS:
        np.testing.assert_array_equal(got[f], want[f], err_msg=f)


def test_oracle_properties_large():
    rng = np.random.default_rng(11)
    n, e, k = 2000, 50000, 10
    row = rng.integers(0, n, e)
    col = np.minimum(rng.zipf(1.5, e) - 1, n - 1)
    ts = np.sort(rng.integers(0, 10 ** 6, e))
    g = so.build_tcsr(n, row, col, np.arange(e), ts)
    assert g.indptr[-1] == e and np.all(np.diff(g.indptr) >= 0)
    nodes = rng.integers(0, n, 5000)
    q_ts = rng.integers(0, 10 ** 6, 5000)
    b = so.sample_layer(g, nodes, q_ts, k)
    cnt = np.diff(b["ptr"])
    assert cnt.max() <= k
    assert np.all(b["delta_ts"] > 0)                       # strictly earlier events only
    assert np.all(b["delta_ts"] == q_ts[b["src_index"]] - b["sample_nodes_ts"])
    assert np.all(col[b["eid"]] == nodes[b["src_index"]])  # in-neighbours of the root
    assert np.all(row[b["eid"]] == b["sample_nodes"])
    # a full window means exactly k events before t; a short one means all of them
    before = np.array([np.searchsorted(ts[col == v], t) for v, t in zip(nodes[:300], q_ts[:300])])
    np.testing.assert_array_equal(cnt[:300], np.minimum(before, k))


def test_oracle_rejects_bad_nodes():
    with pytest.raises(RuntimeError):
        so.build_tcsr(3, [0, 5], [1, 1], [0, 1], [1, 2])
    g = so.build_tcsr(3, [0, 2], [1, 1], [0, 1], [1, 2])
    with pytest.raises(RuntimeError):
        so.sample_layer(g, [3], [10], 2)
