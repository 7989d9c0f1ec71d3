"""The event-stream input pipeline on the CPU: split arithmetic at the
Benchmark stream sizes, batching, the per-split sampler graph, and the
on-disk formats of the reference's loader (data/raw_temporal.py:11-329):
edges.csv + edge_features.pt, the edge-list fallback (<name>.edges /
edges.txt: comments, separators, column layouts, stable time sort, id
remap), node temporal features and their as-of lookup, and the mock ring."""
import numpy as np
import pytest
import torch

from starry_unigraph.backends.ctdg.runtime.data import TGTemporalDataset
from starry_unigraph.data import from_stream, load_raw_temporal_events, write_ctdg_csv
from starry_unigraph.runtime._split import normalize_split_ratio, split_bounds


@pytest.mark.parametrize("total,counts", [(157_474, (110_232, 23_621, 23_621)),
                                          (7_833_140, (5_483_198, 1_174_971, 1_174_971))])
def test_split_counts_at_config_sizes(total, counts):
    """_split.py:17-44 at the cfg1/cfg2 and cfg4/cfg5 stream sizes."""
    got = []
    prev_end = 0
    for split in ("train", "val", "test"):
        a, b = split_bounds(total, split, normalize_split_ratio(None))
        assert a == prev_end          # contiguous, in time order
        prev_end = b
        got.append(b - a)
    assert tuple(got) == counts and prev_end == total


@pytest.mark.parametrize("n,B,steps", [(110_232, 200, 552), (5_483_198, 600, 9139), (5_483_198, 4000, 1371)])
def test_train_steps_per_epoch(n, B, steps):
    assert -(-n // B) == steps


def _small_dataset(tmp_path, n_events=1000, seed=0):
    from starry_unigraph import synth
    s = synth.bipartite_stream(num_src=50, num_dst=20, num_events=n_events, edge_dim=3, seed=seed)
    return s, TGTemporalDataset(tmp_path, "mem", events=from_stream(s))


def test_batches_and_sampler_graph(tmp_path):
    """Batches are consecutive slices of the split (the last one short); the
    sampler graph of a split is every event before the split's end, so it
    holds the events of the batch being trained on (data.py:196-231); its
    times are int64 of the float32 times."""
    s, ds = _small_dataset(tmp_path)
    a, b = split_bounds(ds.num_edges, "train", ds.split_ratio)
    batches = list(ds.iter_batches("train", 64))
    assert [bt.size for bt in batches[:-1]] == [64] * (len(batches) - 1)
    assert sum(bt.size for bt in batches) == b - a
    cat = torch.cat([bt.event_ids for bt in batches])
    assert torch.equal(cat, torch.arange(a, b))
    for bt in batches:
        assert bt.start == int(bt.event_ids[0])
        assert torch.equal(bt.src, torch.from_numpy(s.src)[bt.event_ids])
        assert torch.equal(bt.edge_feat, torch.from_numpy(s.edge_feat)[bt.event_ids])
        assert bt.src_node_feat is None
    g = ds.sampler_graph("train")
    assert torch.equal(g["eid"], torch.arange(0, b))
    mid = batches[len(batches) // 2]
    assert bool(torch.isin(mid.event_ids, g["eid"]).all())
    assert torch.equal(g["ts"], torch.from_numpy(s.ts[:b]).long())
    _, vb = split_bounds(ds.num_edges, "val", ds.split_ratio)
    assert ds.sampler_graph("val")["eid"].numel() == vb


def test_batch_start_needs_consecutive_ids():
    """A batch whose ids are not one consecutive run is gathered by id."""
    from starry_unigraph.backends.ctdg.runtime.data import CTDGDataBatch
    z = torch.zeros(4)
    for ids, want in (([5, 6, 7, 8], 5), ([1, 3, 2, 4], -1), ([1, 2, 4, 5], -1), ([9], 9)):
        t = torch.tensor(ids)
        b = CTDGDataBatch(0, "train", t, t, t, z[:len(ids)], torch.zeros(len(ids), 1))
        assert b.start == want, ids


def test_csv_round_trip(tmp_path):
    from starry_unigraph import synth
    s = synth.unipartite_stream(num_nodes=300, num_events=2000, edge_dim=4, seed=3)
    write_ctdg_csv(tmp_path / "ds", s.src, s.dst, s.ts, s.edge_feat)
    ev = load_raw_temporal_events(tmp_path, "ds", {"data": {}})
    assert torch.equal(ev.src, torch.from_numpy(s.src)) and torch.equal(ev.dst, torch.from_numpy(s.dst))
    assert torch.equal(ev.ts, torch.from_numpy(s.ts))
    assert torch.equal(ev.edge_feat, torch.from_numpy(s.edge_feat))
    assert ev.num_nodes == int(max(s.src.max(), s.dst.max())) + 1
    assert torch.equal(ev.weight, torch.ones(2000))


def test_edge_list_fallback(tmp_path):
    """raw_temporal.py:255-314: comment lines skipped, comma or whitespace
    separated, "u v t" / "u v w t" / "idx u v t ..." rows, events stably
    sorted by time, ids remapped to ranks of the sorted unique ids, ones as
    edge features."""
    d = tmp_path / "g"
    d.mkdir()
    (d / "edges.txt").write_text("% a comment\n# another\n"
                                 "10 20 5.0\n"          # u v t
                                 "30,10,2.5,1.0\n"      # u v w t
                                 "7 30 20 1.0 x y\n"    # idx u v t ...
                                 "\n"
                                 "20 30 0.5 2.5\n"      # u v w t (t = 2.5 ties the second row)
                                 "1 2\n")               # too short: skipped
    ev = load_raw_temporal_events(tmp_path, "g", {"data": {}})
    # rows (u, v, t, w): (10,20,5,1) (30,10,1,2.5) (30,20,1,1) (20,30,2.5,0.5)
    # stable time order: row2 (t=1), row3 (t=1), row4 (t=2.5), row1 (t=5); ids 10,20,30 -> 0,1,2
    assert ev.src.tolist() == [2, 2, 1, 0] and ev.dst.tolist() == [0, 1, 2, 1]
    assert ev.ts.tolist() == [1.0, 1.0, 2.5, 5.0]
    assert ev.weight.tolist() == [2.5, 1.0, 0.5, 1.0]
    assert ev.num_nodes == 3 and ev.num_edges == 4
    assert torch.equal(ev.edge_feat, torch.ones(4, 1))
    # <name>.edges takes precedence over edges.txt
    (d / "g.edges").write_text("5 6 1.0\n")
    ev2 = load_raw_temporal_events(tmp_path, "g", {"data": {}})
    assert ev2.num_edges == 1 and ev2.src.tolist() == [0] and ev2.dst.tolist() == [1]


def test_node_temporal_features(tmp_path):
    """raw_temporal.py:85-163 + data.py:128-157: the table is stably sorted by
    time, raises num_nodes (csv) or joins the id remap (edge list); lookups
    give the latest row with time <= t (the last of equal times), zeros
    before a node's first row."""
    d = tmp_path / "nf"
    write_ctdg_csv(d, [0, 1, 2], [1, 2, 0], [1.0, 2.0, 3.0])
    (d / "node_temporal_features.csv").write_text(
        "node_id,ts,f1,f2,label\n"
        "1,5.0,1.0,10.0,a\n"
        "1,2.0,2.0,20.0,b\n"
        "6,1.0,3.0,30.0,c\n"
        "1,2.0,4.0,40.0,d\n")
    ev = load_raw_temporal_events(tmp_path, "nf", {"data": {}})
    nf = ev.node_temporal_features
    assert nf.feature_names == ("f1", "f2") and nf.dim == 2
    assert nf.ts.tolist() == [1.0, 2.0, 2.0, 5.0] and nf.node_ids.tolist() == [6, 1, 1, 1]
    assert ev.num_nodes == 7          # node 6 only appears in the features
    ds = TGTemporalDataset(tmp_path, "nf", events=ev)
    assert ds.node_feat_dim == 2
    got = ds.lookup_node_features(torch.tensor([1, 1, 1, 1, 6, 0]), torch.tensor([1.9, 2.0, 4.9, 5.0, 0.5, 9.0]))
    assert got.tolist() == [[0, 0], [4, 40], [4, 40], [1, 10], [0, 0], [0, 0]]
    b = next(ds.iter_batches("train", 10))
    assert b.src_node_feat.shape == (b.size, 2) and b.dst_node_feat.shape == (b.size, 2)
    # the edge-list loader remaps the feature ids with the event ids
    d2 = tmp_path / "nf2"
    d2.mkdir()
    (d2 / "edges.txt").write_text("100 200 1.0\n200 300 2.0\n")
    (d2 / "node_features.csv").write_text("node,time,v\n300,0.0,1.5\n999,0.0,2.5\n")
    ev2 = load_raw_temporal_events(tmp_path, "nf2", {"data": {}})
    assert ev2.num_nodes == 4        # 100, 200, 300, 999
    assert ev2.node_temporal_features.node_ids.tolist() == [2, 3]


def test_mock_fallback(tmp_path):
    ev = load_raw_temporal_events(tmp_path, "nothing_here", {"data": {}, "train": {"snaps": 8}})
    assert ev.source.startswith("mock:") and ev.num_edges == 32 and ev.num_nodes == 16
    assert ev.src.tolist()[:3] == [0, 1, 2] and ev.dst.tolist()[:3] == [1, 2, 3]
