"""Benchmark of the MI355X-native CTDG training step (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints ONE JSON line. Workloads:
  tgn-large  (default) config 4: TGN, 1,140,149 nodes, 7,833,140 events
             (Zipf 1.5), 16-d edge features, D = T = 100, 2 heads, k = 10,
             1 mailbox slot, batch 600. A step is one training batch.
  tgn-small  config 1: bipartite 8,227 + 1,000 nodes, 157,474 events, F = 172, B = 200.
  jodie      config 2: the same stream, memory + GRU + the JODIE time
             projection (ctdg.embedding = time_projection), no attention.
  tgn-stress config 5: the config-4 stream, D = 172, 4 heads, k = 20,
             2 sampled hops and 1 attention layer (the reference's conv reads
             only the first hop's block, runtime.py:164-167), 4 mailbox
             slots, batch 4,000.
  sampler    config 3 alone (temporal sampler microbench).
  gather-scatter  the memory / mailbox gather-scatter microbench: config-5 state
             (1,140,149 nodes, D = 172, K = 4, F = 16) under batches of 600, 4,000
             and 1,048,576 events of the config-4 stream: batch preparation,
             sampling (k = 20), GRU + mailbox, memory commit, edge-row gather.
The default run also measures config 3 and reports it under "sampler", the
gather/scatter microbench under "gather_scatter", and short runs of configs 1,
2, 5 and of config 4 with dropout 0.1 under "configs".

Timed region: W untimed warm-up steps, then K steps bracketed by
torch.cuda.synchronize(); value = events / s over the K steps. The event
stream and node state are resident in HBM before the timed region; each
step draws its negatives inside it (the runtime draws a few consecutive
batches' negatives per CPU call and looks them up on the device) and
computes its (loss, AP, AUC, "mrr") on the device ("step_metrics").
The node state and optimizer are then restored and the same K steps are
replayed with HIP events around every library call (per-kernel breakdown and
the algorithmic work of the dominant kernel); the dominant kernel's events are
also recorded inside the timed region itself.
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import platform
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "starrygl-unidyngraph_amd"))

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
BF16_PEAK_TFLOPS = 2500.0   # dense bf16 MFMA
METRIC = "TGN train events/sec on 1 MI355X; sampler Mqueries/s; % HBM roofline"

WORKLOADS = {
    # precision: the benchmark's GEMM precision of the configuration (configs 4 and 5:
    # "bf16 GEMMs with fp32 memory"; configs 1 and 2: fp32)
    "tgn-large": dict(config="cfg4", stream="unipartite", family="tgn", D=100, T=100, H=2, k=10, K=1, B=600,
                      history=1, precision="bf16"),
    "tgn-small": dict(config="cfg1", stream="bipartite", family="tgn", D=100, T=100, H=2, k=10, K=1, B=200,
                      history=1),
    # config 2: memory + GRU + the JODIE time projection, no attention
    "jodie": dict(config="cfg2", stream="bipartite", family="jodie", D=100, T=100, H=2, k=10, K=1, B=200,
                  history=1, embedding="time_projection"),
    "tgn-stress": dict(config="cfg5", stream="unipartite", family="tgn", D=172, T=100, H=4, k=20, K=4, B=4000,
                       history=2, precision="bf16"),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def host_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


# --------------------------------------------------------------------------- sampler (config 3)
def sampler_bytes(deg_q, cnt) -> float:
    """Algorithmic bytes of the recent-k kernel, summed over queries:
    12 (node + t) + 16 (two row offsets) + 8*ceil(log2(deg+1)) (probes)
    + 16*k_eff (nbr i32 + eid i32 + ts i64 read) + 12*k_eff (nbr, eid, dt
    written) + 4 (count written)."""
    import torch
    probes = torch.ceil(torch.log2(deg_q.double() + 1.0))
    k = cnt.double()
    return float((12 + 16 + 8 * probes + 28 * k + 4).sum().item())


def run_sampler(steps: int, warmup: int, cases: bool = True, cpu: bool = True) -> dict:
    import torch

    from starry_unigraph import synth
    from starry_unigraph.native.tcsr import RecentSampler, build_tcsr

    dev = torch.device("cuda:0")
    t0 = time.time()
    g_np = synth.powerlaw_sampler_graph(seed=0)
    nodes_np, qt_np = synth.degree_weighted_queries(g_np, seed=1)
    log(f"config-3 graph generated in {time.time() - t0:.1f}s")
    g = build_tcsr(g_np.num_nodes, torch.from_numpy(g_np.row), torch.from_numpy(g_np.col), None,
                   torch.from_numpy(g_np.ts), device=dev)
    nodes = torch.from_numpy(nodes_np).to(dev)
    qt = torch.from_numpy(qt_np).to(dev)
    torch.cuda.synchronize()
    s = RecentSampler(g)
    deg = g.deg
    stream = torch.cuda.current_stream(dev)
    nq = nodes.numel()
    head = s.sample(nodes, qt, 10)
    for _ in range(warmup):
        s.sample(nodes, qt, 10, out=head)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    w0 = time.perf_counter()
    for a, b in evs:
        a.record(stream)
        s.sample(nodes, qt, 10, out=head)
        b.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    avg_ms = sum(a.elapsed_time(b) for a, b in evs) / len(evs)
    alg = sampler_bytes(deg[nodes], head.cnt)
    traffic = HBM_TRAFFIC.get(("cfg3", "int64", "recent_sample"))
    traffic_src = TRAFFIC_SOURCE["cfg3"] if traffic else None
    # diagnostics: the probe-free (compulsory) bytes, and the counter-measured bytes over the same time
    compulsory = float((12 + 16 + 28 * head.cnt.double() + 4).sum().item())
    out = {"value": nq * steps / wall / 1e6, "unit": "Mqueries/s", "ms_per_pass": wall * 1e3 / steps,
           "workload": "cfg3: 1e7 nodes, 1e8 edges, 4e6 degree-weighted queries, recent k=10, 1 hop",
           "roofline": {"bound": "hbm", "kernel": "k_recent_padded", "kernel_avg_ms": avg_ms,
                        "alg_bytes_per_launch": alg, "achieved": alg / (avg_ms * 1e-3) / 1e9,
                        "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": alg / (avg_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                        "traffic": traffic, "traffic_source": traffic_src,
                        "compulsory_bytes_per_launch": compulsory,
                        "traffic_rate_GBps": traffic / (avg_ms * 1e-3) / 1e9 if traffic else None}}
    del head
    if cases:
        res = {}
        for k in (10, 20):
            for hops in (1, 2):
                q_nodes, q_t, valid, stride = nodes, qt, None, 0
                per_hop = []
                for h in range(hops):
                    want_ts = h < hops - 1
                    ph = s.sample(q_nodes, q_t, k, want_ts=want_ts, valid_cnt=valid, stride=stride)
                    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    a.record(stream)
                    for _ in range(3):
                        s.sample(q_nodes, q_t, k, want_ts=want_ts, valid_cnt=valid, stride=stride, out=ph)
                    b.record(stream)
                    torch.cuda.synchronize()
                    ms = a.elapsed_time(b) / 3
                    if valid is None:
                        dq, cnt, live = deg[q_nodes], ph.cnt, q_nodes.numel()
                    else:
                        mask = (torch.arange(q_nodes.numel(), device=dev) % stride) < \
                            valid.long().repeat_interleave(stride)
                        dq, cnt, live = deg[q_nodes[mask].long()], ph.cnt[mask], int(mask.sum().item())
                    alg_h = sampler_bytes(dq, cnt) + 4 * (q_nodes.numel() - live)
                    per_hop.append({"queries": live, "ms": round(ms, 4), "alg_GBs": round(alg_h / ms / 1e6, 1),
                                    "entries": int(ph.cnt.sum().item())})
                    q_nodes, q_t, valid, stride = ph.nbr, ph.ts, ph.cnt, k
                tot = sum(p["ms"] for p in per_hop)
                res[f"k{k}_hop{hops}"] = {"ms": round(tot, 4), "Mqueries_per_s": round(nq / tot / 1e3, 1),
                                          "hops": per_hop}
                del ph, q_nodes, q_t, valid
                torch.cuda.empty_cache()
        out["cases"] = res
    if cpu:
        out["cpu_baseline"] = sampler_cpu_baseline(g_np, nodes_np, qt_np)
    del g, s, nodes, qt
    torch.cuda.empty_cache()
    return out


def sampler_cpu_baseline(g_np, nodes_np, qt_np) -> dict:
    """The C oracle (OpenMP over all host threads) on a bounded sample: the
    first 1e6 of the 4e6 queries, 1 hop, k = 10."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import numpy as np
    cores = host_cores()
    nq = len(nodes_np)
    nq1 = min(500_000, nq)
    try:
        import sampler_oracle as so
        so.set_threads(cores)
        og = so.build_tcsr(g_np.num_nodes, g_np.row, g_np.col, np.arange(g_np.num_edges), g_np.ts)
        so.sample_layer(og, nodes_np[:1000], qt_np[:1000], 10)
        t0 = time.perf_counter()
        so.sample_layer(og, nodes_np[:nq], qt_np[:nq], 10)
        dt = time.perf_counter() - t0
        # one thread: the reference's own setting on one GPU (workers = 1)
        so.set_threads(1)
        t0 = time.perf_counter()
        so.sample_layer(og, nodes_np[:nq1], qt_np[:nq1], 10)
        dt1 = time.perf_counter() - t0
        so.set_threads(cores)
        return {"value": nq / dt / 1e6, "unit": "Mqueries/s", "cores": cores, "kind": "port",
                "sample": f"1-hop k=10 recent over the {nq} config-3 queries (C oracle, OpenMP)",
                "cpu_model": cpu_model(),
                "one_thread": {"value": nq1 / dt1 / 1e6, "cores": 1,
                               "sample": f"the first {nq1} queries, 1 thread"}}
    except Exception as e:  # reported, never required
        return {"value": None, "unit": "Mqueries/s", "cores": cores, "kind": "port", "sample": f"failed: {e}"}


# --------------------------------------------------------------------------- gather / scatter
GS_BATCHES = (600, 4000, 1 << 20)


def gs_bytes(name: str, U: float, E: float, B: int, D: int, F: int, K: int) -> float:
    """Algorithmic HBM bytes of one launch of a front-part kernel."""
    S = 2 * D + F
    if name == "memory_commit":
        # root id, new row read, memory row + memory_ts written, sample count, bitmap word
        return U * (8 + 8 * D + 12)
    if name == "edge_rows":
        # per sampled edge: nbr, eid, the memory row and edge feature read and written into the edge's row
        return E * (8 + 8 * (D + F)) + U * 4
    if name == "memory_update":
        # per root: memory row, K mailbox rows + times read, new row written, one message (S + ts) written;
        # per event: src, dst, ts, edge feature read
        return U * (8 * D + 4 * K * S + 4 * K + 4 * S + 4) + B * (8 + 8 + 4 + 4 * F)
    if name == "batch_prepare":
        return B * (8 + 8 + 8 + 4) + U * 8
    return 0.0


# HBM bytes per launch at B = 1,048,576 (rocprofv3 FETCH_SIZE x 2.000 + WRITE_SIZE x 1.000, mean over
# four batches: profiles/gather_scatter_cfg5_B1M.md): k_memory_commit + k_edge_rows, and the same with
# the bf16 GRU + mailbox kernel (k_gru_mailbox_wide)
GS_TRAFFIC_1M = 43_632_742 + 92_720_026
GS_TRAFFIC_FULL_1M = GS_TRAFFIC_1M + 326_161_920


def run_gather_scatter(steps: int, warmup: int, batches=GS_BATCHES) -> dict:
    """The gather / scatter microbench: config-5 node state (the config-4
    stream's 1,140,149 nodes, D = 172, K = 4 mailbox slots, F = 16), batches of
    B consecutive events of that stream for B in `batches`: batch
    preparation, recent-k sampling (k = 20), the fused GRU + mailbox update
    (the roots' memory and mailbox rows gathered, the new messages
    scattered), the memory commit (scatter) and the edge-row gather; the
    one-kernel calls timed at their dispatch, the others by an event pair
    around the call; algorithmic bytes per call against HBM."""
    import torch

    from starry_unigraph import synth
    from starry_unigraph.native.step import ConvDims, DeviceStep, NodeState, gru_packed
    from starry_unigraph.native.tcsr import RecentSampler, build_tcsr

    dev = torch.device("cuda:0")
    t0 = time.time()
    es = synth.unipartite_stream(seed=0)
    log(f"gather/scatter: stream generated in {time.time() - t0:.1f}s ({es.num_events} events)")
    N, D, K, F, T, H, k = es.num_nodes, 172, 4, 16, 100, 4, 20
    src = torch.from_numpy(es.src).to(dev)
    dst = torch.from_numpy(es.dst).to(dev)
    ts = torch.from_numpy(es.ts).to(dev)
    ef = torch.from_numpy(es.edge_feat).to(dev)
    # the sampler graph over the whole stream (row = src, col = dst, int64 times truncated from float32)
    g = build_tcsr(N, src, dst, None, ts.to(torch.int64), device=dev)
    sampler = RecentSampler(g)
    state = NodeState(N, D, K, F, dev)
    gen = torch.Generator().manual_seed(0)
    S = 2 * D + F
    rnd = lambda *shape: ((torch.rand(*shape, generator=gen) * 2 - 1) / D ** 0.5).to(dev)
    gru = {"w_ih": rnd(3 * D, S), "w_hh": rnd(3 * D, D), "b_ih": rnd(3 * D), "b_hh": rnd(3 * D),
           "wc_ih": rnd(3 * D, D), "wc_hh": rnd(3 * D, D), "bc_ih": rnd(3 * D), "bc_hh": rnd(3 * D)}
    dims = ConvDims(D=D, F=F, T=T, H=H, fanout=k)
    names = ("batch_prepare", "recent_sample", "memory_update", "memory_commit", "edge_rows")
    cases = {}
    for B in batches:
        step = DeviceStep(state, dims, B, attention=False)
        nb = es.num_events // B
        agg = {n: [] for n in names}
        shapes = []
        # the one-kernel calls are timed at their own dispatch (sgl_time_next_launch:
        # no launch gaps); batch preparation and sampling launch several kernels
        # each and are timed by an event pair around the call, on the same stream
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
        single = {"memory_update", "memory_commit", "edge_rows"}
        timer = []
        step.timed = single
        for i in range(warmup + steps):
            step.timer = timer if i >= warmup else None
            # batches from the middle of the stream on, where the sampled windows are full
            a = ((nb // 2 + i) % nb) * B
            sb, db, tb = src[a:a + B], dst[a:a + B], ts[a:a + B]
            neg = db.roll(1)
            evs[0].record()
            step.prepare(sb, db, neg, tb)
            evs[1].record()
            step.sample(sampler)
            evs[2].record()
            step.update_memory(gru, sb, db, ef[a:a + B], tb)
            evs[3].record()
            step.commit()
            evs[4].record()
            step.edge_rows(ef)
            evs[5].record()
            if i >= warmup:
                torch.cuda.synchronize()
                U = int(step.buf.num_roots.item())
                E = int(step.buf.hop.cnt[:U].sum().item())
                shapes.append((U, E))
                for j, name in enumerate(names):
                    if name not in single:
                        agg[name].append((evs[j].elapsed_time(evs[j + 1]), U, E))
                for name, ev0, ev1 in timer:
                    agg[name].append((ev0.elapsed_time(ev1), U, E))
                timer.clear()
        # the same batches through the bf16-MFMA GRU (bf16 copies of the four weight matrices)
        gru16 = gru_packed(dict(gru, **{w: gru[w].to(torch.bfloat16).contiguous()
                                        for w in ("w_ih", "w_hh", "wc_ih", "wc_hh")}))
        agg["memory_update_bf16"] = []
        step.timed = {"memory_update"}
        for i in range(warmup + steps):
            a = ((nb // 2 + i) % nb) * B
            sb, db, tb = src[a:a + B], dst[a:a + B], ts[a:a + B]
            step.timer = timer if i >= warmup else None
            step.prepare(sb, db, db.roll(1), tb)
            step.update_memory(gru16, sb, db, ef[a:a + B], tb)
            step.timer = None
            step.commit()
            if i >= warmup:
                torch.cuda.synchronize()
                U = int(step.buf.num_roots.item())
                for name, ev0, ev1 in timer:
                    agg["memory_update_bf16"].append((ev0.elapsed_time(ev1), U, 0))
                timer.clear()
        step.timer = step.timed = None
        out = {}
        for name in names + ("memory_update_bf16",):
            ms = sum(x[0] for x in agg[name]) / len(agg[name])
            alg = sum(gs_bytes(name.replace("_bf16", ""), U, E, B, D, F, K) for _, U, E in agg[name]) / len(agg[name])
            row = {"avg_us": round(ms * 1e3, 2), "calls": len(agg[name])}
            if alg > 0:
                gbs = alg / (ms * 1e-3) / 1e9
                row.update({"alg_bytes": round(alg), "achieved": round(gbs, 1), "unit": "GB/s",
                            "frac": round(gbs / HBM_PEAK_GBS, 4)})
            out[name] = row
        cases[str(B)] = {"mean_roots": round(sum(u for u, _ in shapes) / len(shapes), 1),
                         "mean_sampled_edges": round(sum(e for _, e in shapes) / len(shapes), 1), "kernels": out}
        log(f"gather/scatter B={B}: " + ", ".join(f"{n} {v['avg_us']} us" + (f" ({v['achieved']} GB/s)" if
                                                                            "achieved" in v else "")
                                                 for n, v in out.items()))
        del step
        torch.cuda.empty_cache()
    big = cases[str(max(batches))]
    # the gather / scatter path of a step: the fused GRU + mailbox kernel (bf16 GEMMs, config 5's setting:
    # memory and mailbox rows gathered, messages scattered), the memory commit and the edge-row gather
    gs_names = ("memory_update_bf16", "memory_commit", "edge_rows")
    gb = sum(big["kernels"][n]["alg_bytes"] for n in gs_names)
    us = sum(big["kernels"][n]["avg_us"] for n in gs_names)
    gb2 = sum(big["kernels"][n]["alg_bytes"] for n in ("memory_commit", "edge_rows"))
    us2 = sum(big["kernels"][n]["avg_us"] for n in ("memory_commit", "edge_rows"))
    # the fused GRU + mailbox kernel is MFMA-bound at this state: 6DS K + 6D^2 (K-1) + 12D^2 flops per root
    gru_flop = big["mean_roots"] * (6 * D * S * K + 6 * D * D * (K - 1) + 12 * D * D)
    gru_tf = gru_flop / (big["kernels"]["memory_update"]["avg_us"] * 1e-6) / 1e12
    gru16_tf = gru_flop / (big["kernels"]["memory_update_bf16"]["avg_us"] * 1e-6) / 1e12
    return {"value": gb / (us * 1e-6) / 1e9, "unit": "GB/s",
            "workload": f"gather/scatter: cfg5 state (N={N}, D={D}, K={K}, F={F}), k={k}, batches {list(batches)}",
            "cases": cases,
            "roofline": {"bound": "hbm", "kernel": "k_gru_mailbox_wide<bf16> + k_memory_commit + k_edge_rows",
                         "batch": max(batches), "alg_bytes_per_launch": gb,
                         "achieved": gb / (us * 1e-6) / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
                         "traffic": GS_TRAFFIC_FULL_1M if max(batches) == 1 << 20 else None,
                         "traffic_source": "profiles/gather_scatter_cfg5_B1M.md",
                         "copy_kernels_only": {"kernel": "k_memory_commit + k_edge_rows",
                                               "achieved": gb2 / (us2 * 1e-6) / 1e9,
                                               "frac": gb2 / (us2 * 1e-6) / 1e9 / HBM_PEAK_GBS,
                                               "traffic": GS_TRAFFIC_1M if max(batches) == 1 << 20 else None,
                                               "traffic_source": "profiles/gather_scatter_cfg5_B1M.md"}},
            "gru_mfma": {"kernel": "k_gru_mailbox<float>", "batch": max(batches), "flop_per_launch": round(gru_flop),
                         "achieved": gru_tf, "peak": 157.3, "unit": "TFLOP/s", "frac": gru_tf / 157.3},
            "gru_mfma_bf16": {"kernel": "k_gru_mailbox_wide (bf16 GEMMs, fp32 accumulation, 64-root tiles)",
                              "batch": max(batches), "flop_per_launch": round(gru_flop), "achieved": gru16_tf,
                              "peak": 2500.0, "unit": "TFLOP/s", "frac": gru16_tf / 2500.0}}


# --------------------------------------------------------------------------- TGN end to end
def make_stream(wl: dict):
    from starry_unigraph import synth
    if wl["stream"] == "bipartite":
        return synth.bipartite_stream(seed=0)
    return synth.unipartite_stream(seed=0)


def build_session(wl: dict, stream):
    import torch

    from starry_unigraph import SchedulerSession
    from starry_unigraph.data import from_stream
    cfg = {"model": {"family": wl["family"], "hidden_dim": wl["D"]},
           "data": {"name": f"bench_{wl['config']}", "format": "synthetic"},
           "train": {"batch_size": wl["B"], "lr": 1e-3}, "runtime": {"device": "cuda"},
           "ctdg": {"mailbox_slots": wl["K"], "dim_time": wl["T"], "num_head": wl["H"],
                    "dropout": wl.get("dropout", 0.0), "att_dropout": wl.get("dropout", 0.0),
                    "memory_gemm_dtype": wl.get("gemm", "fp32"),
                    "attention_gemm_dtype": wl.get("attention_gemm", wl.get("gemm", "fp32"))
                    if wl.get("embedding", "attention") == "attention" else "fp32",
                    "embedding": wl.get("embedding", "attention")},
           "sampling": {"neighbor_limit": [wl["k"]] * wl["history"], "history": wl["history"],
                        "strategy": "recent"}}
    torch.manual_seed(0)
    sess = SchedulerSession.from_config(cfg).with_events(from_stream(stream))
    sess.build_runtime()
    return sess


class Epochs:
    """Training batches in order, epoch after epoch (memory is never reset
    between epochs, as in the reference). The runtime draws each batch's
    negatives inside its train_step (a few consecutive batches per CPU draw),
    so the draws fall inside the timed region."""

    def __init__(self, rt, B):
        self.rt, self.B = rt, B
        self._it = None

    def next(self):
        while True:
            if self._it is None:
                self._it = iter(self.rt.iter_batches("train", self.B))
            try:
                return next(self._it)
            except StopIteration:
                self._it = None


def _snapshot(rt):
    st = rt.memory.state
    opt = rt.optimizer.inner
    return ([t.clone() for t in (st.memory, st.mailbox, st.mailbox_ts, st.memory_ts, st.next_mail_pos)],
            [t.clone() for t in (opt.flat, opt.exp_avg, opt.exp_avg_sq)] + [seg[2].clone() for seg in opt.segments])


def _restore(rt, snap):
    st = rt.memory.state
    opt = rt.optimizer.inner
    for dst, src in zip((st.memory, st.mailbox, st.mailbox_ts, st.memory_ts, st.next_mail_pos), snap[0]):
        dst.copy_(src)
    for dst, src in zip([opt.flat, opt.exp_avg, opt.exp_avg_sq] + [seg[2] for seg in opt.segments], snap[1]):
        dst.copy_(src)
    rt.fence()


# HBM bytes per launch (read + written) of a kernel on a workload, from the
# rocprofv3 FETCH_SIZE / WRITE_SIZE runs summarised in
# profiles/tgn_cfg4_hbm_traffic.md and profiles/sampler_cfg3_hbm_traffic.md
# (counters scaled by a copy kernel of known size); None where no counter run
# was made.
HBM_TRAFFIC = {  # cfg4: read requests x their sizes (32/64/128 B) + write requests x theirs (64/32 B)
    ("cfg4", "bf16", "conv_backward"): 64 * 5720 + 128 * 28901 + 64 * 44874 + 32 * (48862 - 44874),
    ("cfg4", "bf16", "edge_rows"): 64 * 464 + 128 * 1622 + 64 * 4438 + 32 * (5072 - 4438),
    ("cfg4", "bf16", "memory_commit"): 64 * 288 + 128 * 875 + 64 * 1197 + 32 * (1827 - 1197),
    ("cfg4", "bf16", "conv_forward"): 64 * 5582 + 128 * 14860 + 64 * 29197 + 32 * (32231 - 29197),
    ("cfg4", "bf16", "memory_update"): 64 * 2673 + 128 * 23921 + 64 * 4539 + 32 * (5134 - 4539),
    ("cfg4", "bf16", "predictor"): 64 * 2512 + 128 * 4298 + 64 * 8194 + 32 * (10052 - 8194),
    ("cfg4", "bf16", "param_update"): 64 * 988 + 128 * 35652 + 64 * 30950 + 32 * (34587 - 30950),
    ("cfg4", "bf16", "batch_prepare"): 64 * 128 + 128 * 1305 + 64 * 691 + 32 * (3409 - 691),
    ("cfg4", "bf16", "recent_sample"): 64 * 472 + 128 * 5531 + 64 * 123 + 32 * (585 - 123),
    ("cfg4", "bf16", "link_metrics"): 64 * 1096 + 128 * 307 + 64 * 3 + 32 * (25 - 3),
    ("cfg3", "int64", "recent_sample"): round((2 * 1342192 + 449830) * 1024)}
# the counter runs the HBM_TRAFFIC figures come from (the same kernels at the same workload)
TRAFFIC_SOURCE = {"cfg4": "profiles/tgn_cfg4_hbm_traffic.md", "cfg3": "profiles/sampler_cfg3_hbm_traffic.md"}

# step stage name -> the C-ABI entry point that launches it
ENTRY_POINTS = {"batch_prepare": "sgl_batch_prepare", "recent_sample": "sgl_recent_sample",
                "memory_update": "sgl_memory_update", "memory_commit": "sgl_memory_commit",
                "edge_rows": "sgl_edge_rows", "conv_forward": "sgl_conv_forward", "predictor": "sgl_predictor",
                "conv_backward": "sgl_conv_backward", "param_update": "sgl_grad_adam",
                "time_projection": "sgl_time_projection_forward",
                "time_projection_backward": "sgl_time_projection_backward"}


def mfma_peak(name: str, wl: dict) -> float:
    """The dense MFMA peak of the precision a step kernel's products run in
    (the fused Adam's weight-gradient products are fp32 in every mode)."""
    bf = wl.get("gemm") == "bf16" and name in ("conv_forward", "conv_backward", "predictor", "memory_update")
    return BF16_PEAK_TFLOPS if bf else FP32_PEAK_TFLOPS


def kernel_work(name: str, wl: dict, U: int, E: int, B: int, dims) -> tuple[str, float, float]:
    """Work of one launch: (bound, algorithmic, executed) -- ("hbm", bytes,
    bytes) or ("mfma", flops, flops). The attention's algorithmic flops are
    the reference algorithm's (per-edge K / V projections):
    2U(D+T)D + 4E(D+F+T)D + 4UD^2 forward and twice that backward; the
    executed count is what the re-associated kernels do (K / V projected
    per root, q~ = W_k^T q per head)."""
    D, F, T, H, k, K = wl["D"], dims.F, wl["T"], wl["H"], wl["k"], wl["K"]
    C = D + F + T
    S = 2 * D + F
    fwd_alg = float(U) * (2 * (D + T) * D + 4 * D * D) + float(E) * 4 * C * D
    if name == "memory_update":
        # GRU over K slots + GRUCell per updated root
        f = float(U) * (6 * D * S * K + 6 * D * D * (K - 1) + 12 * D * D)
        return "mfma", f, f
    if name == "conv_forward":
        # executed: Q (2D(D+T)), qt (2DC), per edge 4HC (scores + weighted sum), agg (2CD), z (4D*D)
        return "mfma", fwd_alg, float(U) * (2 * D * (D + T) + 2 * D * C + 2 * C * D + 4 * D * D) + float(E) * 4 * H * C
    if name == "conv_backward":
        # executed: dL/dy from the predictor rows (4D*D), gagg (2D*D), gxbar (2D*C), per edge 8HC, gQ (2CD)
        return "mfma", 2 * fwd_alg, float(U) * (4 * D * D + 2 * D * D + 2 * D * C + 2 * C * D) + float(E) * 8 * H * C
    if name == "predictor":
        # per event: src_fc, dst_fc (positive and negative) 6D^2, out_fc and the logit gradients 12D
        f = float(B) * (6 * D * D + 12 * D)
        return "mfma", f, f
    if name == "param_update":
        # weight-gradient reductions over the roots: w_q (D x (D+T)), w_k, w_v (D x C), w_out (D x 2D),
        # src_fc / dst_fc (D x D over U + 1 rows); 2 flops per multiply-add
        f = float(U) * 2 * (D * (D + T) + 2 * D * C + 2 * D * D) + float(U + 1) * 2 * 2 * D * D
        return "mfma", f, f
    if name == "memory_commit":
        b = float(U) * (8 + 4 * D * 2 + 4)
    elif name == "edge_rows":
        # per sampled edge: nbr, eid read, the memory row and edge feature gathered and written into the
        # edge's row; per root its count
        b = float(E) * (8 + 8 * D + 8 * F) + float(U) * 4
    elif name == "recent_sample":
        b = float(U) * (12 + 16 + 8 * 8 + 4) + float(E) * 28
    elif name == "batch_prepare":
        b = float(B) * (8 + 8 + 8 + 4) + float(U) * 8
    else:
        b = 0.0
    return "hbm", b, b


def param_update_bytes(wl: dict, U: float, dims, n_params: int, n_shadow: int, tile_rows: int) -> float:
    """Algorithmic HBM bytes of one fused weight-gradient + Adam launch
    (sgl_grad_adam): every per-root row its reductions read once -- gQ,
    new_mem, Q, gagg, gz, agg [U][D], G, xbar [U][H][C], sigma [U][H]; y,
    g_src, g_dst [U+1][D] for src_fc / dst_fc; the LayerNorm and
    time-encoding partials [U/tile][2][D], [U/tile][2][T] -- plus Adam's
    28 bytes per parameter (parameter, gradient and both moments read;
    parameter and moments written) and the bf16 weight copies written."""
    D, T, H = wl["D"], wl["T"], wl["H"]
    C = D + dims.F + T
    rows = U * 4.0 * (6 * D + 2 * H * C + H) + (U + 1) * 4.0 * 3 * D
    parts = (U / max(1, tile_rows)) * 4.0 * 2 * (D + T)
    return rows + parts + 28.0 * n_params + 2.0 * n_shadow


def copy_bandwidth(mib: int = 2048, reps: int = 10) -> dict:
    """A device-to-device copy of a known size (read + write), the measured
    HBM bandwidth the roofline fractions can also be read against."""
    import torch
    n = mib * (1 << 18)
    a = torch.ones(n, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del a, b
    torch.cuda.empty_cache()
    return {"GBps": 2 * n * 4 / (ms * 1e-3) / 1e9, "bytes_per_copy": 2 * n * 4, "ms": ms,
            "kernel": "torch copy_ (device to device)"}


def run_tgn(args, wl: dict) -> dict:
    import torch

    t0 = time.time()
    stream = make_stream(wl)
    log(f"{wl['config']} stream generated in {time.time() - t0:.1f}s ({stream.num_events} events)")
    sess = build_session(wl, stream)
    rt = sess.ctdg_session.online_runtime
    rt.collect_results = False
    rt.use_plans = not args.no_plans
    ep = Epochs(rt, wl["B"])
    dev = torch.device("cuda:0")
    if args.epoch:  # the reference's definition: one warm-up epoch, then one timed epoch of train batches
        n_train = -(-int(rt.dataset.split_event_ids("train").numel()) // wl["B"])
        args.steps = args.warmup = n_train
        log(f"epoch mode: {n_train} train batches per epoch")
    # the eager per-kernel replay below starts from this snapshot and replays
    # the warm-up steps first; taken (and the collector run) before the
    # warm-up, so that neither the snapshot's copies nor a collection evict
    # the GPU's and the host's caches just before the timed region
    warm = [ep.next() for _ in range(args.warmup)]
    snap = _snapshot(rt)
    gc.collect()
    for b in warm:
        out = rt.train_step(b)
    torch.cuda.synchronize()
    log(f"warm-up done ({args.warmup} steps)")

    batches = [ep.next() for _ in range(args.steps)]
    dom = args.roofline_kernel or ("memory_update" if wl.get("embedding") == "time_projection" else "conv_forward")
    timer: list = []
    if args.no_plans:   # eager steps: time the dominant kernel inside the timed region
        for st in rt.steps:
            st.timer, st.timed = timer, {dom}
    else:   # planned steps: HIP events at the dominant kernel's dispatch in steps 10, 74, 138, ...
        # (a timed dispatch costs the host tens of microseconds: few samples, none at the cold start)
        every, first = 64, min(10, args.steps - 1)
        pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                 for _ in range((args.steps - first + every - 1) // every)]
        for a, b in pairs:   # torch creates the HIP event at its first record
            a.record()
            b.record()
        count = [0]

        def next_pair():
            i = count[0]
            count[0] += 1
            if i < first or (i - first) % every:
                return None
            p = pairs[(i - first) // every]
            timer.append((dom, p[0], p[1]))
            return p

        rt.plan_timer = (ENTRY_POINTS[dom], next_pair)
    torch.cuda.synchronize()
    gc.disable()   # no collector pauses on the host inside the timed region
    waited0 = rt._draws.wait_s
    w0 = time.perf_counter()
    out = None
    for b in batches:
        out = rt.train_step(b)
    host = time.perf_counter() - w0
    # the host blocks only when it runs a full draw ring (four chunks of draws) ahead of the GPU
    waited = rt._draws.wait_s - waited0
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    gc.enable()
    rt.plan_timer = None
    rt.check_sync()
    log(f"host-side loop {host * 1e6 / args.steps:.1f} us/step, of which {waited * 1e6 / args.steps:.1f} waiting "
        f"for the GPU (a full draw ring ahead of it): {(host - waited) * 1e6 / args.steps:.1f} us/step of host "
        f"work (the rest is the GPU draining its queue)")
    events = sum(b.size for b in batches)
    # every timed step's (loss, AP, AUC, "mrr"), computed on the device at the end
    # of its back part (sgl_link_metrics) inside the timed region; read once here
    met = rt.metrics_of_last_steps(args.steps) if rt.device_metrics else None
    step_metrics = None
    if met is not None and met.shape[0] == args.steps:
        mean = met.mean(0).tolist()
        step_metrics = {"steps": int(met.shape[0]), "mean_loss": mean[0], "mean_ap": mean[1], "mean_auc": mean[2],
                        "mean_mrr": mean[3], "last": met[-1].tolist(),
                        "computed": "per step on the device inside the timed region (sgl_link_metrics: "
                                    "runtime.py:202-214's sklearn AP/AUC and pairwise mrr), no host sync"}
    dom_ms = [a.elapsed_time(b) for _, a, b in timer]
    # the step's loss is a view of a reused step buffer: read the last one
    final_loss = float(out["loss"].item()) if out is not None else float("nan")
    log(f"timed {args.steps} steps: {wall * 1e3 / args.steps:.3f} ms/step, {events / wall:.0f} events/s")

    # replay the same steps eagerly with every library call timed + per-step counts
    _restore(rt, snap)
    for b in warm:   # untimed: back to the state the timed region started from
        rt.train_step(b)
    for st in rt.steps:
        st.timer, st.timed = timer, None
    timer.clear()
    per_step = []
    for b in batches:
        n0 = len(timer)
        rt.train_step(b)
        buf = rt.step.buf
        U = int(buf.num_roots.item())
        E = int(buf.hop.cnt[:U].sum().item())
        per_step.append((n0, len(timer), U, E, b.size))
    torch.cuda.synchronize()
    agg: dict[str, list] = {}
    work: dict[str, list] = {}
    for n0, n1, U, E, B in per_step:
        for name, a, b in timer[n0:n1]:
            agg.setdefault(name, []).append(a.elapsed_time(b))
            work.setdefault(name, []).append(kernel_work(name, wl, U, E, B, rt.dims)[1:])
    breakdown = {}
    for name, ms in agg.items():
        avg = sum(ms) / len(ms)
        bound = kernel_work(name, wl, 1, 1, 1, rt.dims)[0]
        wavg = sum(w[0] for w in work[name]) / len(work[name])
        if bound == "mfma":
            ach, peak, unit = wavg / (avg * 1e-3) / 1e12, mfma_peak(name, wl), "TFLOP/s"
        else:
            ach, peak, unit = wavg / (avg * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s"
        breakdown[name] = {"avg_us": round(avg * 1e3, 2), "calls": len(ms), "bound": bound,
                           "achieved": round(ach, 3), "unit": unit, "frac": round(ach / peak, 5),
                           "traffic": HBM_TRAFFIC.get((wl["config"], wl.get("gemm", "fp32"), name))}
        if name == "param_update" and wl.get("embedding", "attention") == "attention":
            # the fused launch is also a streaming kernel: its algorithmic bytes against HBM
            from starry_unigraph.lib import _capi
            U_avg = sum(p[2] for p in per_step) / len(per_step)
            d = rt.dims
            tile_rows = int(_capi.lib().sgl_conv_backward_tile_rows(d.D, d.F, d.T, d.H, int(rt._bf16 is not None)))
            nb = param_update_bytes(wl, U_avg, rt.dims, rt.optimizer.inner.flat.numel(),
                                    rt._bf16.buf.numel() if rt._bf16 is not None else 0, tile_rows)
            gbs = nb / (avg * 1e-3) / 1e9
            breakdown[name]["hbm"] = {"alg_bytes": round(nb), "achieved": round(gbs, 1), "unit": "GB/s",
                                      "frac": round(gbs / HBM_PEAK_GBS, 5),
                                      "formula": "param_update_bytes(): rows read once + 28 B per parameter "
                                                 "+ the bf16 copies"}
    mean_U = sum(p[2] for p in per_step) / len(per_step)
    mean_E = sum(p[3] for p in per_step) / len(per_step)
    if not dom_ms:   # no timed launches in the timed region: the eager replay's
        dom_ms = agg[dom]
    dom_avg = sum(dom_ms) / max(1, len(dom_ms))
    bound = kernel_work(dom, wl, 1, 1, 1, rt.dims)[0]
    dwork = sum(w[0] for w in work[dom]) / len(work[dom])
    dexec = sum(w[1] for w in work[dom]) / len(work[dom])
    scale = 1e12 if bound == "mfma" else 1e9
    peak, unit = (mfma_peak(dom, wl), "TFLOP/s") if bound == "mfma" else (HBM_PEAK_GBS, "GB/s")
    ach = dwork / (dom_avg * 1e-3) / scale
    tkey = (wl["config"], wl.get("gemm", "fp32"), dom)
    res = {
        "value": events / wall, "unit": "events/s", "ms_per_step": wall * 1e3 / args.steps,
        "final_train_loss": final_loss,
        "step_metrics": step_metrics,
        "roofline": {"bound": bound, "kernel": dom, "achieved": ach, "peak": peak, "unit": unit,
                     "frac": ach / peak, "traffic": HBM_TRAFFIC.get(tkey),
                     "traffic_source": TRAFFIC_SOURCE.get(wl["config"]) if tkey in HBM_TRAFFIC
                     else None,
                     "kernel_avg_ms": dom_avg, "work_per_launch": dwork,
                     "work_formula": "attention projections, uncombined (models.py:77-137): 2U(D+T)D + 4E(D+F+T)D + 4UD^2 "
                                     "(x2 backward)" if dom.startswith("conv_") else "see kernel_work()",
                     "work_executed_per_launch": dexec,
                     "frac_executed": dexec / (dom_avg * 1e-3) / scale / peak},
        "kernels": breakdown,
        "step_shape": {"mean_roots": round(mean_U, 1), "mean_sampled_edges": round(mean_E, 1)},
    }
    for st in rt.steps:
        st.timer = None
    if not args.no_cpu:
        res["cpu_baseline"] = tgn_cpu_baseline(wl, stream, rt)
    return res


def run_tgn_short(wl: dict, steps: int, warmup: int) -> dict:
    """A configuration's training steps timed as the headline's are (W warm-up
    steps, then K planned asynchronous steps between synchronizes, negatives
    and per-step device metrics inside the timed region), without the
    per-kernel replay: the driver-timed number of a configuration other than
    the headline's."""
    import torch

    stream = make_stream(wl)
    sess = build_session(wl, stream)
    rt = sess.ctdg_session.online_runtime
    rt.collect_results = False
    ep = Epochs(rt, wl["B"])
    for _ in range(warmup):
        rt.train_step(ep.next())
    torch.cuda.synchronize()
    batches = [ep.next() for _ in range(steps)]
    gc.collect()
    gc.disable()
    w0 = time.perf_counter()
    for b in batches:
        rt.train_step(b)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    gc.enable()
    rt.check_sync()
    met = rt.metrics_of_last_steps(steps).mean(0).tolist()
    events = sum(b.size for b in batches)
    gemm = wl.get("gemm", "fp32")
    att = wl.get("attention_gemm", gemm) if wl.get("embedding", "attention") == "attention" else None
    out = {"value": events / wall, "unit": "events/s", "ms_per_step": wall * 1e3 / steps, "steps": steps,
           "warmup": warmup,
           "config": {"workload": wl["config"], "model": wl["family"] + (" (time projection)"
                                                                       if wl.get("embedding") == "time_projection"
                                                                       else ""),
                      "D": wl["D"], "T": wl["T"], "H": wl["H"], "k": wl["k"], "sampled_hops": wl["history"],
                      "attention_layers": 1 if att is not None else 0, "K": wl["K"], "B": wl["B"],
                      "dropout": wl.get("dropout", 0.0)},
           "dtype": f"GRU {gemm}" + (f", attention and predictor {att}" if att is not None else "")
                    + " GEMMs; fp32 memory and Adam",
           "mean_step_metrics": {"loss": met[0], "ap": met[1], "auc": met[2], "mrr": met[3]}}
    del rt, sess, stream
    gc.collect()
    torch.cuda.empty_cache()
    return out


def tgn_cpu_baseline(wl: dict, stream, rt) -> dict:
    """The torch-CPU oracle step (C oracle sampler + memory/GRU + attention +
    predictor + Adam), all host threads, on a bounded prefix of the training
    stream: the first N batches from zero memory."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import numpy as np
    import torch
    cores = host_cores()
    nsteps = 2000 if wl["B"] <= 1000 else 100   # ~10 s of host work at config 4
    nsteps1 = 200 if wl["B"] <= 1000 else 10    # the one-thread run
    try:
        import ctdg_oracle as co
        import sampler_oracle as so
        torch.set_num_threads(cores)
        so.set_threads(cores)
        ds = rt.dataset
        model, updater = co.build_models(wl["D"], ds.edge_feat_dim, wl["T"], wl["H"], wl["K"], seed=0)
        opt = torch.optim.Adam(list(model.parameters()) + list(updater.parameters()), lr=1e-3)
        mem = co.MemoryO(ds.num_nodes, wl["D"], wl["K"], ds.edge_feat_dim)
        g = ds.sampler_graph("train")
        og = so.build_tcsr(ds.num_nodes, g["row"].numpy(), g["col"].numpy(), g["eid"].numpy(), g["ts"].numpy())
        pool = ds.dst.unique()
        gen = torch.Generator().manual_seed(0)
        it = ds.iter_batches("train", wl["B"])
        k = wl["k"]
        fn = lambda r, t: co.block_from_oracle_sampler(og, r, t, k)
        b = next(it)
        neg = co.negative_sample(pool, b.dst, gen)
        co.train_step(model, updater, opt, mem, fn, b.src, b.dst, b.ts, b.edge_feat, neg, ds.edge_feat)
        t0 = time.perf_counter()
        n = 0
        for _ in range(nsteps):
            b = next(it)
            neg = co.negative_sample(pool, b.dst, gen)
            co.train_step(model, updater, opt, mem, fn, b.src, b.dst, b.ts, b.edge_feat, neg, ds.edge_feat)
            n += b.size
        dt = time.perf_counter() - t0
        # one thread (the reference's own setting on one GPU), the next batches
        torch.set_num_threads(1)
        so.set_threads(1)
        t0 = time.perf_counter()
        n1 = 0
        for _ in range(nsteps1):
            b = next(it)
            neg = co.negative_sample(pool, b.dst, gen)
            co.train_step(model, updater, opt, mem, fn, b.src, b.dst, b.ts, b.edge_feat, neg, ds.edge_feat)
            n1 += b.size
        dt1 = time.perf_counter() - t0
        torch.set_num_threads(cores)
        so.set_threads(cores)
        return {"value": n / dt, "unit": "events/s", "cores": cores, "kind": "port",
                "sample": f"{nsteps} training steps (batches 2..{nsteps + 1} of the epoch, B={wl['B']}) of the "
                          f"torch-CPU oracle step incl. the C oracle sampler; {dt:.1f}s",
                "cpu_model": cpu_model(),
                "one_thread": {"value": n1 / dt1, "cores": 1,
                               "sample": f"the next {nsteps1} steps, 1 thread; {dt1:.1f}s"}}
    except Exception as e:  # reported, never required
        return {"value": None, "unit": "events/s", "cores": cores, "kind": "port", "sample": f"failed: {e!r}"}


# --------------------------------------------------------------------------- main
def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-plans", action="store_true",
                    help="run steps eagerly (one library call at a time) instead of as recorded launch plans")
    ap.add_argument("--workload", default="tgn-large",
                    choices=sorted(list(WORKLOADS) + ["sampler", "gather-scatter"]))
    ap.add_argument("--roofline-kernel", default=None,
                    choices=["batch_prepare", "recent_sample", "memory_update", "memory_commit", "edge_rows",
                             "conv_forward", "conv_backward"],
                    help="the kernel the roofline object measures (default: conv_forward, or memory_update "
                         "for the time-projection workload, which has no attention)")
    ap.add_argument("--no-sampler", action="store_true", help="skip the config-3 sampler sub-benchmark")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the short runs of configs 1, 2, 5 and config 4 with dropout")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--epoch", action="store_true",
                    help="TGN workloads: one warm-up epoch, then time one epoch of train batches (overrides "
                         "--steps / --warmup)")
    ap.add_argument("--gemm-dtype", default="auto", choices=["auto", "fp32", "bf16"],
                    help="the GRU, attention and edge-predictor GEMMs of the TGN workloads: fp32 MFMA, or bf16 "
                         "MFMA on bf16 weight copies with fp32 accumulation and fp32 memory; auto: the "
                         "configuration's benchmark precision (configs 4 and 5 bf16, configs 1 and 2 fp32)")
    ap.add_argument("--no-gather-scatter", action="store_true",
                    help="skip the gather/scatter sub-benchmark of the default run")
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="first run 3 device-to-device copies of this many MiB (a known-size kernel for "
                         "calibrating FETCH_SIZE / WRITE_SIZE counter runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU (the GPU boxes here have one); multi-GPU "
                                   "sharding is a design note, not a measured path", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    if args.copy_probe_mb > 0:
        src = torch.ones(args.copy_probe_mb * (1 << 18), device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)   # an elementwise kernel: reads and writes the size once
        torch.cuda.synchronize()
        log(f"copy probe: 3 device copies of {args.copy_probe_mb} MiB")
        del src, dst
    base = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "data": "synthetic (seeded PCG64 generators, starry_unigraph.synth)"}
    if args.workload == "gather-scatter":
        r = run_gather_scatter(args.steps, args.warmup)
        line = dict(base, value=r["value"], unit=r["unit"], ms_per_step=None, dtype="fp32",
                    config={"workload": r["workload"], "global_batch": max(GS_BATCHES), "parallelism": "single GPU"},
                    roofline=r["roofline"], cpu_baseline=None, cases=r["cases"])
        print(json.dumps(line), flush=True)
        return
    if args.workload == "sampler":
        r = run_sampler(args.steps, args.warmup, cpu=not args.no_cpu)
        line = dict(base, value=r["value"], unit=r["unit"], ms_per_step=r["ms_per_pass"], dtype="int64",
                    config={"workload": r["workload"], "global_batch": 4_000_000, "parallelism": "single GPU"},
                    roofline=r["roofline"], cpu_baseline=r.get("cpu_baseline"), cases=r.get("cases"))
        print(json.dumps(line), flush=True)
        return
    wl = WORKLOADS[args.workload]
    gemm = wl.get("precision", "fp32") if args.gemm_dtype == "auto" else args.gemm_dtype
    wl = dict(wl, gemm=gemm)
    r = run_tgn(args, wl)
    base.update(steps=args.steps, warmup=args.warmup)  # --epoch sets them from the split
    line = dict(base, value=r["value"], unit=r["unit"], ms_per_step=r["ms_per_step"],
                dtype="fp32" if gemm == "fp32" else "bf16 (GEMM operands; fp32 accumulation, memory and Adam)",
                config={"workload": (f"{wl['config']} ({args.workload}): JODIE train step (memory + GRU + time "
                                     f"projection, no attention), D={wl['D']} K={wl['K']} B={wl['B']}"
                                     if wl.get("embedding") == "time_projection" else
                                     f"{wl['config']} ({args.workload}): TGN train step, D={wl['D']} T={wl['T']} "
                                     f"H={wl['H']} k={wl['k']} sampled_hops={wl['history']} attention_layers=1 K={wl['K']} "
                                     f"B={wl['B']}, "
                                     "dropout 0"),
                        "global_batch": wl["B"], "parallelism": "single GPU"},
                roofline=r["roofline"], cpu_baseline=r.get("cpu_baseline"), kernels=r["kernels"],
                step_shape=r["step_shape"], final_train_loss=r["final_train_loss"], step_metrics=r["step_metrics"])
    line["hbm_copy"] = copy_bandwidth()
    if args.workload == "tgn-large" and not args.no_configs:
        # every other configuration's training step, driver-timed (20 steps after 5 warm-up steps):
        # configs 1, 2 and 5, and config 4 with the reference's default dropout 0.1
        # (config/default.yaml:152-153; the dropout passes run the fp32 attention instances)
        others = {"cfg1": WORKLOADS["tgn-small"], "cfg2": WORKLOADS["jodie"],
                  "cfg5": dict(WORKLOADS["tgn-stress"], gemm=WORKLOADS["tgn-stress"]["precision"]),
                  "cfg4_dropout": dict(WORKLOADS["tgn-large"], gemm="bf16", attention_gemm="fp32", dropout=0.1)}
        line["configs"] = {}
        for name, w in others.items():
            r2 = run_tgn_short(w, 20, 5)
            log(f"{name}: {r2['ms_per_step']:.3f} ms/step, {r2['value']:.0f} events/s")
            line["configs"][name] = r2
    if args.workload == "tgn-large" and not args.no_sampler:
        line["sampler"] = run_sampler(20, 3, cases=True, cpu=not args.no_cpu)
    if args.workload == "tgn-large" and not args.no_gather_scatter:
        gs = run_gather_scatter(5, 1)
        line["gather_scatter"] = {k: gs[k] for k in ("value", "unit", "workload", "roofline", "gru_mfma",
                                                      "gru_mfma_bf16")}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
