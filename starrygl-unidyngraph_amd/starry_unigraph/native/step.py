"""Device side of one CTDG step: HBM-resident node state, capacity-sized step
buffers and the kernel sequence (all through the C ABI, no host syncs).

Kernel order of a training step (reference: CTDGOnlineRuntime.train_step,
backends/ctdg/runtime/runtime.py:225-297):

  sgl_batch_prepare   roots, query time, per-role last writers     (runtime.py:138-144)
  sgl_recent_sample   hop-0 recent-k windows of the roots          (sampler.py:93-128)
  sgl_memory_update   GRU over mailbox + memory, mailbox write     (runtime.py:268-282)
  sgl_memory_commit   memory/memory_ts scatter                     (memory.py:254-269)
  sgl_conv_forward    time encoding + temporal attention           (models.py:77-137)
  sgl_predictor       edge predictor + BCE, per-root gradient sums (models.py:313-324, runtime.py:290-292)
  sgl_conv_backward   attention backward                           (loss.backward(), runtime.py:296)
  sgl_grad_adam       weight gradients + Adam, the attention segments
                      gated by "block has edges"                   (optimizer.step(), runtime.py:297)

The first three are a step's front part, the memory commit its split point,
the rest its back part (see the runtime's launch plans).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from starry_unigraph.lib import _capi
from starry_unigraph.native.tcsr import PaddedHop, RecentSampler

TILE = 16


def _round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


def per_workgroup_jobs(jobs: list, deal: list[int]) -> list:
    """sgl_grad_adam's job table without tile_job: one copy of its job per
    entry of ``deal`` (xcd_tile_deal), the tile's index within the job in
    tile0, and a job of kind -1 for a padding slot (workgroup t reads entry t,
    one load where the indexed form takes two in a row)."""
    out = []
    for e in deal:
        if e < 0:
            j = _capi.GradJob()
            j.kind = -1
        else:
            j = _capi.GradJob.from_buffer_copy(jobs[e & 0xFF])
            j.tile0 = e >> 8
        out.append(j)
    return out


def xcd_tile_deal(counts: list[int], xcds: int = 8) -> list[int]:
    """The tile_job table of sgl_grad_adam / sgl_grad_shadows for jobs of
    ``counts`` tiles: entry t (workgroup t, which runs on XCD t % xcds) is
    job | (index among the job's tiles << 8), or -1 for a padding slot. Each
    XCD takes at most ceil(total / xcds) tiles; the jobs go, largest first, to
    the XCD with the fewest tiles, a job that does not fit split into ranges
    of consecutive tiles, so that most jobs' activation strips are fetched by
    one XCD's L2."""
    if len(counts) > 256:
        raise ValueError("xcd_tile_deal: more than 256 jobs")
    total = sum(counts)
    if total == 0:
        return []
    cap = -(-total // xcds)
    bins: list[list[int]] = [[] for _ in range(xcds)]
    for job in sorted(range(len(counts)), key=lambda k: (-counts[k], k)):
        local, left = 0, counts[job]
        if left >= 1 << 23:
            raise ValueError("xcd_tile_deal: a job of more than 2^23 tiles")
        while left > 0:
            b = min(range(xcds), key=lambda k: (len(bins[k]), k))
            take = min(left, cap - len(bins[b]))
            bins[b].extend(job | (loc << 8) for loc in range(local, local + take))
            local += take
            left -= take
    n = max(len(b) for b in bins)
    return [bins[t % xcds][t // xcds] if t // xcds < len(bins[t % xcds]) else -1 for t in range(n * xcds)]


class NodeState:
    """Per-node memory and K-slot mailbox in HBM (memory.py:98-102):
    memory [N,D] f32 = 0, mailbox [N,K,2D+F] f32 = 0, mailbox_ts [N,K] = 0,
    memory_ts [N] = -1, next_mail_pos [N] (int32 here) = 0; plus the node
    bitmap the batch preparation uses (kept all-zero between steps)."""

    def __init__(self, num_nodes: int, hidden_dim: int, slots: int, edge_dim: int, device):
        dev = _capi.require_gpu(device)
        self.device = dev
        self.N, self.D, self.K, self.F = int(num_nodes), int(hidden_dim), int(slots), int(edge_dim)
        self.S = 2 * self.D + self.F
        with torch.cuda.device(dev):
            self.memory = torch.zeros(self.N, self.D, dtype=torch.float32, device=dev)
            self.mailbox = torch.zeros(self.N, self.K, self.S, dtype=torch.float32, device=dev)
            self.mailbox_ts = torch.zeros(self.N, self.K, dtype=torch.float32, device=dev)
            self.memory_ts = torch.full((self.N,), -1.0, dtype=torch.float32, device=dev)
            self.next_mail_pos = torch.zeros(self.N, dtype=torch.int32, device=dev)
            # node bitmap + its summary (layout owned by the library)
            self.node_bits = torch.zeros(int(_capi.lib().sgl_node_bits_words(self.N)), dtype=torch.int32, device=dev)
            self.word_prefix = torch.zeros((self.N + 31) // 32 + 3 & ~3, dtype=torch.int32, device=dev)
        # count of writes queued by tensor code outside the fused step (a
        # pipelined step orders itself after them when the count changes)
        self.writes = 0

    def touched(self) -> None:
        """Record that tensor code queued writes to the state on the current stream."""
        self.writes += 1

    def reset(self) -> None:
        self.touched()
        self.memory.zero_()
        self.mailbox.zero_()
        self.mailbox_ts.zero_()
        self.memory_ts.fill_(-1.0)
        self.next_mail_pos.zero_()
        self.node_bits.zero_()

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in
                   (self.memory, self.mailbox, self.mailbox_ts, self.memory_ts, self.next_mail_pos))


@dataclass
class ConvDims:
    D: int
    F: int
    T: int
    H: int
    fanout: int

    @property
    def C(self) -> int:
        return self.D + self.F + self.T


class StepBuffers:
    """Scratch for batches of up to ``max_batch`` events; root-indexed arrays
    hold cap = round_up(2*max_batch, 16) rows (the most roots a batch can
    have), so launch shapes never depend on the batch."""

    def __init__(self, max_batch: int, dims: ConvDims, device, attention: bool = True,
                 more_fanouts: tuple[int, ...] = (), passes: int = 1):
        """``attention`` False: only the buffers of the front part (batch
        preparation, sampling, memory / mailbox update, commit, edge rows).
        ``more_fanouts``: the fanouts of the hops after hop 0 (history > 1):
        hop l's queries are hop l-1's padded rows, so it holds
        cap * fanout_0 * ... * fanout_l slots. ``passes``: 3 for training with
        dropout (the attention runs once per role, runtime.py:193-195, each
        pass with its own saved state, stacked along the rows), else 1."""
        dev = torch.device(device)
        self.device = dev
        self.max_batch = int(max_batch)
        self.cap = _round_up(max(2 * self.max_batch, TILE), TILE)
        c, B, D, H, C, k = self.cap, self.max_batch, dims.D, dims.H, dims.C, dims.fanout
        z = lambda *s, dt=torch.float32: torch.zeros(*s, dtype=dt, device=dev)
        i32, i64 = torch.int32, torch.int64
        self.num_roots = z(1, dt=i32)
        self.num_roots64 = z(1, dt=i64)
        self.batch_start = z(1, dt=i64)
        self.ts_max = z(1)
        self.t_query = z(1, dt=i64)
        self.any_edges = z(1, dt=i32)
        self.err = _capi.ErrorFlag(dev)
        self.roots = z(c, dt=i64)
        self.root_ts = z(c, dt=i64)
        self.ridx_src = z(max(B, 1), dt=i32)
        self.ridx_dst = z(max(B, 1), dt=i32)
        self.ridx_neg = z(max(B, 1), dt=i32)
        self.win_src = z(c, dt=i64)
        self.win_dst = z(c, dt=i64)
        self.cnt_src = z(c, dt=i32)
        self.cnt_dst = z(c, dt=i32)
        self.new_mem = z(c, D)
        self.root_dt = z(c)   # time since each root's previous memory update (the commit writes it)
        more = tuple(int(f) for f in more_fanouts)
        self.hop = PaddedHop(cnt=z(c, dt=i32), nbr=z(max(c * k, 1), dt=i32), eid=z(max(c * k, 1), dt=i32),
                             dt=z(max(c * k, 1)), ts=z(max(c * k, 1), dt=i64) if more else None,
                             q_ts=self.root_ts, fanout=k)
        # hops 1.. (sampler.h:393-399): queried from the previous hop's rows,
        # sampled for the step's result (the attention reads hop 0 only)
        self.more_hops: list[PaddedHop] = []
        q, prev = c * k, self.hop
        for li, f in enumerate(more):
            last = li == len(more) - 1
            self.more_hops.append(PaddedHop(
                cnt=z(max(q, 1), dt=i32), nbr=z(max(q * f, 1), dt=i32), eid=z(max(q * f, 1), dt=i32),
                dt=z(max(q * f, 1)), ts=None if last else z(max(q * f, 1), dt=i64), q_ts=prev.ts, fanout=f))
            prev, q = self.more_hops[-1], q * f
        # each sampled edge's row [memory[nbr] | efeat[eid] | cos(w dt + b)]
        # (sgl_edge_rows, then the forward)
        self.X = z(max(c * k * C, 1))
        if not attention:
            return
        # attention saved state and gradients, `passes` blocks of rows
        P = self.passes = int(passes)
        self.Q, self.agg, self.z = z(P * c, D), z(P * c, D), z(P * c, D)
        # rows >= cap of each pass stay zero (row U is read by the predictor's reductions)
        self.y_rows = c + TILE
        self.y = z(P * self.y_rows, D)
        self.qt, self.xbar = z(P * c, H, C), z(P * c, H, C)
        self.score, self.ml, self.stats = z(max(P * c * k * H, 1)), z(P * c, H, 2), z(P * c, 2)
        self.sdrop = z(P * c, H)                      # kept-weight sums of attention dropout
        self.rng_step = z(1, dt=i64)                  # the dropout masks' step (sgl_adam_coef)
        self.phi0 = z(max(dims.T, 1))
        self.S = z(max(c * k * dims.T, 1))   # the sines of the edges' time encodings
        self.gy = z(c, D)
        # per-root sums of the predictor's hidden-layer gradients (+ the
        # non-root-negatives row U): fixed-point accumulators the predictor
        # adds into and the attention backward clears (zero between steps),
        # and their float values for the weight reductions; src, dst (and
        # with dropout the negatives' own rows), one block of cap + 1 rows each
        na = 3 if P > 1 else 2
        self.acc_all, self.g_all = z(na, c + 1, D, dt=i64), z(na, c + 1, D)
        self.acc_src, self.acc_dst = self.acc_all[0], self.acc_all[1]
        self.g_src, self.g_dst = self.g_all[0], self.g_all[1]
        self.acc_neg = self.acc_all[2] if P > 1 else None
        self.g_neg = self.g_all[2] if P > 1 else None
        self.acc_out = z(D + 2, dt=i64)      # the predictor's loss / out_fc accumulator
        self.pred_done = z(_capi.SGL_DONE_WORDS, dt=i32)   # and its completion counter
        self.pos = z(max(B, 1))
        self.neg = z(max(B, 1))
        self.loss = z(1)
        self.gz, self.gagg, self.gQ = z(P * c, D), z(P * c, D), z(P * c, D)
        self.G, self.sigma = z(P * c, H, C), z(P * c, H)
        # per-workgroup partial sums of the attention backward: one tile per
        # workgroup of the instance that runs, conv_rows roots (fp32 and
        # dropout instances) or conv_rows_bf16 (with bf16 weight copies); the
        # arrays hold the tiles of the smaller
        lib = _capi.lib()
        self.conv_rows = int(lib.sgl_conv_backward_tile_rows(D, dims.F, dims.T, H, 0))
        self.conv_rows_bf16 = int(lib.sgl_conv_backward_tile_rows(D, dims.F, dims.T, H, 1))
        if min(self.conv_rows, self.conv_rows_bf16) <= 0 or TILE % self.conv_rows or TILE % self.conv_rows_bf16:
            raise RuntimeError(f"sgl_conv_backward_tile_rows: unsupported attention dimensions {dims}")
        self.proj_part = z(c // TILE, 2, D)   # the time projection's per-tile gradient partials
        self.tiles = c // min(self.conv_rows, self.conv_rows_bf16)
        self.ln_part = z(P * self.tiles, 2, D)
        self.te_part = z(P * self.tiles, 2, max(dims.T, 1))


class Bf16Shadow:
    """bf16 copies of the attention and edge-predictor weights for the bf16
    products of sgl_conv_forward / sgl_conv_backward / sgl_predictor
    (struct sgl_bf16_weights): padded row-major matrices in one zeroed device
    buffer, kept current by the fused update's shadow stores
    (StepParamUpdate) and rebuilt from the fp32 parameters by refresh()
    after the parameters were written otherwise. ``offsets`` maps each
    matrix to its element offset in ``buf``."""

    NAMES = ("wq", "wk", "wv", "wout", "wkt", "wvt", "wot", "ws", "wd", "wst", "wdt")

    def __init__(self, dims: "ConvDims", device: torch.device):
        D, T, H, C = dims.D, dims.T, dims.H, dims.C
        dh = D // H
        r8 = lambda x: _round_up(x, 8)
        self.dims = dims
        self.ld = {"ld_q": r8(D + T), "ld_c": r8(C), "ld_o": r8(2 * D), "hp": r8(dh), "ld_d": r8(D)}
        self.ld["ld_h"] = H * self.ld["hp"]
        L = self.ld
        rows = {"wq": (D, L["ld_q"]), "wk": (D, L["ld_c"]), "wv": (D, L["ld_c"]), "wout": (D, L["ld_o"]),
                "wkt": (C, L["ld_h"]), "wvt": (C, L["ld_h"]), "wot": (D, L["ld_d"]), "ws": (D, L["ld_d"]),
                "wd": (D, L["ld_d"]), "wst": (D, L["ld_d"]), "wdt": (D, L["ld_d"])}
        self.offsets, n = {}, 0
        for name in self.NAMES:
            self.offsets[name] = n
            n += rows[name][0] * rows[name][1]   # ld % 8 == 0: every matrix starts 16-byte aligned
        self.buf = torch.zeros(n, dtype=torch.int16, device=device)
        base = self.buf.data_ptr()
        self.struct = _capi.Bf16Weights(**{k: base + 2 * o for k, o in self.offsets.items()}, **L)
        self.ptr = ctypes.addressof(self.struct)
        self._refresh = None

    def jobs_for(self, which: str, head: int = 0, col0: int = 0) -> dict:
        """The shadow fields of a StepParamUpdate job over a block of a
        shadowed parameter: ``which`` in w_q (columns from col0), w_k / w_v
        (head ``head``'s rows), w_out (columns from col0), w_s, w_d."""
        o, L = self.offsets, self.ld
        dh = self.dims.D // self.dims.H
        if which == "w_q":
            return dict(sh_off=o["wq"] + col0, sh_ld=L["ld_q"])
        if which in ("w_k", "w_v"):
            s = "wk" if which == "w_k" else "wv"
            return dict(sh_off=o[s] + head * dh * L["ld_c"], sh_ld=L["ld_c"], sht_off=o[s + "t"] + head * L["hp"],
                        sht_ld=L["ld_h"])
        if which == "w_out":
            if col0 == 0:
                return dict(sh_off=o["wout"], sh_ld=L["ld_o"], sht_off=o["wot"], sht_ld=L["ld_d"])
            return dict(sh_off=o["wout"] + col0, sh_ld=L["ld_o"])
        if which in ("w_s", "w_d"):
            s = "ws" if which == "w_s" else "wd"
            return dict(sh_off=o[s], sh_ld=L["ld_d"], sht_off=o[s + "t"], sht_ld=L["ld_d"])
        raise ValueError(which)

    def refresh(self, w_q: torch.Tensor, w_k: torch.Tensor, w_v: torch.Tensor, w_out: torch.Tensor,
                w_s: torch.Tensor, w_d: torch.Tensor) -> None:
        """Rebuild every copy from the fp32 parameters (sgl_grad_shadows on
        the current stream)."""
        key = tuple(p.data_ptr() for p in (w_q, w_k, w_v, w_out, w_s, w_d))
        if self._refresh is None or self._refresh[0] != key:
            d = self.dims
            D, T, H, C = d.D, d.T, d.H, d.C
            dh = D // H
            base = min(key)
            jobs, tiles = [], []

            def add(p, rows, cols, ldo, elem0, sh):
                job = _capi.GradJob(off=(p.data_ptr() - base) // 4 + elem0, ldo=ldo, rows=rows, cols=cols, kind=0,
                                    tiles_b=(cols + 15) // 16, tile0=len(tiles), **sh)
                tiles.extend([len(jobs)] * (((rows + 15) // 16) * job.tiles_b))
                jobs.append(job)

            add(w_q, D, D + T, D + T, 0, self.jobs_for("w_q"))
            for h in range(H):
                add(w_k, dh, C, C, h * dh * C, self.jobs_for("w_k", h))
                add(w_v, dh, C, C, h * dh * C, self.jobs_for("w_v", h))
            add(w_out, D, D, 2 * D, 0, self.jobs_for("w_out"))
            add(w_out, D, D, 2 * D, D, self.jobs_for("w_out", col0=D))
            add(w_s, D, D, D, 0, self.jobs_for("w_s"))
            add(w_d, D, D, D, 0, self.jobs_for("w_d"))
            arr = (_capi.GradJob * len(jobs))(*jobs)
            dev = self.buf.device
            raw = torch.frombuffer(bytearray(bytes(arr)), dtype=torch.uint8).to(dev)
            deal = xcd_tile_deal([tiles.count(k) for k in range(len(jobs))])
            self._refresh = (key, raw, torch.as_tensor(deal, dtype=torch.int32, device=dev), len(deal), base)
        _, raw, tiles, nt, base = self._refresh
        _capi.check(_capi.lib().sgl_grad_shadows(raw.data_ptr(), tiles.data_ptr(), nt, base, self.buf.data_ptr(),
                                                 _capi.stream_of(self.buf.device)), "sgl_grad_shadows")


def gru_packed(gru: dict) -> dict:
    """A copy of the GRU operand dict ``gru`` (bf16 weight matrices) with the
    wide-tile kernel's fragment-order copy of its four matrices under
    ``"packed"`` (sgl_gru_pack_bf16); the memory updater module keeps its own."""
    w = gru["w_ih"]
    D = int(gru["w_hh"].shape[1])
    F = int(w.shape[1]) - 2 * D
    pk = torch.empty(int(_capi.lib().sgl_gru_packed_elems(D, F)), dtype=torch.bfloat16, device=w.device)
    P = _capi.ptr
    _capi.check(_capi.lib().sgl_gru_pack_bf16(D, F, P(gru["w_ih"]), P(gru["w_hh"]), P(gru["wc_ih"]),
                                              P(gru["wc_hh"]), P(pk), _capi.stream_of(w.device)),
                "sgl_gru_pack_bf16")
    return dict(gru, packed=pk)


class DeviceStep:
    """The kernel sequence of one step over a NodeState (no host syncs)."""

    def __init__(self, state: NodeState, dims: ConvDims, max_batch: int, attention: bool = True,
                 more_fanouts: tuple[int, ...] = (), passes: int = 1):
        self.state = state
        self.dims = dims
        self.buf = StepBuffers(max_batch, dims, state.device, attention=attention, more_fanouts=more_fanouts,
                               passes=passes)
        self.dev = state.device
        self.lib = _capi.lib()
        # optional per-launch timing: a list that receives (name, start, end)
        # HIP events around each library call, or None
        self.timer: list | None = None
        self.timed: set[str] | None = None   # names to time (None = all)
        # bf16 weight copies for the attention / predictor products (Bf16Shadow), or None: fp32
        self.bf16: Bf16Shadow | None = None

    def _s(self) -> int:
        return _capi.stream_of(self.dev)

    def _bw(self) -> int | None:
        return self.bf16.ptr if self.bf16 is not None else None

    def bwd_tile_rows(self, bf16: bool | None = None) -> int:
        """Roots per ln_part / te_part tile of the attention backward that
        runs: with the bf16 weight copies (``bf16``, default: whether this
        step has them) or the fp32 / dropout instances."""
        use = self.bf16 is not None if bf16 is None else bf16
        return self.buf.conv_rows_bf16 if use else self.buf.conv_rows

    def _call(self, name: str, fn):
        t = self.timer
        if t is None or (self.timed is not None and name not in self.timed):
            return fn()
        # the call's kernel records the events at its own start and end
        # (sgl_time_next_launch), so launch gaps are not counted
        stream = torch.cuda.current_stream(self.dev)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)   # torch creates the HIP events at their first record
        b.record(stream)
        _capi.check(self.lib.sgl_time_next_launch(a.cuda_event, b.cuda_event), "sgl_time_next_launch")
        try:
            r = fn()
        finally:
            self.lib.sgl_time_next_launch(None, None)
        t.append((name, a, b))
        return r

    # -- batch preparation --------------------------------------------------
    def prepare(self, src: torch.Tensor, dst: torch.Tensor, neg: torch.Tensor | None, ts: torch.Tensor,
                n: int | None = None, cursor: torch.Tensor | None = None) -> None:
        """Batch preparation. With ``cursor`` (device int64 [1]) src/dst/neg/ts
        are the whole stream, the batch is its ``n`` events from the cursor,
        buf.batch_start receives the cursor and the cursor advances by n."""
        b, st, P = self.buf, self.state, _capi.ptr
        n = src.numel() if n is None else int(n)
        if n > b.max_batch:
            raise RuntimeError(f"batch of {n} events exceeds the step capacity {b.max_batch}")
        self._call("batch_prepare", lambda: _capi.check(_capi.call("sgl_batch_prepare", 
            st.N, n, P(src), P(dst), P(neg), P(ts), P(cursor), P(b.batch_start) if cursor is not None else None,
            P(st.node_bits), P(st.word_prefix), P(b.num_roots),
            P(b.num_roots64), P(b.ts_max), P(b.t_query), P(b.roots), P(b.root_ts), P(b.ridx_src), P(b.ridx_dst),
            P(b.ridx_neg), P(b.win_src), P(b.win_dst), P(b.cnt_src), P(b.cnt_dst), P(b.any_edges), P(b.err.t),
            self._s()), "sgl_batch_prepare"))

    def prepare_metrics(self, src: torch.Tensor, dst: torch.Tensor, neg: torch.Tensor | None, ts: torch.Tensor,
                        n: int, cursor: torch.Tensor | None, n_prev: int, seq: torch.Tensor, ring: torch.Tensor,
                        work: tuple[torch.Tensor, torch.Tensor]) -> None:
        """prepare() of this batch and, in the same launch, link_metrics() of
        the step these buffers held before (its n_prev events' logits and
        loss, which the preparation does not write): sgl_batch_prepare_metrics."""
        b, st, P = self.buf, self.state, _capi.ptr
        pb = b
        if n > b.max_batch:
            raise RuntimeError(f"batch of {n} events exceeds the step capacity {b.max_batch}")
        self._call("batch_prepare", lambda: _capi.check(_capi.call("sgl_batch_prepare_metrics",
            st.N, n, P(src), P(dst), P(neg), P(ts), P(cursor), P(b.batch_start) if cursor is not None else None,
            P(st.node_bits), P(st.word_prefix), P(b.num_roots),
            P(b.num_roots64), P(b.ts_max), P(b.t_query), P(b.roots), P(b.root_ts), P(b.ridx_src), P(b.ridx_dst),
            P(b.ridx_neg), P(b.win_src), P(b.win_dst), P(b.cnt_src), P(b.cnt_dst), P(b.any_edges), P(b.err.t),
            n_prev, n_prev, P(pb.pos), P(pb.neg), P(pb.loss), P(seq), P(ring), int(ring.shape[0]), None,
            P(work[0]), P(work[1]), self._s()), "sgl_batch_prepare_metrics"))

    def sample(self, sampler: RecentSampler) -> PaddedHop:
        """Hop 0 of the roots at their query time, then every further hop
        from the previous hop's padded rows (its entries' nodes and times,
        masked by its counts); returns hop 0."""
        b = self.buf
        want_ts = b.hop.ts is not None
        hop = self._call("recent_sample", lambda: sampler.sample(b.roots, b.root_ts, self.dims.fanout, out=b.hop,
                                                                  num_live=b.num_roots64, want_ts=want_ts))
        prev = hop
        for h in b.more_hops:
            prev = sampler.sample(prev.nbr[:h.num_queries], prev.ts[:h.num_queries], h.fanout,
                                  want_ts=h.ts is not None, valid_cnt=prev.cnt, stride=prev.fanout, out=h)
        return hop

    # -- memory -------------------------------------------------------------
    def update_memory(self, gru: dict, src, dst, efeat, ts, from_cursor: bool = False) -> None:
        """GRU + mailbox (sgl_memory_update); ``from_cursor``: the event arrays
        span the stream and the batch starts at buf.batch_start."""
        event_offset = self.buf.batch_start if from_cursor else None
        b, st, P = self.buf, self.state, _capi.ptr
        # bf16 weight matrices select the bf16-MFMA entry point
        fn = "sgl_memory_update_bf16" if gru["w_ih"].dtype == torch.bfloat16 else "sgl_memory_update"
        self._call("memory_update", lambda: _capi.check(_capi.call(fn, 
            st.D, st.K, st.F, b.cap, P(b.num_roots), P(b.roots), P(st.memory), P(st.mailbox), P(st.mailbox_ts),
            P(st.next_mail_pos), P(gru["w_ih"]), P(gru["w_hh"]), P(gru["b_ih"]), P(gru["b_hh"]), P(gru["wc_ih"]),
            P(gru["wc_hh"]), P(gru["bc_ih"]), P(gru["bc_hh"]), P(src), P(dst), P(efeat), P(ts), P(event_offset),
            P(b.win_src),
            P(b.win_dst), P(b.cnt_src), P(b.cnt_dst), P(b.new_mem),
            *([P(gru.get("packed"))] if fn == "sgl_memory_update_bf16" else []), self._s()), fn))

    def commit(self) -> None:
        b, st, P = self.buf, self.state, _capi.ptr
        self._call("memory_commit", lambda: _capi.check(_capi.call("sgl_memory_commit", 
            st.D, b.cap, P(b.num_roots), P(b.roots), P(b.new_mem), P(st.memory), P(st.memory_ts), P(b.ts_max),
            P(st.node_bits), P(b.hop.cnt), P(b.any_edges), P(b.root_dt), self._s()), "sgl_memory_commit"))

    def gather_memory(self) -> None:
        """The commit's place without a memory updater: the roots' memory rows
        into new_mem (the attention's root rows), memory left as it is."""
        b, st, P = self.buf, self.state, _capi.ptr
        self._call("memory_gather", lambda: _capi.check(_capi.call("sgl_memory_gather",
            st.D, b.cap, P(b.num_roots), P(b.roots), P(st.memory), P(b.new_mem), P(st.node_bits), P(b.hop.cnt),
            P(b.any_edges), self._s()), "sgl_memory_gather"))

    # -- time projection (config 2's JODIE embedding) ------------------------
    def proj_forward(self, tp) -> torch.Tensor:
        """y = h * (1 + proj(x)) for the live roots (sgl_time_projection_forward);
        ``tp``: the model's TimeProjection."""
        b, P = self.buf, _capi.ptr
        w, bias = tp.proj.weight.detach(), tp.proj.bias.detach()
        self._call("time_projection", lambda: _capi.check(_capi.call(
            "sgl_time_projection_forward", self.dims.D, b.y_rows, P(b.num_roots), P(b.new_mem), P(b.root_dt),
            tp.shift, tp.scale, P(w), P(bias), P(b.y), self._s()), "sgl_time_projection_forward"))
        return b.y

    def proj_backward(self, tp, pred_w: tuple) -> None:
        """The projection's gradient partials from the predictor's per-root
        rows (sgl_time_projection_backward); ``pred_w`` = (src_fc.weight,
        dst_fc.weight)."""
        b, P = self.buf, _capi.ptr
        self._call("time_projection_backward", lambda: _capi.check(_capi.call(
            "sgl_time_projection_backward", self.dims.D, b.cap, P(b.num_roots), P(b.new_mem), P(b.root_dt),
            tp.shift, tp.scale, P(b.acc_src), P(b.acc_dst), P(pred_w[0]), P(pred_w[1]), P(b.g_src), P(b.g_dst),
            P(b.proj_part), self._s()), "sgl_time_projection_backward"))

    # -- attention ----------------------------------------------------------
    def edge_rows(self, efeat_all: torch.Tensor) -> None:
        """The sampled edges' rows X (sgl_edge_rows: the neighbours' memory and
        edge features) from the committed memory table: after commit(), before
        the attention."""
        b, st, d, P = self.buf, self.state, self.dims, _capi.ptr
        hop = b.hop
        self._call("edge_rows", lambda: _capi.check(_capi.call(
            "sgl_edge_rows", d.D, d.F, d.T, d.fanout, b.cap, P(b.num_roots), P(st.memory), P(efeat_all),
            P(hop.cnt), P(hop.nbr), P(hop.eid), P(b.X), self._s()), "sgl_edge_rows"))

    def _at(self, t: torch.Tensor, p: int, rows: int | None = None) -> int:
        """Pointer to pass p's block of a pass-stacked buffer (``rows``: the
        block's element count when it is not the tensor's share)."""
        n = t.numel() // self.buf.passes if rows is None else rows
        return t.data_ptr() + p * n * t.element_size()

    def conv_forward(self, params: list[torch.Tensor], efeat_all: torch.Tensor, drop=None) -> torch.Tensor:
        """The attention forward over the edge rows of the last edge_rows()
        (it adds the rows' time encodings and their sines S). ``drop`` =
        (p_att, p_out, seed): every pass of the buffers with its own dropout
        masks; None: one pass without dropout."""
        b, d, P = self.buf, self.dims, _capi.ptr
        te_w, te_b, w_q, b_q, w_k, b_k, w_v, b_v, w_out, b_out, ln_g, ln_b = params
        pa, po, seed = drop if drop is not None else (0.0, 0.0, 0)
        for p in range(b.passes if drop is not None else 1):
            a = lambda t: self._at(t, p)
            self._call("conv_forward", lambda: _capi.check(_capi.call(
                "sgl_conv_forward", d.D, d.F, d.T, d.H, d.fanout, b.cap, P(b.num_roots), P(b.any_edges),
                P(b.new_mem), P(b.hop.cnt), P(b.X), P(b.hop.dt), P(w_q), P(b_q), P(w_k), P(b_k), P(w_v), P(b_v),
                P(w_out), P(b_out), P(ln_g), P(ln_b), P(te_w), P(te_b), a(b.Q), a(b.qt), a(b.xbar), a(b.score),
                a(b.ml), a(b.agg), a(b.z), a(b.stats), P(b.phi0), P(b.S), self._at(b.y, p, b.y_rows * d.D),
                pa, po, seed, P(b.rng_step), p, a(b.sdrop), self._bw(), self._s()), "sgl_conv_forward"))
        return b.y

    def predictor(self, n: int, train: bool, pred: list[torch.Tensor], out_grads: list[torch.Tensor] | None,
                  passes: int = 1):
        """Edge predictor + BCE over the step's roots (sgl_predictor). ``pred``:
        src_fc.weight, src_fc.bias, dst_fc.weight, dst_fc.bias, out_fc.weight,
        out_fc.bias; ``out_grads``: the out_fc weight / bias gradient buffers
        (overwritten). In training the per-root gradient sums are added into
        the step's fixed-point accumulators, which the attention backward
        (conv_backward_kernel) consumes and clears. ``passes`` 3: src, dst
        and negative rows from the three dropout passes' outputs, the
        negatives' sums in their own rows."""
        b, P = self.buf, _capi.ptr
        g = out_grads if (train and out_grads is not None) else [None, None]
        ys = b.y_rows * self.dims.D if passes > 1 else 0
        acc_neg = P(b.acc_neg) if (train and passes > 1) else None
        self._call("predictor", lambda: _capi.check(_capi.call(
            "sgl_predictor", n, self.dims.D, b.cap, 1 if train else 0, P(b.num_roots), P(b.y), P(b.ridx_src),
            P(b.ridx_dst), P(b.ridx_neg), P(pred[0]), P(pred[1]), P(pred[2]), P(pred[3]), P(pred[4]), P(pred[5]),
            P(b.pos), P(b.neg), P(b.loss), P(b.acc_src) if train else None, P(b.acc_dst) if train else None,
            P(g[0]), P(g[1]), P(b.acc_out), P(b.pred_done), ys, acc_neg, self._bw(), self._s()), "sgl_predictor"))
        return b.pos[:n], b.neg[:n], b.loss

    def link_metrics(self, n: int, seq: torch.Tensor | None, ring: torch.Tensor | None,
                     work: tuple[torch.Tensor, torch.Tensor], out: torch.Tensor | None = None) -> None:
        """The step's (loss, AP, AUC, "mrr") from its n positive and n
        negative logits on the device (sgl_link_metrics): into ``out``
        (float64 [4]) and / or the next slot of ``ring`` (float64 [R, 4],
        slot *seq % R; ``seq`` device int64 [1], incremented). ``work``: the
        partial sums (float64, sgl_link_metrics_work_doubles(n)) and the
        done word (int32 [1], zero)."""
        b, P = self.buf, _capi.ptr
        R = int(ring.shape[0]) if ring is not None else 0
        self._call("link_metrics", lambda: _capi.check(_capi.call(
            "sgl_link_metrics", n, n, P(b.pos), P(b.neg), P(b.loss), P(seq), P(ring), R, P(out), P(work[0]),
            P(work[1]), self._s()), "sgl_link_metrics"))

    def conv_backward_kernel(self, params: list[torch.Tensor], efeat_all: torch.Tensor,
                             gy: torch.Tensor | None = None, pred_w: tuple | None = None, drop=None) -> None:
        """sgl_conv_backward only: per-root gradient rows and per-tile partials
        in the step buffers (the weight gradients are StepParamUpdate's).
        dL/dy is ``gy``, or (gy None) comes from the predictor's per-root rows
        with ``pred_w`` = (src_fc.weight, dst_fc.weight). With ``drop`` (the
        forward's) every pass runs: pass 0 takes dL/dy from the src rows and
        src_fc, pass 1 from the dst rows and dst_fc, pass 2 from the
        negatives' rows and dst_fc."""
        b, d, P = self.buf, self.dims, _capi.ptr
        te_w, te_b, w_q, b_q, w_k, b_k, w_v, b_v, w_out, b_out, ln_g, ln_b = params
        hop = b.hop
        pa, po, seed = drop if drop is not None else (0.0, 0.0, 0)
        passes = b.passes if drop is not None else 1
        if gy is not None:
            gy = gy.contiguous()
        for p in range(passes):
            if gy is not None:
                acc_a = acc_b = g_a = g_b = w_a = w_b = None
            elif passes == 1:
                acc_a, acc_b, g_a, g_b = b.acc_src, b.acc_dst, b.g_src, b.g_dst
                w_a, w_b = pred_w
            else:
                acc_a, g_a, w_a = b.acc_all[p], b.g_all[p], pred_w[0 if p == 0 else 1]
                acc_b = g_b = w_b = None
            a = lambda t: self._at(t, p)
            self._call("conv_backward", lambda: _capi.check(_capi.call(
                "sgl_conv_backward", d.D, d.F, d.T, d.H, d.fanout, b.cap, P(b.num_roots), P(b.any_edges),
                P(hop.cnt), P(b.X), P(b.S), P(hop.dt), P(w_q), P(b_q), P(w_k), P(b_k), P(w_v), P(b_v), P(w_out),
                P(b_out), P(ln_g), P(ln_b), P(te_b), a(b.Q), a(b.qt), a(b.xbar), a(b.score), a(b.ml), a(b.agg),
                a(b.z), a(b.stats), P(gy), P(acc_a), P(acc_b), P(w_a), P(w_b), P(g_a), P(g_b), a(b.gz), a(b.gagg),
                a(b.G), a(b.sigma), a(b.gQ), a(b.ln_part), a(b.te_part), pa, po, seed, P(b.rng_step), p,
                a(b.sdrop), self._bw(), self._s()), "sgl_conv_backward"))

    def conv_backward(self, params: list[torch.Tensor], efeat_all: torch.Tensor, gy: torch.Tensor, drop=None):
        """The backward kernel plus the weight gradients as torch products (the
        autograd path, one pass). Returns the 12 parameter gradients
        (TimeEncode w, b; w_q, b_q, w_k, b_k, w_v, b_v, w_out, b_out, ln
        weight, ln bias)."""
        self.conv_backward_kernel(params, efeat_all, gy, drop=drop)
        b, d = self.buf, self.dims
        te_w, te_b, w_q, b_q, w_k, b_k, w_v, b_v, w_out, b_out, ln_g, ln_b = params
        # weight gradients: per-root products reduced over the live root rows
        # (the kernels leave the rows past them unwritten)
        D, H, C, T = d.D, d.H, d.C, d.T
        dh = D // H
        c = int(b.num_roots.item())
        gz, gagg, gQ, new_mem = b.gz[:c], b.gagg[:c], b.gQ[:c], b.new_mem[:c]
        g_w_out = torch.cat([gz.t() @ b.agg[:c], gz.t() @ new_mem], dim=1)
        g_b_out = gz.sum(0)
        ga = gagg.reshape(c, H, dh).permute(1, 2, 0).contiguous()          # [H, dh, U]
        g_w_v = torch.bmm(ga, b.xbar[:c].permute(1, 0, 2).contiguous()).reshape(D, C)
        if drop is not None and drop[0] > 0:   # the kept weights sum to s_h, not 1
            g_b_v = (gagg.reshape(c, H, dh) * b.sdrop[:c].unsqueeze(-1)).sum(0).reshape(D)
        else:
            g_b_v = gagg.sum(0)
        qh = b.Q[:c].reshape(c, H, dh)
        g_w_k = torch.bmm(qh.permute(1, 2, 0).contiguous(), b.G[:c].permute(1, 0, 2).contiguous()).reshape(D, C)
        g_b_k = (qh * b.sigma[:c].unsqueeze(-1)).sum(0).reshape(D)
        sq = gQ.sum(0)
        phi0 = torch.cos(te_b)
        g_w_q = torch.cat([gQ.t() @ new_mem, torch.outer(sq, phi0)], dim=1)
        g_b_q = sq
        nt = b.cap // self.bwd_tile_rows(self.bf16 is not None and drop is None)
        g_ln_g = b.ln_part[:nt, 0].sum(0)
        g_ln_b = b.ln_part[:nt, 1].sum(0)
        te = b.te_part[:nt, :, :T].sum(0)
        g_te_w = te[0].reshape(T, 1)
        g_te_b = te[1]   # includes the query's cos(b) term (folded in by the kernel)
        return [g_te_w, g_te_b, g_w_q, g_b_q, g_w_k, g_b_k, g_w_v, g_b_v, g_w_out, g_b_out, g_ln_g, g_ln_b]


class StepParamUpdate:
    """Weight gradients of the attention and Adam over the whole model in one
    launch (sgl_grad_adam), preceded by the step-count advance and bias
    corrections (sgl_adam_coef). The job table points at the step buffers and
    at the optimizer's flat buffers, so it is rebuilt when either is
    re-created. The optimizer's three segments are the embedding's first
    parameter, the rest of the embedding (the attention, both gated by the
    step's "block has edges" flag) and the edge predictor, whose out_fc
    takes its gradients from sgl_predictor (Adam-only jobs); each job's
    segment is the one holding its outputs. Each step-buffer set has its own bias
    corrections, so one step's advance may run while the previous step's
    update still reads its own. ``passes`` 3 (dropout): every attention
    gradient sums the three passes' rows, dst_fc's the dst and negative
    passes'; ``counter`` (device int64): the training-step counter the
    advance increments and copies to the buffers' dropout step; ``shadow``
    (Bf16Shadow): the update also stores the bf16 copies of the weights it
    holds."""

    def __init__(self, step: "DeviceStep", opt: "FusedAdam", conv_params: list[torch.Tensor],
                 pred_params: list[torch.Tensor], gates: list[torch.Tensor | None], passes: int = 1,
                 counter: torch.Tensor | None = None, kind: str = "attention", shadow: Bf16Shadow | None = None):
        if len(opt.segments) != 3:
            raise ValueError("StepParamUpdate expects three segments: the embedding's first parameter, the rest "
                             "of the embedding and the predictor")
        if passes not in (1, step.buf.passes):
            raise ValueError(f"StepParamUpdate: {passes} passes on buffers of {step.buf.passes}")
        self.step, self.opt = step, opt
        self.passes = int(passes)
        self.counter = counter
        if kind not in ("attention", "projection"):
            raise ValueError(f"StepParamUpdate: unknown kind {kind!r}")
        self.kind = kind
        if shadow is not None and (kind != "attention" or self.passes != 1):
            raise ValueError("StepParamUpdate: bf16 weight copies need the attention without dropout passes")
        self.shadow = shadow
        self.lib = _capi.lib()
        dev = opt.flat.device
        self.one = torch.ones(1, dtype=torch.float32, device=dev)
        self.coef = torch.zeros(2 * len(opt.segments), dtype=torch.float32, device=dev)
        jobs, tiles = self._jobs(conv_params, pred_params)
        deal = xcd_tile_deal([tiles.count(k) for k in range(len(jobs))])
        # one job copy per workgroup (no tile_job table: one load less at the
        # front of every workgroup's chain)
        arr = (_capi.GradJob * len(deal))(*per_workgroup_jobs(jobs, deal))
        raw = torch.frombuffer(bytearray(bytes(arr)), dtype=torch.uint8)
        self.jobs = raw.to(dev)
        self.num_tiles = len(deal)
        P = _capi.ptr
        self._steps = (ctypes.c_void_p * len(opt.segments))(*[P(seg[2]) for seg in opt.segments])
        if len(gates) != len(opt.segments):
            raise ValueError(f"StepParamUpdate: {len(gates)} gates for {len(opt.segments)} segments")
        self._gates = (ctypes.c_void_p * len(opt.segments))(*[P(g) for g in gates])

    def _jobs(self, conv_params, pred_params):
        b, d, opt = self.step.buf, self.step.dims, self.opt
        D, T, H, C = d.D, d.T, d.H, d.C
        dh = D // H
        ntiles = b.tiles   # a pass's block of the per-tile partials
        tile_rows = self.step.bwd_tile_rows(self.shadow is not None)
        base = opt.flat.data_ptr()

        def off(p):
            o = p.data_ptr() - base
            if o < 0 or o % 4 or p.data_ptr() + 4 * p.numel() > base + 4 * opt.flat.numel():
                raise RuntimeError("StepParamUpdate: parameter outside the optimizer's flat buffer")
            return o // 4

        def at(t, k=0):
            return t.data_ptr() + 4 * k

        jobs, tiles = [], []
        bounds = [(st, st + k) for st, k, _ in opt.segments]

        def seg_of(first, last):   # the segment holding a job's outputs
            for i, (lo, hi) in enumerate(bounds):
                if lo <= first and last < hi:
                    return i
            raise RuntimeError("StepParamUpdate: a job's outputs span optimizer segments")

        def add(job, ntile):
            job.seg = seg_of(job.off, job.off + (job.rows - 1) * job.ldo + job.cols - 1)
            job.tile0 = len(tiles)
            tiles.extend([len(jobs)] * ntile)
            jobs.append(job)

        P = self.passes
        c = b.cap

        sh = self.shadow

        def shf(*a, **k):   # a job's bf16-copy fields (none without a shadow)
            return sh.jobs_for(*a, **k) if sh is not None else {}

        def gemm(x1, s1, x2, s2, o, ldo, rows, cols, r_fixed=-1, r_extra=0, npass=1, ps1=0, ps2=0, shd=None):
            assert s1 >= rows
            tb = (cols + 15) // 16
            add(_capi.GradJob(x1=x1, x2=x2, s1=s1, s2=s2, off=o, ps1=ps1, ps2=ps2, ldo=ldo, rows=rows, cols=cols,
                              kind=0, r_fixed=r_fixed, r_extra=r_extra, tiles_b=tb, npass=npass,
                              **(shd or {})),
                ((rows + 15) // 16) * tb)

        # the attention's reductions run over every pass's rows (rows of
        # width w: pass stride c * w; the per-tile partials: ntiles * w)
        def conv(x1, s1, x2, s2, o, ldo, rows, cols, x1w=None, x2w=None, r_fixed=-1, shd=None):
            gemm(x1, s1, x2, s2, o, ldo, rows, cols, r_fixed=r_fixed, npass=P,
                 ps1=0 if x1w is None else x1w, ps2=0 if x2w is None else x2w, shd=shd)

        one = at(self.one)
        if self.kind == "projection":
            # the time projection's weight [D, 1] and bias [D] from the
            # per-tile partials of sgl_time_projection_backward
            pw, pb = conv_params
            nt = b.cap // TILE
            gemm(at(b.proj_part), 2 * D, one, 0, off(pw), 1, D, 1, nt)
            gemm(at(b.proj_part, D), 2 * D, one, 0, off(pb), 1, D, 1, nt)
            self._pred_jobs(gemm, add, at, off, one, pred_params, 1)
            return self._check(jobs, tiles, conv_params, pred_params)
        te_w, te_b, w_q, b_q, w_k, b_k, w_v, b_v, w_out, b_out, ln_g, ln_b = conv_params
        # per-tile partials: the tiles holding live rows (the others' are zero)
        rt = -tile_rows
        conv(at(b.te_part), 2 * T, one, 0, off(te_w), 1, T, 1, x1w=ntiles * 2 * T, r_fixed=rt)
        conv(at(b.te_part, T), 2 * T, one, 0, off(te_b), 1, T, 1, x1w=ntiles * 2 * T, r_fixed=rt)
        conv(at(b.gQ), D, at(b.new_mem), D, off(w_q), D + T, D, D, x1w=c * D, shd=shf("w_q"))
        conv(at(b.gQ), D, at(b.phi0), 0, off(w_q) + D, D + T, D, T, x1w=c * D, shd=shf("w_q", col0=D))
        conv(at(b.gQ), D, one, 0, off(b_q), 1, D, 1, x1w=c * D)
        for h in range(H):
            conv(at(b.Q, h * dh), D, at(b.G, h * C), H * C, off(w_k) + h * dh * C, C, dh, C, x1w=c * D,
                 x2w=c * H * C, shd=shf("w_k", h))
            conv(at(b.Q, h * dh), D, at(b.sigma, h), H, off(b_k) + h * dh, 1, dh, 1, x1w=c * D, x2w=c * H)
            conv(at(b.gagg, h * dh), D, at(b.xbar, h * C), H * C, off(w_v) + h * dh * C, C, dh, C, x1w=c * D,
                 x2w=c * H * C, shd=shf("w_v", h))
        if P > 1:   # attention dropout: agg_h = W_v xbar'_h + s_h b_v[h]
            for h in range(H):
                conv(at(b.gagg, h * dh), D, at(b.sdrop, h), H, off(b_v) + h * dh, 1, dh, 1, x1w=c * D, x2w=c * H)
        else:
            conv(at(b.gagg), D, one, 0, off(b_v), 1, D, 1, x1w=c * D)
        conv(at(b.gz), D, at(b.agg), D, off(w_out), 2 * D, D, D, x1w=c * D, x2w=c * D, shd=shf("w_out"))
        conv(at(b.gz), D, at(b.new_mem), D, off(w_out) + D, 2 * D, D, D, x1w=c * D, shd=shf("w_out", col0=D))
        conv(at(b.gz), D, one, 0, off(b_out), 1, D, 1, x1w=c * D)
        conv(at(b.ln_part), 2 * D, one, 0, off(ln_g), 1, D, 1, x1w=ntiles * 2 * D, r_fixed=rt)
        conv(at(b.ln_part, D), 2 * D, one, 0, off(ln_b), 1, D, 1, x1w=ntiles * 2 * D, r_fixed=rt)
        # edge predictor: src_fc / dst_fc as reductions over roots 0..U (row U
        # of g_dst holds the non-root negatives; y's row U is zero); out_fc's
        # gradients come from sgl_predictor (Adam only). With dropout dst_fc
        # sums the dst pass's rows and the negatives' pass's rows
        self._pred_jobs(gemm, add, at, off, one, pred_params, P, shf)
        return self._check(jobs, tiles, conv_params, pred_params)

    def _pred_jobs(self, gemm, add, at, off, one, pred_params, P, shf=lambda *a, **k: {}):
        b, D = self.step.buf, self.step.dims.D
        c = b.cap
        w_s, b_s, w_d, b_d, w_o, b_o = pred_params
        nd = 2 if P > 1 else 1
        gs, ys = (c + 1) * D, b.y_rows * D
        yd = at(b.y, ys) if P > 1 else at(b.y)
        gemm(at(b.g_src), D, at(b.y), D, off(w_s), D, D, D, r_extra=1, shd=shf("w_s"))
        gemm(at(b.g_src), D, one, 0, off(b_s), 1, D, 1, r_extra=1)
        gemm(at(b.g_dst), D, yd, D, off(w_d), D, D, D, r_extra=1, npass=nd, ps1=gs, ps2=ys, shd=shf("w_d"))
        gemm(at(b.g_dst), D, one, 0, off(b_d), 1, D, 1, r_extra=1, npass=nd, ps1=gs)
        if off(b_o) != off(w_o) + D:
            raise RuntimeError("StepParamUpdate: out_fc weight and bias are not contiguous in the flat buffer")
        add(_capi.GradJob(x1=None, x2=None, s1=0, s2=0, off=off(w_o), ldo=1, rows=D + 1, cols=1, kind=1,
                          r_fixed=0, tiles_b=1), (D + 1 + 255) // 256)

    def _check(self, jobs, tiles, conv_params, pred_params):
        opt = self.opt
        if sum(p.numel() for p in conv_params) != opt.segments[0][1] + opt.segments[1][1]:
            raise RuntimeError("StepParamUpdate: the embedding segments hold parameters the jobs do not cover")
        if sum(p.numel() for p in pred_params) != opt.segments[2][1]:
            raise RuntimeError("StepParamUpdate: the predictor segment holds parameters the jobs do not cover")
        return jobs, tiles

    def advance(self) -> None:
        """Advance the open segments' step counts and write this step's bias
        corrections (after the step's gates are written)."""
        opt, P, s = self.opt, _capi.ptr, _capi.stream_of(self.opt.flat.device)
        b1, b2 = opt.betas
        _capi.check(_capi.call("sgl_adam_coef", len(opt.segments), self._steps, self._gates, P(self.coef), opt.lr,
                               b1, b2, P(self.counter), P(self.step.buf.rng_step) if self.counter is not None else None,
                               s), "sgl_adam_coef")

    def run(self) -> None:
        """Gradients + Adam with the bias corrections of the last advance()."""
        opt, P, s = self.opt, _capi.ptr, _capi.stream_of(self.opt.flat.device)
        b1, b2 = opt.betas
        self.step._call("param_update", lambda: _capi.check(_capi.call(
            "sgl_grad_adam", P(self.jobs), None, self.num_tiles, P(self.step.buf.num_roots),
            P(opt.flat), P(opt.flat_grad), P(opt.exp_avg), P(opt.exp_avg_sq), len(opt.segments), self._gates,
            P(self.coef), b1, b2, opt.eps, opt.wd, P(self.shadow.buf) if self.shadow is not None else None, s),
            "sgl_grad_adam"))


class ConvFunction(torch.autograd.Function):
    """Autograd node for the attention: forward/backward are the HIP kernels."""

    @staticmethod
    def forward(ctx, step: DeviceStep, efeat_all: torch.Tensor, drop, *params):
        """``drop``: (p_att, p_out, seed) for one dropout pass (pass 0, the
        buffers' current step counter), or None."""
        if drop is not None and step.buf.passes != 1:
            raise RuntimeError("ConvFunction runs one pass; use step buffers made with passes=1")
        ctx.step = step
        ctx.efeat_all = efeat_all
        ctx.params = params
        ctx.drop = drop
        step.edge_rows(efeat_all)
        return step.conv_forward(list(params), efeat_all, drop=drop)

    @staticmethod
    def backward(ctx, gy):
        grads = ctx.step.conv_backward(list(ctx.params), ctx.efeat_all, gy, drop=ctx.drop)
        return (None, None, None, *grads)


class FusedAdam:
    """torch.optim.Adam arithmetic over flat HIP segments. Parameters are
    re-seated as views of one flat buffer and their .grad as views of one flat
    gradient buffer; each segment may carry a device gate (see sgl_adam_step)."""

    def __init__(self, segments: list[list[torch.nn.Parameter]], lr: float = 1e-3,
                 betas=(0.9, 0.999), eps: float = 1e-8, weight_decay: float = 0.0):
        self.lr, self.betas, self.eps, self.wd = float(lr), betas, float(eps), float(weight_decay)
        params = [p for seg in segments for p in seg]
        if not params:
            raise ValueError("FusedAdam: no parameters")
        dev = params[0].device
        n = sum(p.numel() for p in params)
        self.flat = torch.zeros(n, dtype=torch.float32, device=dev)
        self.flat_grad = torch.zeros(n, dtype=torch.float32, device=dev)
        self.exp_avg = torch.zeros(n, dtype=torch.float32, device=dev)
        self.exp_avg_sq = torch.zeros(n, dtype=torch.float32, device=dev)
        self.segments = []
        off = 0
        for seg in segments:
            start = off
            for p in seg:
                k = p.numel()
                self.flat[off:off + k].copy_(p.data.reshape(-1))
                p.data = self.flat[off:off + k].view_as(p)
                p.grad = self.flat_grad[off:off + k].view_as(p)
                off += k
            self.segments.append((start, off - start, torch.zeros(1, dtype=torch.float32, device=dev)))
        self.params = params

    def zero_grad(self, set_to_none: bool = False) -> None:
        self.flat_grad.zero_()

    def step(self, gates: list[torch.Tensor | None] | None = None, only: list[int] | None = None) -> None:
        """``gates[i]``: device int32 gating the i-th stepped segment (None =
        always update); ``only``: the segments to step (default all)."""
        lib, P = _capi.lib(), _capi.ptr
        s = _capi.stream_of(self.flat.device)
        b1, b2 = self.betas
        segs = self.segments if only is None else [self.segments[i] for i in only]
        gates = gates or [None] * len(segs)
        if len(gates) != len(segs):
            raise ValueError(f"FusedAdam.step: {len(gates)} gates for {len(segs)} segments")
        for (start, n, stepc), gate in zip(segs, gates):
            _capi.check(lib.sgl_adam_step(n, P(self.flat[start:start + n]), P(self.flat_grad[start:start + n]),
                                          P(self.exp_avg[start:start + n]), P(self.exp_avg_sq[start:start + n]),
                                          P(stepc), P(gate), self.lr, b1, b2, self.eps, self.wd, s), "sgl_adam_step")
            _capi.check(lib.sgl_adam_advance(P(stepc), P(gate), s), "sgl_adam_advance")

    def state_dict(self) -> dict:
        return {"exp_avg": self.exp_avg.clone(), "exp_avg_sq": self.exp_avg_sq.clone(),
                "steps": [seg[2].clone() for seg in self.segments], "lr": self.lr}

    def load_state_dict(self, sd: dict) -> None:
        self.exp_avg.copy_(sd["exp_avg"])
        self.exp_avg_sq.copy_(sd["exp_avg_sq"])
        for seg, st in zip(self.segments, sd["steps"]):
            seg[2].copy_(st)
