"""CTDG online runtime (backends/ctdg/runtime/runtime.py:39-391 in the reference).

``train_step`` / ``eval_step`` / ``predict_step`` keep the reference's
signatures and result dicts. Inside, a step is the device kernel sequence of
starry_unigraph.native.step over the HBM-resident event stream:

  negatives (CPU generator draws, device lookup; runtime.py:124-136) ->
  sgl_batch_prepare -> sgl_recent_sample (every hop of the split's sampler)
  -> sgl_memory_update (GRU + mailbox) -> sgl_memory_commit -> edge rows ->
  attention forward -> sgl_predictor (edge predictor + BCE) -> attention
  backward -> fused weight gradients + Adam

The reference runs the attention three times per step, once per role (src,
dst, negative) with three dropout masks (runtime.py:193-195). With dropout 0
the three are identical, so the step runs it once and selects rows for the
three roles; with dropout it runs three passes with independent masks (a
counter-based generator, so the backward regenerates them). No host
synchronisation happens inside a step unless ``collect_results`` asks for the
reference's Python-side result dict.
"""
from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Any, Iterable

import torch
import torch.nn.functional as F

from starry_unigraph.lib import _capi
from starry_unigraph.native.step import Bf16Shadow, ConvDims, DeviceStep, FusedAdam, StepParamUpdate

from .data import CTDGDataBatch, TGTemporalDataset
from .memory import CTDGMemoryBank
from .metrics import link_metrics
from .models import CTDGMemoryUpdater
from .negatives import ChunkedDraws, DrawSlot
from .sampler import NativeTemporalSampler


@dataclass
class StepTensors:
    """Device results of one step (no host sync). ``metrics``: the step's
    row of the device metrics ring, (loss, AP, AUC, "mrr") as float64 (None
    without device metrics; final once the step is done, overwritten
    metric_slots steps later)."""
    loss: torch.Tensor
    pos_logits: torch.Tensor
    neg_logits: torch.Tensor
    batch_size: int
    metrics: torch.Tensor | None = None


class CTDGOnlineRuntime:
    kDrawRing = 4   # pinned staging buffers of the negative draws
    kDrawChunkNumbers = 1 << 17   # draws per chunk at most (1 MB of int64 per staging buffer)

    def __init__(self, dataset: TGTemporalDataset, sampler: NativeTemporalSampler, memory: CTDGMemoryBank,
                 model: torch.nn.Module, optimizer, route: Any, device: str, dist_ctx: Any,
                 memory_updater: CTDGMemoryUpdater | None = None, max_batch: int | None = None):
        self.dataset = dataset
        self.sampler = sampler
        self.memory = memory
        self.model = model
        self.optimizer = optimizer
        self.route = route
        self.device = torch.device(device)
        self.dist_ctx = dist_ctx
        self.memory_updater = memory_updater
        self.collect_results = True
        # Full-size batches of a contiguous split run as launch plans per
        # (split, train/eval, step buffer): the step's library calls recorded
        # once and replayed by one host call (sgl_plan_run). Plans read the
        # events at a device-side cursor and the negatives from a stream-wide
        # array, so one recording serves every batch. With a memory updater
        # the next step's front part (batch preparation, sampling, GRU) runs on
        # a second stream beside this step's back part (attention, predictor,
        # backward, Adam); consecutive steps alternate between two sets of
        # step buffers.
        self.use_plans = True
        self._plans: dict[tuple[str, bool, int], tuple] = {}
        # optional per-op timing of planned steps: (entry point name, callable
        # returning this step's (start, end) torch.cuda.Event pair or None)
        self.plan_timer = None
        self._dst_node_pool: torch.Tensor | None = None
        self._neg_queue: dict[str, tuple[torch.Tensor, int]] = {}
        # negatives are drawn inside the step, for neg_chunk consecutive
        # batches of a contiguous split at a time (1: one draw per step; at
        # most kDrawChunkNumbers numbers a chunk, so large batches take fewer),
        # into a ring of kDrawRing pinned staging buffers (the host waits only
        # for the lookup out of a buffer it filled that many draws ago); the
        # schedule keeps the generator where per-step draws would leave it.
        # A chunk boundary costs the host a lookup launch and the next chunk's
        # set-up (≈20-40 us), so longer chunks spread it over more steps
        self.neg_chunk = 32
        self._draws = ChunkedDraws(lambda: self._dst_pool().numel(), self._split_end, self._alloc_draw_slot,
                                   self._lookup, chunk=self.neg_chunk, ring=self.kDrawRing)
        self._pool_dev: torch.Tensor | None = None
        self._split_bounds: dict[str, tuple[int, int]] = {}   # (first event, one past the last) of a split
        self._neg_err = _capi.ErrorFlag(self.device)
        core = self._core()
        conv = core.conv
        fan = int(sampler.fanout[0]) if sampler.fanout else 0
        # the time-projection model (config 2's JODIE) has no attention: its
        # back part is the projection, the predictor and their backward
        self._proj = conv is None
        if self._proj:
            if memory_updater is None:
                raise ValueError("the time-projection embedding needs the memory updater (it embeds updated memory)")
            self.dims = ConvDims(D=memory.hidden_dim, F=max(1, dataset.edge_feat_dim), T=1, H=1, fanout=fan)
        else:
            self.dims = ConvDims(D=memory.hidden_dim, F=conv.dim_edge, T=conv.dim_time, H=conv.num_head, fanout=fan)
        self._make_steps(int(max_batch or 1))
        self._dev = dataset.device_arrays(self.device)
        self._gru = memory_updater.kernel_weights() if memory_updater is not None else None
        # planned steps read events and negatives at a device cursor that the
        # batch preparation advances; _cursor_host mirrors its value (None:
        # unknown) so it is only rewritten when batches are not consecutive
        self._cursor = torch.zeros(1, dtype=torch.int64, device=self.device)
        self._cursor_host: int | None = None
        self._neg_all = torch.zeros(max(int(dataset.src.numel()), 1), dtype=torch.int64, device=self.device)
        self._neg_all_ptr = self._neg_all.data_ptr()
        self._views: dict[tuple[int, int], tuple] = {}
        self._updates: dict[int, StepParamUpdate] = {}
        # two-stream submission: the front stream runs batch preparation,
        # sampling, the GRU, the memory commit and the edge rows; the caller's
        # current stream the attention, predictor, backward and Adam. The
        # streams order themselves through two device words (sgl_plan_run):
        # _sync[0] the number of the last back part (or fence), _sync[16] of
        # the last front part. _seq is the last number used; _need_back what
        # the next front part waits for.
        self._front_stream: torch.cuda.Stream | None = None
        self._sync = torch.zeros(64, dtype=torch.int32, device=self.device)
        self._sync_ptr = self._sync.data_ptr()
        self._sync_back = self._sync[0:1]
        self._seq = 0
        self._need_back = self._prev_seq = 0
        self._state_writes = memory.state.writes
        # training steps so far (the dropout masks' step; sgl_adam_coef advances it)
        self._rng_counter = torch.zeros(1, dtype=torch.int64, device=self.device)
        # every step's (loss, AP, AUC, "mrr") (runtime.py:202-214, 314-328) computed
        # on the device (sgl_link_metrics) into a ring of metric_slots rows in
        # step order; _metrics_issued counts the steps submitted (the host's
        # copy of the ring's device counter). Eager steps and steps whose
        # results the host collects compute them at the end of their back part;
        # in the asynchronous planned mode a step's metrics are computed by the
        # front part of the next step on the same buffers (off the critical
        # back stream; the logits stay until that step's back part), and
        # _metrics_pending[q] holds the batch size of such a step on buffer set
        # q (_metrics_order: the sets in step order), flushed whenever the
        # ring is read
        self.device_metrics = True
        self._metrics_pending: list[int] = [0, 0]
        self._metrics_order: list[int] = []
        self.metric_slots = 8192
        self.metrics_ring = torch.full((self.metric_slots, 4), float("nan"), dtype=torch.float64,
                                       device=self.device)
        self._metrics_seq = torch.zeros(1, dtype=torch.int64, device=self.device)
        self._metrics_issued = 0
        self._metric_rows = self.metrics_ring.unbind(0)   # a view per slot (no tensor op per step)
        # the kernel's per-workgroup partial sums and completion word (shared
        # by the step buffer sets: the back parts are stream-ordered)
        self._metrics_work = (
            torch.zeros(int(_capi.lib().sgl_link_metrics_work_doubles(_capi.SGL_LINK_METRICS_MAX_SCORES // 2)),
                        dtype=torch.float64, device=self.device),
            torch.zeros(1, dtype=torch.int32, device=self.device))
        # bf16 copies of the attention / predictor weights when the conv runs
        # its products in bf16 (the fused update keeps them current; dirty:
        # rebuild from the parameters before the next step)
        self._bf16: Bf16Shadow | None = None
        self._bf16_dirty = True
        self._bf16_ver: tuple = ()
        self._back_metrics = False

    def _make_steps(self, max_batch: int) -> None:
        # every hop of the sampler (history layers, sampler.py:76-90) is
        # sampled; the attention reads hop 0 (runtime.py:164-167)
        if getattr(self, "steps", None):
            self._flush_metrics()   # their logits are about to be dropped
        hops = [int(f) for f in self.sampler.fanout[:max(1, int(self.sampler.history))]]
        if len(hops) < int(self.sampler.history):
            raise RuntimeError(f"ParallelSampler: num_layers {self.sampler.history} > len(fanouts) {len(hops)}")
        self._passes = self._dropout_passes()
        self.steps = [DeviceStep(self.memory.state, self.dims, max_batch, more_fanouts=tuple(hops[1:]),
                                 passes=self._passes) for _ in range(2)]
        self._parity = 0
        self.step = self.steps[0]   # the step buffers of the latest step

    def _conv_mods(self) -> tuple:
        """(core model, its conv or None, the conv's two dropout modules),
        cached per core model (nn.Module attribute lookups cost microseconds
        on every step)."""
        core = self._core()
        c = self.__dict__.get("_conv_mods_of")
        if c is None or c[0] is not core:
            conv = getattr(core, "conv", None)
            c = self._conv_mods_of = (core, conv, conv.dropout if conv is not None else None,
                                      conv.att_dropout if conv is not None else None)
        return c

    def _dropout_passes(self) -> int:
        """3 attention passes per training step when a dropout is on
        (runtime.py:193-195), else 1."""
        _, conv, d, ad = self._conv_mods()
        return 3 if (conv is not None and (d.p > 0 or ad.p > 0)) else 1

    def fence(self) -> None:
        """Order the next step after all work queued so far on the current
        stream. With ``collect_results`` False consecutive steps overlap, and
        a caller that writes state the step reads (memory, mailbox, GRU
        weights, event arrays) with tensor code between steps calls this
        before the next step; the memory bank's own writers are tracked
        without it. With ``collect_results`` every step is fenced."""
        if self._front_stream is not None:
            self._seq += 1
            # on the current stream, after the work queued so far
            self._sync_back.fill_(self._seq)
            self._need_back = self._prev_seq = self._seq
        self._state_writes = self.memory.state.writes

    def check_sync(self) -> None:
        """Raise if a cross-stream wait of a planned step gave up (after about
        two seconds) instead of seeing its predecessor finish (results from
        then on are unordered), if a batch preparation flagged its input (a
        node id out of range, a node bitmap left set), or if the edge predictor met a gradient or loss
        term outside the range of its fixed-point sums (clamped: the sums since
        the last check are wrong). Synchronizes the device."""
        if self._front_stream is not None and int(self._sync[48].item()):
            raise RuntimeError("sgl_plan_run: a cross-stream wait timed out; the steps since the last check "
                               "ran out of order")
        self._neg_err.raise_if_set("negative sampling (a draw outside the dst pool)")
        for st in self.steps:
            st.buf.err.raise_if_set("sgl_batch_prepare")
        for st in self.steps:
            flag = st.buf.pred_done[_capi.SGL_DONE_RANGE_WORD]
            if int(flag.item()):
                flag.zero_()
                raise RuntimeError("sgl_predictor: a gradient or loss term outside the fixed-point range "
                                   "(|v| >= 2^23 or NaN) was clamped; the loss and gradients since the last "
                                   "check are wrong")

    def _pipeline_streams(self):
        if self._front_stream is None:
            self._front_stream = torch.cuda.Stream(self.device)
            self.fence()
        elif self._seq >= 0x7FFFFFF0:   # keep the sequence numbers in int32 range
            torch.cuda.synchronize(self.device)
            self._sync.zero_()
            self._seq = self._need_back = self._prev_seq = 0
        return self._front_stream

    def _core(self):
        # (hasattr on an nn.Module without the attribute raises and catches
        # inside __getattr__: cached per model object)
        m = self.model
        c = self.__dict__.get("_core_of")
        if c is None or c[0] is not m:
            c = self._core_of = (m, m.module if hasattr(m, "module") else m)
        return c[1]

    # ------------------------------------------------------------- batching
    def iter_batches(self, split: str, batch_size: int) -> Iterable[CTDGDataBatch]:
        yield from self.dataset.iter_batches(split=split, batch_size=batch_size)

    def _dst_pool(self) -> torch.Tensor:
        if self._dst_node_pool is None:
            self._dst_node_pool = self.dataset.dst.unique()
        return self._dst_node_pool

    def _negative_sample(self, batch: CTDGDataBatch) -> torch.Tensor:
        """runtime.py:124-136: uniform over the sorted unique dst pool (global CPU
        generator), collisions with the true dst bumped to the next pool entry."""
        pool = self._dst_pool()
        self._draws.release()   # the generator where the steps so far left it
        idx = torch.randint(low=0, high=pool.numel(), size=batch.dst.shape, dtype=torch.long)
        neg = pool[idx]
        col = neg.eq(batch.dst.cpu())
        if col.any():
            idx[col] = (idx[col] + 1) % pool.numel()
            neg = pool[idx]
        return neg

    def precompute_negatives(self, split: str, batch_size: int) -> None:
        """Draw the negatives of every batch of ``split`` in one call and keep them
        in HBM. torch.randint on the CPU generator yields the same numbers in one
        call as in per-batch calls, so this equals per-step sampling."""
        pool = self._dst_pool()
        ids = self.dataset.split_event_ids(split)
        self._draws.release()
        idx = torch.randint(low=0, high=pool.numel(), size=(ids.numel(),), dtype=torch.long)
        dst = self.dataset.dst[ids]
        neg = pool[idx]
        col = neg.eq(dst)
        if col.any():
            idx[col] = (idx[col] + 1) % pool.numel()
            neg = pool[idx]
        lo = int(ids[0]) if ids.numel() else 0
        if ids.numel() and int(ids[-1]) - lo + 1 == ids.numel():   # contiguous split: in place
            view = self._neg_all[lo:lo + ids.numel()]
            view.copy_(neg)
            self._neg_queue[split] = (view, 0)
        else:
            self._neg_queue[split] = (neg.to(self.device), 0)
        self.fence()   # the next batch preparation reads them

    def _negatives(self, batch: CTDGDataBatch) -> torch.Tensor:
        """The batch's negatives, ready for work on the current stream."""
        buf, off = self._negatives_at(batch)
        if self._front_stream is not None:   # drawn on the front stream
            torch.cuda.current_stream(self.device).wait_stream(self._front_stream)
        return buf[off:off + batch.size] if off >= 0 else buf

    def _negatives_at(self, batch: CTDGDataBatch) -> tuple[torch.Tensor, int]:
        """(buffer, offset) of the batch's negatives (offset -1: the buffer is
        exactly the batch's negatives); consumes the split's precomputed queue,
        else the negatives drawn ahead for consecutive batches."""
        q = self._neg_queue.get(batch.split)
        if q is not None:
            buf, off = q
            n = batch.size
            if off + n <= buf.numel():
                self._neg_queue[batch.split] = (buf, off + n)
                return buf, off
            del self._neg_queue[batch.split]
        s, n = batch.start, batch.size
        if s >= 0 and self.neg_chunk > 1:
            self._draws.chunk = max(1, min(self.neg_chunk, self.kDrawChunkNumbers // max(n, 1)))
            self._draws.serve(batch.split, s, n)
            return self._neg_all, s
        return self._negative_sample(batch).to(self.device, non_blocking=True), -1

    def _split_end(self, split: str, s: int, n: int) -> int:
        """One past the last event of the contiguous split holding batch
        [s, s + n) (s + n when the batch lies outside it)."""
        key = "test" if split == "predict" else split
        b = self._split_bounds.get(key)
        if b is None:
            ids = self.dataset.split_event_ids(key)
            b = self._split_bounds[key] = (int(ids[0]), int(ids[-1]) + 1) if ids.numel() else (0, 0)
        return b[1] if b[0] <= s < b[1] else s + n

    def _alloc_draw_slot(self, m: int) -> DrawSlot:
        """A pinned staging buffer for at least m draws (a chunk of batches),
        read in place by the device lookup through its device-visible
        address."""
        buf = torch.empty(max(m, 1), dtype=torch.long, pin_memory=True)
        done = torch.cuda.Event()
        done.record(torch.cuda.current_stream(self.device))   # created now, not on a later step
        return DrawSlot(buf, done, _capi.host_device_pointer(buf))

    def _lookup(self, slot: DrawSlot, s: int, m: int) -> None:
        """The pool lookup and collision rule of the m draws in a ring
        buffer for events [s, s + m) (sgl_negatives_from_draws, in place in
        the stream-wide array)."""
        if self._pool_dev is None:
            self._pool_dev = self._dst_pool().to(self.device)
            for t in (self._dev["dst"], self._neg_all):
                if t.dtype != torch.int64 or not t.is_contiguous():
                    raise RuntimeError("negatives lookup: the dst and negative arrays must be contiguous int64")
        front = self._front_stream
        stream = front if front is not None else torch.cuda.current_stream(self.device)
        # on the front stream, where the batch preparations read them (an
        # eager step orders its stream after the front stream first); the
        # lookup reads the pinned draws in place (no separate copy). The
        # launch and the event take the stream explicitly, and the int64
        # arrays' pointers are offset directly (a draw boundary's host time
        # counts in short runs)
        P = _capi.ptr
        dst, out = self._dev["dst"], self._neg_all
        _capi.check(_capi.call("sgl_negatives_from_draws", m, slot.addr, P(self._pool_dev), self._pool_dev.numel(),
                               dst.data_ptr() + 8 * s, out.data_ptr() + 8 * s, P(self._neg_err.t), stream.cuda_stream),
                    "sgl_negatives_from_draws")
        if slot.done is None:
            slot.done = torch.cuda.Event()
        slot.done.record(stream)

    def _device_batch(self, batch: CTDGDataBatch):
        d = self._dev
        s = batch.start
        n = batch.size
        if s >= 0:
            return (d["src"][s:s + n], d["dst"][s:s + n], d["ts"][s:s + n], d["edge_feat"][s:s + n])
        ev = batch.event_ids.to(self.device)
        return d["src"][ev], d["dst"][ev], d["ts"][ev], d["edge_feat"][ev].contiguous()

    # ------------------------------------------------------------- the step
    def params_changed(self) -> None:
        """Parameters were written outside the fused update in a way their
        version counters do not show (through ``.data``, or by a kernel):
        rebuild the bf16 weight copies before the next step. Writes through
        torch (``load_state_dict``, ``nn.init``, in-place ops under
        ``no_grad``) are detected without it."""
        self._bf16_dirty = True

    def _bf16_sync(self) -> None:
        """With bf16 attention products: the weight copies exist, every step
        buffer set uses them and they match the parameters (rebuilt on the
        current stream when marked dirty or when a shadowed weight's storage
        or version counter changed: torch writes bump the counter, the fused
        update's own stores keep the copies current and do not)."""
        core, conv, _, _ = self._conv_mods()
        if conv is None or conv.gemm_dtype != "bf16":
            return
        if self._bf16 is None:
            self._bf16 = Bf16Shadow(self.dims, self.device)
            # the fused updates are rebuilt with the copies' stores (and the
            # plans that point at their job tables dropped first)
            self.reset_plans()
            self._updates.clear()
            self._bf16_dirty = True
        for st in self.steps:
            st.bf16 = self._bf16
        c = self.__dict__.get("_shadowed_of")
        if c is None or c[0] is not core:   # nn.Module attribute lookups cost microseconds: once per model
            c = self._shadowed_of = (core, (conv.w_q.weight, conv.w_k.weight, conv.w_v.weight, conv.w_out.weight,
                                            core.src_fc.weight, core.dst_fc.weight))
        ws = c[1]
        ver = tuple([(w.data_ptr(), w._version) for w in ws])
        if self._bf16_dirty or ver != self._bf16_ver:
            self._bf16.refresh(*ws)
            self._bf16_dirty = False
            self._bf16_ver = ver

    def _forward(self, batch: CTDGDataBatch, split: str, train: bool) -> StepTensors:
        n = batch.size
        if n > self.steps[0].buf.max_batch or self._dropout_passes() != self._passes:
            self._make_steps(max(n, self.steps[0].buf.max_batch))
            self.reset_plans()
        self._bf16_sync()
        q = self._parity
        self._parity = q ^ 1
        step = self.steps[q]
        self.step = step
        buf, off = self._negatives_at(batch)
        b = step.buf
        start = batch.start
        with_metrics = self.device_metrics and 0 < 2 * n <= _capi.SGL_LINK_METRICS_MAX_SCORES
        planned = self.use_plans and n == b.max_batch and start >= 0 and step.timer is None
        # metrics at the end of the back part, or deferred to the next front part on these buffers
        defer = planned and not self.collect_results
        if not defer:
            self._flush_metrics()   # ring rows in step order
        self._back_metrics = with_metrics and not defer
        if not planned:
            if self._front_stream is not None:   # negatives drawn on the front stream
                torch.cuda.current_stream(self.device).wait_stream(self._front_stream)
            src, dst, ts, ef = self._device_batch(batch)
            self._front_body(step, split, n, src, dst, buf[off:off + n] if off >= 0 else buf, ts, ef, None)
            self._commit_body(step, train)
            self._back_body(step, train, n)
            self.fence()
        else:
            # the negatives must sit at the batch's place in the stream-wide array
            if off < 0 or buf.data_ptr() + 8 * off != self._neg_all_ptr + 8 * start:
                self._neg_all[start:start + n].copy_(buf[off:off + n] if off >= 0 else buf)
                self.fence()
            if self._cursor_host != start:
                self._cursor.fill_(start)
                self.fence()
            self._cursor_host = start + n
            # overlap across steps only in the asynchronous mode: a caller
            # that reads each step's results on the host may also write state
            # between steps, so its steps start after everything queued before
            if self.collect_results or self._state_writes != self.memory.state.writes:
                self.fence()
            front_metrics = self._metrics_pending[q] if defer else 0
            key = ("test" if split == "predict" else split, bool(train), q, self._back_metrics, front_metrics)
            plan = self._plans.get(key)
            if plan is None:
                plan = self._record(step, split, train, n, front_metrics)
                self._plans[key] = plan
                self.fence()   # state built on first use (a split's sampler graph) is queued here
            front = self._pipeline_streams()
            seq = self._seq + 1
            top, t0, t1 = -1, None, None
            if self.plan_timer is not None:   # (entry point name, callback giving this step's event pair or None)
                evs = self.plan_timer[1]()
                if evs is not None:
                    top = plan[3].index(self.plan_timer[0])
                    t0, t1 = evs[0].cuda_event, evs[1].cuda_event
            _capi.check(_capi.lib().sgl_plan_run(
                plan[0], plan[1], plan[2], front.cuda_stream, _capi.stream_of(self.device),
                self._sync_ptr, seq, self._need_back, top, t0, t1), "sgl_plan_run")
            # the next step's front part refills the buffers this step's
            # predecessor read; its commit follows this step's backward
            self._need_back, self._prev_seq = self._prev_seq, seq
            self._seq = seq
            if defer:
                if front_metrics:
                    self._metrics_order.remove(q)
                self._metrics_pending[q] = n if with_metrics else 0
                if with_metrics:
                    self._metrics_order.append(q)
        views = self._views.get((n, q))
        if views is None or views[0] is not b:
            views = (b, b.loss[0], b.pos[:n], b.neg[:n])
            self._views[(n, q)] = views
        met = None
        if with_metrics:
            met = self._metric_rows[self._metrics_issued % self.metric_slots]
            self._metrics_issued += 1
        return StepTensors(views[1], views[2], views[3], n, met)

    def _record(self, step: DeviceStep, split: str, train: bool, n: int, front_metrics: int = 0) -> tuple:
        """Record a full step on ``step``'s buffers as a launch plan: (ops,
        #front, #back, entry point names, recorded calls). The front part is
        the batch preparation, sampling, GRU, memory commit, edge rows and (in
        training) the Adam step counts; the back part the attention, the
        predictor and, in training, the backward and the fused update. No back
        part reads the memory table, so a step's front part may run beside
        the previous step's back part."""
        d = self._dev
        if train:
            self._param_update(step)   # any rebuild or host-side sync happens outside the recording
        with _capi.record() as front:
            self._front_body(step, split, n, d["src"], d["dst"], self._neg_all, d["ts"], d["edge_feat"],
                             self._cursor, front_metrics)
            self._commit_body(step, train)
        with _capi.record() as back:
            self._back_body(step, train, n)
        # the front part runs beside the previous step's update: it must not
        # read the trained parameters (every pointer argument outside them)
        inner = getattr(self.optimizer, "inner", None)
        if isinstance(inner, FusedAdam):
            lo = inner.flat.data_ptr()
            hi = lo + 4 * inner.flat.numel()
            for name, args in front:
                if any(isinstance(a, int) and lo <= a < hi for a in args):
                    raise RuntimeError(f"launch plan: {name} in the front part reads the trained parameters")
        calls = front + back
        return (_capi.pack_ops(calls), len(front), len(back), [c[0] for c in calls], calls)

    def reset_plans(self) -> None:
        """Drop recorded plans (after buffers they reference change)."""
        if self._front_stream is not None:
            torch.cuda.current_stream(self.device).wait_stream(self._front_stream)
        self._plans.clear()

    def _front_body(self, step: DeviceStep, split: str, n: int, src, dst, neg, ts, ef, cursor,
                    prev_metrics: int = 0) -> None:
        """Batch preparation, sampling and the GRU memory update of one step.
        With ``cursor`` (device int64 [1]) the event and negative arrays are
        the whole stream and the batch starts at the cursor (which the step
        advances). ``prev_metrics`` > 0: first the metrics of the previous
        step on these buffers (that many events), whose back part the
        preparation's wait has seen finish."""
        if prev_metrics:   # one launch (the metrics' workgroups beside the preparation's)
            step.prepare_metrics(src, dst, neg, ts, n, cursor, prev_metrics, self._metrics_seq, self.metrics_ring,
                                 self._metrics_work)
        else:
            step.prepare(src, dst, neg, ts, n=n, cursor=cursor)
        step.sample(self.sampler.device_sampler("test" if split == "predict" else split))
        if self._gru is not None:
            step.update_memory(self._gru, src, dst, ef, ts, from_cursor=cursor is not None)

    def _commit_body(self, step: DeviceStep, train: bool) -> None:
        """The memory commit (which also sets the step's "block has edges"
        gate), the sampled edges' rows from the committed memory (no trained
        parameter is read, so this may run beside the previous step's update)
        and, in training, the Adam step-count advance and bias corrections
        that the step's fused update reads."""
        if self._gru is not None:
            step.commit()
        else:   # runtime.py:283-285: the conv reads the memory as it is
            step.gather_memory()
        if not self._proj:
            step.edge_rows(self._dev["edge_feat"])
        if train:
            self._param_update(step).advance()

    def _back_body(self, step: DeviceStep, train: bool, n: int) -> None:
        """Attention forward, edge predictor + BCE and, in training, the
        backward and the fused weight-gradient + Adam update."""
        core = self._core()
        conv = core.conv
        efeat_all = self._dev["edge_feat"]
        pparams = [core.src_fc.weight, core.src_fc.bias, core.dst_fc.weight, core.dst_fc.bias, core.out_fc.weight,
                   core.out_fc.bias]
        if self._proj:
            tp = core.time_proj
            pdet = [p.detach() for p in pparams]
            upd = self._param_update(step) if train else None
            step.proj_forward(tp)
            step.predictor(n, train, pdet, [core.out_fc.weight.grad, core.out_fc.bias.grad] if train else None)
            if train:
                step.proj_backward(tp, (pdet[0], pdet[2]))
                upd.run()
            self._metrics_op(step, n)
            return
        cparams = [p.detach() for p in conv.kernel_params()]
        if train:
            # gradients are views of the optimizer's flat buffer (no torch
            # autograd on this path): sgl_predictor writes out_fc's, the fused
            # update every other parameter's
            upd = self._param_update(step)
            out_grads = [core.out_fc.weight.grad, core.out_fc.bias.grad]
        else:
            out_grads = None
        pdet = [p.detach() for p in pparams]
        drop = conv.drop_args() if train else None
        passes = step.buf.passes if drop is not None else 1
        step.conv_forward(cparams, efeat_all, drop=drop)
        step.predictor(n, train, pdet, out_grads, passes=passes)
        if train:
            step.conv_backward_kernel(cparams, efeat_all, pred_w=(pdet[0], pdet[2]), drop=drop)
            upd.run()
        self._metrics_op(step, n)

    def _metrics_op(self, step: DeviceStep, n: int) -> None:
        """The step's metrics into the next ring slot as the last op of its
        back part (the loss and logits are final there), unless they are
        deferred to the next front part on these buffers (_forward decides)."""
        if self._back_metrics:
            step.link_metrics(n, self._metrics_seq, self.metrics_ring, self._metrics_work)

    def _flush_metrics(self) -> None:
        """Compute the deferred metrics of planned steps now, on the current
        stream in step order (their logits are intact until the next back
        part on their buffers, which is issued after this)."""
        if not self._metrics_order:
            return
        if self._front_stream is not None:
            torch.cuda.current_stream(self.device).wait_stream(self._front_stream)
        for q in self._metrics_order:
            self.steps[q].link_metrics(self._metrics_pending[q], self._metrics_seq, self.metrics_ring,
                                       self._metrics_work)
            self._metrics_pending[q] = 0
        self._metrics_order.clear()

    def metrics_of_last_steps(self, count: int) -> torch.Tensor:
        """(loss, AP, AUC, "mrr") of the last ``count`` steps submitted, one row
        each in step order, from the device ring (float64 [count, 4]; rows of
        steps without device metrics are NaN). Synchronizes the device."""
        self._flush_metrics()
        count = min(int(count), self._metrics_issued, self.metric_slots)
        if self._front_stream is not None:
            torch.cuda.current_stream(self.device).wait_stream(self._front_stream)
        torch.cuda.synchronize(self.device)
        end = int(self._metrics_seq.item())
        idx = torch.arange(end - count, end, device=self.device) % self.metric_slots
        return self.metrics_ring[idx].cpu()

    def _param_update(self, step: DeviceStep) -> StepParamUpdate:
        """The fused weight-gradient + Adam launch for a step's buffers and the
        runtime's optimizer (rebuilt if either changed)."""
        inner = getattr(self.optimizer, "inner", None)
        if not isinstance(inner, FusedAdam):
            raise RuntimeError("the fused step needs the runtime's optimizer (GatedAdam over a FusedAdam)")
        upd = self._updates.get(id(step))
        if upd is None or upd.step is not step or upd.opt is not inner:
            core = self._core()
            pred = [core.src_fc.weight, core.src_fc.bias, core.dst_fc.weight, core.dst_fc.bias, core.out_fc.weight,
                    core.out_fc.bias]
            if self._proj:
                tp = core.time_proj.proj
                upd = StepParamUpdate(step, inner, [tp.weight, tp.bias], pred, [None, None, None],
                                      kind="projection")
            else:
                ae = step.buf.any_edges
                upd = StepParamUpdate(step, inner, core.conv.kernel_params(), pred, [ae, ae, None],
                                      passes=step.buf.passes, counter=self._rng_counter, shadow=self._bf16)
            self._updates = {k: u for k, u in self._updates.items() if u.step in self.steps}
            self._updates[id(step)] = upd
        return upd

    def _metric_dict(self, st: StepTensors) -> dict[str, float]:
        """runtime.py:202-214 (AP, AUC and the pairwise "mrr"): the step's row
        of the device metrics ring (sgl_link_metrics), else computed on the
        logits' device (metrics.link_metrics)."""
        if st.metrics is not None:
            self._flush_metrics()
            _, ap, auc, mrr = st.metrics.tolist()
            return {"ap": ap, "auc": auc, "mrr": mrr}
        return link_metrics(st.pos_logits, st.neg_logits)

    def _sample_meta(self, n: int) -> dict[str, int]:
        """CTDGSampleOutput.describe() (sampler.py:27-33, sampler.py:119-120):
        roots, |unique(roots and every hop's nodes)|, |unique(every hop's
        edge ids)|, the number of hops."""
        b = self.step.buf
        u = int(b.num_roots.item())
        nodes, eids = [b.roots[:u]], []
        q = u
        for hop in [b.hop] + b.more_hops:
            k = hop.fanout
            cnt = hop.cnt[:q]
            if k > 0 and q > 0:
                valid = torch.arange(k, device=cnt.device).unsqueeze(0) < cnt.unsqueeze(1)
                nodes.append(hop.nbr[:q * k].view(q, k)[valid].long())
                eids.append(hop.eid[:q * k].view(q, k)[valid].long())
            q *= k
        return {"root_count": u, "sampled_node_count": int(torch.unique(torch.cat(nodes)).numel()),
                "sampled_edge_count": int(torch.unique(torch.cat(eids)).numel()) if eids else 0,
                "num_layers": 1 + len(b.more_hops)}

    def _empty_result(self, batch: CTDGDataBatch, split: str) -> dict[str, Any]:
        return {"loss": 0.0, "predictions": [], "targets": [],
                "meta": {"split": split, "batch_size": 0, "metrics": {}, "memory": self.memory.describe(),
                         "empty_batch": True}}

    def train_step(self, batch: CTDGDataBatch) -> dict[str, Any]:
        if not self.model.training:   # Module.train() walks every submodule
            self.model.train()
        t0 = time.perf_counter()
        if batch.is_empty:
            # runtime.py:248-258: a zero loss's backward and an optimizer
            # step (the model's first parameter alone has a gradient); on the
            # stream of the back parts, after the previous step's update
            inner = getattr(self.optimizer, "inner", None)
            if not isinstance(inner, FusedAdam):
                raise RuntimeError("the fused step needs the runtime's optimizer (GatedAdam over a FusedAdam)")
            self.optimizer.empty_step()
            r = self._empty_result(batch, batch.split)
            r["meta"].update(sync_wait_ms=0.0, sync_submit_ms=0.0, step_ms=(time.perf_counter() - t0) * 1000.0)
            return r
        st = self._forward(batch, batch.split, train=True)
        if not self.collect_results:
            return {"loss": st.loss, "pos_logits": st.pos_logits, "neg_logits": st.neg_logits,
                    "metrics": st.metrics, "meta": {"split": batch.split, "batch_size": st.batch_size}}
        step_ms = (time.perf_counter() - t0) * 1000.0
        return {"loss": float(st.loss.item()), "predictions": torch.sigmoid(st.pos_logits).cpu().tolist(),
                "targets": [1] * batch.size,
                "meta": {"split": batch.split, "batch_size": batch.size, "sample": self._sample_meta(batch.size),
                         "metrics": self._metric_dict(st),
                         "memory": self.memory.describe(), "sync_wait_ms": 0.0, "sync_submit_ms": 0.0,
                         "step_ms": step_ms}}

    def eval_step(self, batch: CTDGDataBatch, split: str) -> dict[str, Any]:
        """runtime.py:330-386: no grad, memory and mailbox still updated."""
        if self.model.training:
            self.model.eval()
        if batch.is_empty:
            return self._empty_result(batch, split)
        with torch.no_grad():
            st = self._forward(batch, split, train=False)
        if not self.collect_results:
            return {"loss": st.loss, "pos_logits": st.pos_logits, "neg_logits": st.neg_logits,
                    "metrics": st.metrics, "meta": {"split": split, "batch_size": st.batch_size}}
        return {"loss": float(st.loss.item()), "predictions": torch.sigmoid(st.pos_logits).cpu().tolist(),
                "targets": [1] * batch.size,
                "meta": {"split": split, "batch_size": batch.size,
                         "metrics": self._metric_dict(st),
                         "memory": self.memory.describe()}}

    def predict_step(self, batch: CTDGDataBatch) -> dict[str, Any]:
        r = self.eval_step(batch, split=batch.split)
        r["meta"]["predict"] = True
        return r
