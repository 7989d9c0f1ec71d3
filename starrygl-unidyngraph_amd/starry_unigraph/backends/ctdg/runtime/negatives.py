"""Host-side schedule of the negatives' CPU draws (runtime.py:124-136 in the
reference: one ``torch.randint(0, len(pool), (B,))`` on the global CPU
generator per step, then a pool lookup and a collision bump).

The runtime draws the numbers of several consecutive batches of a split in
one call (torch.randint on one generator yields the same numbers in one call
as in consecutive calls) into pinned staging buffers, and a device kernel
does the pool lookup in place. To keep no step waiting for a whole chunk,
the next chunk's numbers are drawn a batch's worth at a time during the
current chunk's steps. The generator therefore runs ahead of the steps
served so far; ``ChunkedDraws`` keeps the generator state at the start of
the chunk being served and, when the next batch is not that chunk's
continuation (another split, a batch out of order, or a draw outside this
schedule), puts the generator back to where the reference's per-step draws
would have left it: the chunk's start state advanced by the numbers the
served batches consumed. The draws every batch gets are thus the reference's
per-step draws in the order the steps run, whatever the interleaving.

Staging buffers form a ring; a buffer holding the next chunk's partial draw
is reserved until its lookup is issued, so no other chunk is drawn into it.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Any, Callable

import torch


@dataclass
class DrawSlot:
    """A staging buffer: ``buf`` (int64 CPU tensor, pinned in the product),
    ``done`` (an object with ``synchronize()`` once a lookup read it, or
    None) and ``addr`` (what the lookup needs to read it)."""
    buf: torch.Tensor
    done: Any = None
    addr: int = 0
    views: dict = field(default_factory=dict)   # (at, k) -> buf[at:at + k], built once

    def view(self, at: int, k: int) -> torch.Tensor:
        v = self.views.get((at, k))
        if v is None:
            if len(self.views) >= 256:   # batch sizes that keep changing
                self.views.clear()
            if at % k == 0:   # every batch-aligned view of the buffer at once, at its first use
                for a in range(0, self.buf.numel() - k + 1, k):
                    self.views[(a, k)] = self.buf[a:a + k]
            v = self.views.get((at, k))
            if v is None:
                v = self.views[(at, k)] = self.buf[at:at + k]
        return v

    def wait(self) -> None:
        if self.done is not None:
            self.done.synchronize()


@dataclass
class _Chunk:
    split: str
    start: int       # first event of the chunk
    hi: int          # one past its last event
    state: torch.Tensor   # the generator state before the chunk's first draw
    consumed: int = 0     # numbers used by the batches served from it
    next: int = 0         # the event the next batch of this chunk starts at


@dataclass
class _PreDraw:
    slot: DrawSlot
    start: int
    m: int
    state: torch.Tensor
    drawn: int = 0


class ChunkedDraws:
    """``serve(split, s, n)`` makes the negatives' draws of events
    ``[s, s + n)`` of a contiguous split available through ``lookup`` (the
    device lookup of a slot's first m numbers for events [s, s + m)), in
    order with every earlier ``serve``. ``split_end(split, s, n)`` gives one
    past the last event of the split that holds batch [s, s + n); ``alloc(size)`` a new staging slot;
    ``pool_size()`` the size of the dst pool."""

    def __init__(self, pool_size: Callable[[], int], split_end: Callable[[str, int, int], int],
                 alloc: Callable[[int], DrawSlot], lookup: Callable[[DrawSlot, int, int], None],
                 chunk: int = 8, ring: int = 4):
        self.pool_size = pool_size
        self.split_end = split_end
        self.alloc = alloc
        self.lookup = lookup
        self.chunk = chunk
        self.ring_size = ring
        self._ring: list[DrawSlot] = []
        self._next = 0
        self.wait_s = 0.0   # host seconds spent waiting for a ring buffer's lookup to finish
        self._cur: _Chunk | None = None
        self._pre: _PreDraw | None = None

    # ------------------------------------------------------------ draws
    def _draw(self, slot: DrawSlot, at: int, k: int) -> None:
        # the numbers of torch.randint(0, pool, (k,)) (randint fills its
        # output with random_(low, high)), into a view made once per slot
        # and range: a slice and randint's out= handling cost more host time
        # per step than the draw itself
        slot.view(at, k).random_(0, self.pool_size())

    def _slot(self, m: int) -> DrawSlot:
        """The next ring buffer not reserved by the pending next-chunk draw,
        once the lookup that last read it is done (grown to m entries)."""
        if not self._ring:   # the whole ring at once: a pinned allocation costs several steps' time
            self._ring = [self.alloc(m) for _ in range(self.ring_size)]
        for _ in range(len(self._ring)):
            i = self._next
            self._next = (self._next + 1) % len(self._ring)
            slot = self._ring[i]
            if self._pre is not None and slot is self._pre.slot:
                continue
            t0 = time.perf_counter()
            slot.wait()
            self.wait_s += time.perf_counter() - t0
            if slot.buf.numel() < m:
                slot = self._ring[i] = self.alloc(m)
            return slot
        raise AssertionError("draw ring: every buffer reserved")  # at most one is

    def release(self) -> None:
        """Put the generator back to the end of the draws that served batches
        used (the chunk's start state advanced by the numbers consumed) and
        drop what was drawn ahead. Called before any draw outside the
        current chunk's continuation."""
        cur = self._cur
        if cur is None:
            return
        torch.set_rng_state(cur.state)
        if cur.consumed:
            torch.randint(low=0, high=self.pool_size(), size=(cur.consumed,), dtype=torch.long)
        self._cur = None
        self._pre = None

    def serve(self, split: str, s: int, n: int) -> None:
        cur = self._cur
        if cur is not None and (cur.split != split or cur.next != s):
            self.release()
            cur = None
        if cur is None or s + n > cur.hi:
            cur = self._draw_ahead(split, s, n)
        cur.consumed += n
        cur.next = s + n
        pre = self._pre
        if pre is not None and pre.drawn < pre.m:   # this step's share of the next chunk's draw
            k = min(n, pre.m - pre.drawn)
            self._draw(pre.slot, pre.drawn, k)
            pre.drawn += k

    def _draw_ahead(self, split: str, s: int, n: int) -> _Chunk:
        end = self.split_end(split, s, n)
        hi = max(s + n, min(end, s + self.chunk * n))
        m = hi - s
        pre = self._pre
        if pre is not None and pre.start == s and pre.m == m:
            # the continuation drawn during the previous chunk's steps (which
            # consumed all of that chunk: pre.start is its end)
            self._pre = None
            slot, state = pre.slot, pre.state
            if pre.drawn < m:
                self._draw(slot, pre.drawn, m - pre.drawn)
        else:
            # anything else (a batch straddling the chunk's end, a first
            # chunk): from the position the served batches left
            self.release()
            state = torch.get_rng_state()
            slot = self._slot(m)
            self._draw(slot, 0, m)
        self.lookup(slot, s, m)
        self._cur = _Chunk(split, s, hi, state, 0, s)
        if hi < end:   # the next chunk of the split, drawn during this chunk's steps
            m2 = min(end, hi + self.chunk * n) - hi
            self._pre = _PreDraw(self._slot(m2), hi, m2, torch.get_rng_state())
        return self._cur
