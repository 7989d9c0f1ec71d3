"""The negatives' draw schedule (backends/ctdg/runtime/negatives.py) against
the reference's per-step draws (runtime.py:124-136: one torch.randint of the
batch's size on the global CPU generator per step), on the CPU: whatever the
order of the steps -- a split interrupted mid-chunk by a multi-chunk pass
over another split, batches out of order, a draw outside the schedule, a
batch size that changes -- every batch gets the numbers that sequential
per-step draws give in the order the steps ran. A planted mistake (no
rewind of the generator) must fail the same check."""
import pytest
import torch

from starry_unigraph.backends.ctdg.runtime.negatives import ChunkedDraws, DrawSlot

POOL = 1000
SPLITS = {"train": (0, 6000), "val": (6000, 7000), "test": (7000, 8000)}


class Harness:
    """The device side modelled as deferred work: a lookup reads its staging
    buffer only when the host waits for it (DrawSlot.wait) or when the step
    that needs it runs (the end of serve), as the GPU's queue would."""

    def __init__(self, chunk=3, ring=4, draws_cls=ChunkedDraws):
        self.out = torch.full((8000,), -1, dtype=torch.long)
        self.pending = []
        h = self

        class Done:
            def synchronize(self):
                h.flush()

        def split_end(split, s, n):
            a, b = SPLITS[split]
            return b if a <= s < b else s + n

        def alloc(m):
            return DrawSlot(torch.empty(max(m, 1), dtype=torch.long))

        def lookup(slot, s, m):
            self.pending.append((slot, s, m))
            slot.done = Done()

        self.d = draws_cls(lambda: POOL, split_end, alloc, lookup, chunk=chunk, ring=ring)

    def flush(self):
        for slot, s, m in self.pending:
            self.out[s:s + m] = slot.buf[:m]
        self.pending.clear()

    def serve(self, split, s, n):
        self.d.serve(split, s, n)
        self.flush()
        return self.out[s:s + n].clone()


def _run(sequence, **kw):
    """sequence: (split, start, size) batches or ("raw", size) draws outside
    the schedule. Returns [(got, want)] per entry."""
    torch.manual_seed(77)
    h = Harness(**kw)
    got = []
    for item in sequence:
        if item[0] == "raw":
            h.d.release()
            got.append(torch.randint(0, POOL, (item[1],), dtype=torch.long))
        else:
            got.append(h.serve(*item))
    torch.manual_seed(77)
    want = [torch.randint(0, POOL, ((item[1] if item[0] == "raw" else item[2]),), dtype=torch.long)
            for item in sequence]
    return got, want


def _train(i, B=100):
    return ("train", i * B, B)


def _val(i, B=100):
    return ("val", 6000 + i * B, B)


SEQUENCES = {
    "whole splits in order": [_train(i) for i in range(60)] + [_val(i) for i in range(10)],
    "mid-epoch val of several chunks": ([_train(i) for i in range(7)] + [_val(i) for i in range(8)]
                                        + [_train(i) for i in range(7, 20)]),
    "val pass twice inside train": ([_train(i) for i in range(4)] + [_val(i) for i in range(5)]
                                    + [_train(i) for i in range(4, 9)] + [_val(i) for i in range(5)]
                                    + [_train(i) for i in range(9, 15)]),
    "out of order and repeated batches": ([_train(i) for i in range(5)] + [_train(20), _train(21), _train(3)]
                                          + [_train(i) for i in range(4, 10)]),
    "raw draws between steps": ([_train(i) for i in range(5)] + [("raw", 37)] + [_train(i) for i in range(5, 12)]
                                + [("raw", 5)]),
    "batch size change inside a chunk": ([_train(i) for i in range(4)] + [("train", 400, 250), ("train", 650, 250)]
                                         + [("train", 900 + 100 * i, 100) for i in range(6)]),
    "split tail and predict": ([("test", 7000 + 300 * i, 300) for i in range(3)] + [("test", 7900, 100)]
                               + [_train(i) for i in range(3)]),
}


@pytest.mark.parametrize("name", sorted(SEQUENCES))
@pytest.mark.parametrize("chunk,ring", [(3, 4), (8, 4), (2, 2)])
def test_draws_equal_per_step_draws(name, chunk, ring):
    got, want = _run(SEQUENCES[name], chunk=chunk, ring=ring)
    for i, (g, w) in enumerate(zip(got, want)):
        assert torch.equal(g, w), (name, i, SEQUENCES[name][i])


class _NoRewind(ChunkedDraws):
    """Planted mistake: what was drawn ahead stays consumed."""

    def release(self):
        self._cur = None
        self._pre = None


@pytest.mark.parametrize("cls,name", [(_NoRewind, "mid-epoch val of several chunks"),
                                      (_NoRewind, "raw draws between steps"),
                                      (_NoRewind, "out of order and repeated batches")])
def test_planted_mistakes_fail(cls, name):
    got, want = _run(SEQUENCES[name], chunk=3, ring=2, draws_cls=cls)
    assert not all(torch.equal(g, w) for g, w in zip(got, want))
