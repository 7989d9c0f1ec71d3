"""The host-side deal of the fused weight-gradient + Adam tiles to XCDs
(starry_unigraph.native.step.xcd_tile_deal): the tile_job table that
sgl_grad_adam and sgl_grad_shadows decode (job in bits 0-7, the tile's index
within its job above, -1 for a padding slot; workgroup t runs on XCD t % 8)."""
import random

import pytest

from starry_unigraph.native.step import per_workgroup_jobs, xcd_tile_deal


def _decode(table):
    return [(e & 0xFF, e >> 8) for e in table if e >= 0]


@pytest.mark.parametrize("counts", [
    [1],
    [7, 7, 49, 49, 56, 56, 56, 56, 1, 7, 7, 49, 49, 7, 7, 49, 49, 7, 7, 1],   # config-4-like jobs
    [3, 0, 5],
    [300],
    [8] * 8,
    [1] * 17,
])
def test_every_tile_once_and_per_xcd_share(counts):
    table = xcd_tile_deal(counts)
    total = sum(counts)
    got = sorted(_decode(table))
    want = sorted((j, l) for j, c in enumerate(counts) for l in range(c))
    assert got == want
    assert len(table) % 8 == 0
    cap = -(-total // 8)
    per_xcd = [sum(1 for t, e in enumerate(table) if e >= 0 and t % 8 == x) for x in range(8)]
    assert max(per_xcd) <= cap and sum(per_xcd) == total
    # padding only after an XCD's last tile
    for x in range(8):
        col = [table[t] for t in range(x, len(table), 8)]
        assert all(e >= 0 for e in col[:per_xcd[x]]) and all(e == -1 for e in col[per_xcd[x]:])


def test_a_job_that_fits_stays_on_one_xcd_in_order():
    counts = [7, 7, 49, 49, 56, 56, 56, 56, 1, 7, 7, 49, 49, 7, 7, 49, 49, 7, 7, 1]
    table = xcd_tile_deal(counts)
    where = {}
    for t, e in enumerate(table):
        if e >= 0:
            where.setdefault(e & 0xFF, []).append((t % 8, e >> 8, t))
    for j in (4, 5, 6, 7):   # the 56-tile jobs: below the 60-tile share, one XCD each
        xcds = {x for x, _, _ in where[j]}
        assert len(xcds) == 1
    # on an XCD a job's tiles are consecutive indices in workgroup order
    for j, lst in where.items():
        for x in {x for x, _, _ in lst}:
            locs = [l for xx, l, _ in sorted(lst, key=lambda v: v[2]) if xx == x]
            assert locs == list(range(locs[0], locs[0] + len(locs)))


def test_random_counts():
    rng = random.Random(5)
    for _ in range(200):
        counts = [rng.randint(0, 90) for _ in range(rng.randint(1, 40))]
        table = xcd_tile_deal(counts)
        assert sorted(_decode(table)) == sorted((j, l) for j, c in enumerate(counts) for l in range(c))


def test_limits():
    assert xcd_tile_deal([]) == [] and xcd_tile_deal([0, 0]) == []
    with pytest.raises(ValueError):
        xcd_tile_deal([1] * 257)


def test_per_workgroup_jobs_match_the_deal():
    """sgl_grad_adam's table without tile_job: workgroup t's entry is a copy
    of the job the deal's entry t names, tile0 = the tile's index within it,
    kind -1 for a padding slot; the other fields are the job's."""
    from starry_unigraph.lib import _capi
    counts = [7, 0, 49, 3, 56, 1]
    jobs = []
    for k, c in enumerate(counts):
        j = _capi.GradJob()
        j.kind = k % 2
        j.rows, j.cols, j.seg, j.r_fixed, j.off = 16 * c + 1, 3 + k, k % 3, -k, 1000 * k
        j.tile0 = 12345   # replaced in the copies
        jobs.append(j)
    deal = xcd_tile_deal(counts)
    table = per_workgroup_jobs(jobs, deal)
    assert len(table) == len(deal)
    for e, t in zip(deal, table):
        if e < 0:
            assert t.kind == -1
            continue
        src = jobs[e & 0xFF]
        assert t.tile0 == e >> 8
        for f in ("kind", "rows", "cols", "seg", "r_fixed", "off"):
            assert getattr(t, f) == getattr(src, f), f
    assert jobs[0].tile0 == 12345   # the source jobs are not modified
