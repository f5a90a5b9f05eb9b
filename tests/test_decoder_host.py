"""The decoder's host-side checks, without a GPU: decoding past the caches
and RoPE tables (max_pos) is refused before anything is queued, as the
reference's cache slicing and table lookups panic there
(internal/needle/rope.go:69-81, internal/needle/cache.go:78-112)."""

import pytest

from go_whistle_amd import decoder as dec
from go_whistle_amd._lib import CQPanic


def _bare(max_pos):
    d = dec.Decoder.__new__(dec.Decoder)  # the host state only: no device arrays
    d.cfg = dec.DecoderConfig(max_pos=max_pos)
    d.steps = 0
    return d


def test_decode_past_max_pos_raises():
    d = _bare(16)
    with pytest.raises(CQPanic):
        d.decode([1], 17)
    with pytest.raises(CQPanic):
        d.resume(17)
    d.steps = 10
    with pytest.raises(CQPanic):
        d.resume(7)
    with pytest.raises(CQPanic):
        d.resume(-1)
    d.steps = 16
    with pytest.raises(CQPanic):
        d.step()


def test_reserve_allows_exactly_max_pos():
    d = _bare(16)
    d._reserve(16)
    d.steps = 15
    d._reserve(1)


def _simulate_forks(seed, streams, per, rows, rounds):
    """Beam-like rounds of appends and forks over a paged pool, against
    every stream's history kept as its own list (a deep copy on each fork,
    the semantics KVCache.Fork shares rows for, internal/needle/cache.go:
    62-67). Returns the largest copy count of one fork."""
    import numpy as np

    g = np.random.default_rng(seed)
    pool = streams * per
    pt = np.arange(pool, dtype=np.int32).reshape(streams, per)
    data = np.full((pool, rows), -1, np.int64)  # the pool's rows: a value per row
    want = [[] for _ in range(streams)]
    pos = np.zeros(streams, np.int64)
    most = 0
    tag = 0
    for _ in range(rounds):
        for _ in range(int(g.integers(0, 4))):  # every stream appends a few rows
            for b in range(streams):
                if pos[b] >= per * rows:
                    continue
                page = pt[b, pos[b] // rows]
                tag += 1
                data[page, pos[b] % rows] = tag
                want[b].append(tag)
                pos[b] += 1
        parents = g.integers(0, streams, size=streams)
        new_pt, copies = dec.fork_page_tables(pt, parents, pos[parents], rows, pool)
        most = max(most, len(copies))
        assert len(copies) <= streams
        for src, dst in copies:
            data[dst] = data[src]
        pt = new_pt
        pos = pos[parents]
        want = [list(want[p]) for p in parents]
        assert pt.min() >= 0 and pt.max() < pool
        for b in range(streams):  # pages a stream still writes on are its own
            lp0 = pos[b] // rows
            for lp in range(lp0, per):
                assert (pt == pt[b, lp]).sum() == 1, (b, lp)
            got = [data[pt[b, r // rows], r % rows] for r in range(pos[b])]
            assert got == want[b], b
    return most


def test_fork_page_tables_match_deep_copies():
    # random parents over many rounds: each stream reads exactly its own
    # history through its table, and a fork copies at most one page per
    # stream, at any position
    for seed in range(6):
        _simulate_forks(seed, streams=6, per=8, rows=4, rounds=40)


def _fork_page_tables_in_turn(pt, parents, pos, page_rows, pool_pages):
    """fork_page_tables one reference at a time, in stream-then-page order:
    each page a stream must own from pos // page_rows on is replaced by the
    smallest free page while another entry still references it."""
    import numpy as np

    pt = np.asarray(pt, np.int32)[np.asarray(parents, np.int64)].copy()
    streams, per = pt.shape
    counts = np.bincount(pt.ravel(), minlength=pool_pages)
    free = list(np.flatnonzero(counts == 0)[::-1])
    copies = []
    for b in range(streams):
        lp0 = min(int(pos[b]) // page_rows, per)
        for lp in range(lp0, per):
            ph = int(pt[b, lp])
            if counts[ph] > 1:
                nf = int(free.pop())
                counts[ph] -= 1
                counts[nf] += 1
                pt[b, lp] = nf
                if lp == lp0 and pos[b] % page_rows:
                    copies.append((ph, nf))
    return pt, copies


def test_fork_page_tables_equal_the_reference_at_a_time_form():
    # the vectorised bookkeeping gives the same tables and copies as taking
    # the references one at a time, over random beam rounds (256 streams of
    # 16 pages of 16 rows, as the decoder's batch-256 paged step)
    import numpy as np

    g = np.random.default_rng(7)
    streams, per, rows = 256, 16, 16
    pool = streams * per
    pt = np.arange(pool, dtype=np.int32).reshape(streams, per)
    pos = np.zeros(streams, np.int64)
    for _ in range(30):
        pos = np.minimum(pos + g.integers(0, 24, size=streams), per * rows)
        parents = g.integers(0, streams, size=streams)
        want, wc = _fork_page_tables_in_turn(pt, parents, pos[parents], rows, pool)
        got, gc = dec.fork_page_tables(pt, parents, pos[parents], rows, pool)
        assert np.array_equal(got, want) and gc == wc
        pt, pos = got, pos[parents]


def test_fork_page_tables_no_copy_on_boundaries():
    import numpy as np

    pt = np.arange(12, dtype=np.int32).reshape(3, 4)
    new, copies = dec.fork_page_tables(pt, [0, 0, 0], np.array([8, 8, 8]), 4, 12)
    assert copies == []  # full pages are shared, the next ones are fresh
    assert list(new[:, 0]) == [0, 0, 0] and list(new[:, 1]) == [1, 1, 1]
    assert len(set(new[:, 2:].ravel().tolist())) == 6
    new, copies = dec.fork_page_tables(pt, [1, 1, 2], np.array([5, 5, 9]), 4, 12)
    assert len(copies) == 1 and copies[0][0] == 5  # stream 1's partly filled page 5, once
