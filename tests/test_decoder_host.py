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


def test_fork_page_tables_no_copy_on_boundaries():
    import numpy as np

    pt = np.arange(12, dtype=np.int32).reshape(3, 4)
    new, copies = dec.fork_page_tables(pt, [0, 0, 0], np.array([8, 8, 8]), 4, 12)
    assert copies == []  # full pages are shared, the next ones are fresh
    assert list(new[:, 0]) == [0, 0, 0] and list(new[:, 1]) == [1, 1, 1]
    assert len(set(new[:, 2:].ravel().tolist())) == 6
    new, copies = dec.fork_page_tables(pt, [1, 1, 2], np.array([5, 5, 9]), 4, 12)
    assert len(copies) == 1 and copies[0][0] == 5  # stream 1's partly filled page 5, once
