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
