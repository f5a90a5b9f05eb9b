"""Pins the oracle's mHC pieces (RMSUnit, the heads and Sinkhorn, the lane
sum and the mix; internal/needle/norm.go:68-81, mhc.go:182-417) against
go-whistle's own golden fixture, testdata/needle/mhc.safetensors (upstream's
Flax mHC at float32 on Whistle's layers 0 and 1; tests/golden/mhc_fixture.npz,
written by tests/golden/make_mhc_fixture.py), to its contract of 1e-5, and
against the properties the reference's Sinkhorn tests hold
(mhc_test.go:66-196)."""

import os

import numpy as np
import pytest

from oracle import binding as orc

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "mhc_fixture.npz")


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(np.max(np.abs(a - b)) / max(1.0, np.max(np.abs(b))))


def layer_stream(f, l):
    if l == 0:  # ExpandLanes of x (mhc.go:140-154)
        return np.repeat(f["x"][0][:, None, :], 4, axis=1)
    return f["layer1__stream_in"][0]


@pytest.mark.parametrize("l", [0, 1])
def test_mhc_pieces_match_upstream(l):
    f = np.load(FIX)
    L = lambda k: f[f"layer{l}__{k}"]
    stream = layer_stream(f, l)
    assert rel(orc.rms_unit(stream.reshape(8, 2048), 8, 2048), L("nx")) <= 1e-6
    hp, hq, hr, u = orc.mhc_heads(L("h_pre_logits"), L("h_post_logits"), L("h_res_logits"), stream, 8, 4, 512)
    assert rel(hp, L("h_pre")) <= 1e-6 and rel(hq, L("h_post")) <= 1e-6
    assert rel(hr, L("h_res")) <= 2e-7  # 20 iterations (mhc_test.go:121-147: 1.2e-7)
    assert rel(u, L("u")) <= 1e-6
    out = orc.mhc_mix(stream, hr, hq, L("block_out"), u, 8, 4, 512)
    assert rel(out, L("stream_out")) <= 1e-6


def test_sinkhorn_iteration_count_matters():
    """19 or 21 iterations miss the fixture's h_res by far more than 20 do
    (mhc_test.go:121-147)."""
    f = np.load(FIX)
    logits, want = f["layer0__h_res_logits"].reshape(-1, 16), f["layer0__h_res"].reshape(-1, 16)
    errs = {it: max(rel(orc.sinkhorn(r, 4, it), w) for r, w in zip(logits, want)) for it in (19, 20, 21)}
    assert errs[20] <= 2e-7 and errs[19] > 1e-5 and errs[21] > 1e-5


def test_sinkhorn_properties():
    """Columns sum to 1 within 4e-7, entries in [0, 1], the float64 exp and
    the float32 log domains (large logits) alike; equal logits give 1/4
    exactly (mhc_test.go:66-196)."""
    g = np.random.default_rng(4)
    for scale in (0.1, 1.0, 4.0, 1e3, 1e4, 1e30):
        for trial in range(10):
            k = (g.standard_normal(16) * scale).astype(np.float32)
            if trial % 2:
                k[[0, 5, 10, 15]] += 4
            h = orc.sinkhorn(k, 4).astype(np.float64).reshape(4, 4)
            assert np.all(np.isfinite(h)) and np.all(h >= 0) and np.all(h <= 1), (scale, trial)
            assert np.max(np.abs(h.sum(0) - 1)) <= 4e-7, (scale, trial)
    assert np.all(orc.sinkhorn(np.full(16, 3.5, np.float32), 4) == np.float32(0.25))


def test_rms_unit_closed_form():
    """A constant row c: ms = c^2, the output c / sqrt(c^2 + 1e-6) rounded."""
    c = np.float32(3.0)
    row = np.full(512, c, np.float32)
    got = orc.rms_unit(row, 1, 512)
    inv = np.float32(1.0 / np.sqrt(np.float64(np.float32(c * c) + np.float32(1e-6))))
    assert np.all(got == c * inv)
