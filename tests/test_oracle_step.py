"""Pins the oracle's decode-step float blocks: ZCRMSNorm (norm.go:53-109)
against float64 and a closed form, RoPE (rope.go:69-81) against the float64
rotation and the identity at position 0, argmax (greedy.go:181-191)
against numpy's first-index argmax with ties, SiLU against float64."""

import math

import numpy as np
import pytest

from go_whistle_amd import decoder as dec
from go_whistle_amd import synth
from oracle import binding as orc


def test_zc_rmsnorm_vs_float64_and_constant_row():
    g = synth.rng(1)
    x = (g.standard_normal(5 * 512) * 3).astype(np.float32)
    gain = (1 + g.standard_normal(512) * 0.1).astype(np.float32)
    y = orc.zc_rmsnorm(x, gain, 512).reshape(5, 512)
    x64 = x.reshape(5, 512).astype(np.float64)
    want = gain * x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6)
    assert np.max(np.abs(y - want) / np.abs(want).max()) < 4e-7
    # a constant row c: mean square c^2 exactly, y = gain * c / float32(sqrt(c^2 + 1e-6))
    c = np.float32(2.0)
    y = orc.zc_rmsnorm(np.full(512, c, np.float32), np.ones(512, np.float32), 512)
    rms = np.float32(np.sqrt(np.float64(np.float32(np.float32(4.0) + np.float32(1e-6)))))
    assert np.all(y == np.float32(c / rms))


def test_rope_identity_and_float64_rotation():
    cos, sin = dec.rope_tables(64, 16, 1e5)
    assert np.all(cos[0] == 1) and np.all(sin[0] == 0)
    g = synth.rng(2)
    x = g.standard_normal(8 * 64).astype(np.float32)
    assert np.array_equal(orc.rope(x, 8, 64, cos, sin, [0]), x)
    y = orc.rope(x, 8, 64, cos, sin, [7]).reshape(8, 64)
    xx = x.reshape(8, 64).astype(np.float64)
    c64, s64 = cos[7].astype(np.float64), sin[7].astype(np.float64)
    want = np.concatenate([xx[:, :32] * c64 - xx[:, 32:] * s64, xx[:, 32:] * c64 + xx[:, :32] * s64], axis=1)
    assert np.max(np.abs(y - want)) < 1e-6 * np.abs(xx).max() * 4
    # the tables: angle t / theta^(2i/d) (rope.go:33-41)
    t, i = 7, 5
    ang = 7 / (1e5 ** (2 * i / 64))
    assert abs(cos[t, i] - np.cos(ang)) < 1e-6 and abs(sin[t, i] - np.sin(ang)) < 1e-6


def test_argmax_first_on_ties():
    g = synth.rng(3)
    v = g.standard_normal((4, 1000)).astype(np.float32)
    v[1, 17] = v[1, 900] = 50
    v[2, :] = 0
    v[3, 999] = 9
    got = orc.argmax(v, 4, 1000)
    assert list(got) == [int(np.argmax(v[0])), 17, 0, 999]


def test_argmax_nan_and_signed_zero():
    # greedy.go's loop compares x > v[best] from best = 0: NaN never wins, a
    # NaN at index 0 is never beaten, and +0 does not beat -0. Stated here
    # as its closed form: 0 if v[0] is NaN, else the first index of the
    # largest non-NaN value.
    nan = np.float32("nan")
    rows = [
        [1, nan, 5, 5, 2],
        [nan, 9, 8, 7, 6],
        [-0.0, 0.0, -1, -2, -3],
        [-np.inf, -np.inf, -np.inf, -np.inf, -np.inf],
        [nan, nan, nan, nan, nan],
        [3, nan, nan, 3, nan],
    ]
    v = np.array(rows, np.float32)

    def closed_form(r):
        if np.isnan(r[0]):
            return 0
        m = np.nanmax(r)
        return int(np.flatnonzero(r == m)[0])

    assert list(orc.argmax(v, len(rows), 5)) == [closed_form(r) for r in v] == [2, 0, 0, 0, 0, 0]


def test_silu_vs_float64():
    x = np.concatenate([np.linspace(-30, 30, 20001), [0.0, -0.0, 1e-30, -1e-30, 80.0, -80.0]]).astype(np.float32)
    got = orc.silu(x).astype(np.float64)
    xx = x.astype(np.float64)
    want = xx / (1 + np.exp(-xx))
    err = np.abs(got - want)
    assert np.all(err <= 4 * 2.0 ** -23 * np.abs(want) + 1e-37)


def test_exp64_vs_libm_and_exact_points():
    """fdlibm's exp against the C library's (Python's math.exp): within 1 ulp
    everywhere, bit-equal in most cases, and the closed forms exp(0) = 1,
    exp(k ln 2) = 2^k to 1 ulp, the overflow and underflow edges."""
    g = np.random.default_rng(11)
    x = np.concatenate([g.standard_normal(4000) * 4, g.uniform(-740, 705, 4000), g.standard_normal(500) * 1e-9])
    got = orc.exp64(x)
    want = np.array([math.exp(v) for v in x])
    ulps = np.abs(got.view(np.int64) - want.view(np.int64))
    assert ulps.max() <= 1
    assert (ulps == 0).mean() > 0.8
    assert orc.exp64([0.0])[0] == 1.0 and abs(orc.exp64([1.0])[0] - math.e) <= 2.0 ** -51  # 1 ulp of e
    y = g.uniform(-700, 700, 2000)
    prod = orc.exp64(y) * orc.exp64(-y)  # exp(y) exp(-y) = 1
    assert np.all(np.abs(prod - 1.0) <= 3 * 2.0 ** -52)
    big = orc.exp64([709.0, 710.0, -745.0, -746.0, float("nan")])
    assert np.isfinite(big[0]) and np.isinf(big[1]) and big[2] > 0 and big[3] == 0 and np.isnan(big[4])


def test_gate_sigmoid_bit_exact_and_closed_forms():
    """The gate's sigmoid (load.go:120-123) against float32(1/(1 + exp(-x)))
    with the C library's exp, bit for bit, and its fixed points: 0.5 at 0,
    exactly 1 and 0 in the tails, the smallest subnormal just before 0."""
    g = np.random.default_rng(12)
    x = (g.standard_normal(50000) * 8).astype(np.float32)
    got = orc.gate_sigmoid(x)
    want = np.array([np.float32(1.0 / (1.0 + math.exp(-float(v)))) for v in x], np.float32)
    assert np.array_equal(got.view(np.int32), want.view(np.int32))
    edge = orc.gate_sigmoid([0.0, -0.0, 40.0, 800.0, -103.0, -104.0, float("inf"), float("-inf")])
    assert list(edge[:4]) == [0.5, 0.5, 1.0, 1.0]
    assert edge[4] == np.float32(2.0 ** -149) and edge[5] == 0.0 and edge[6] == 1.0 and edge[7] == 0.0
    # 1 - sigmoid(x) = sigmoid(-x) for float64; in float32 within an ulp of the larger
    s, t = orc.gate_sigmoid(x[:2000]).astype(np.float64), orc.gate_sigmoid(-x[:2000]).astype(np.float64)
    assert np.all(np.abs(s + t - 1.0) <= 2.0 ** -23)


def test_sigmoid_gate_updates_both():
    """Attention.output (attention.go:245-249): gate becomes sigmoid(gate),
    out becomes out * gate, each rounded to float32; a plain restatement of
    the planted case where the gate is 0 (sigmoid 1/2: out halves exactly)."""
    out = np.array([3.0, -5.0, 1e-30, 7.0], np.float32)
    gate = np.zeros(4, np.float32)
    o, gg = orc.sigmoid_gate(out, gate)
    assert list(gg) == [0.5] * 4 and list(o) == list(out / 2)
    g = np.random.default_rng(13)
    out, gate = g.standard_normal(300).astype(np.float32), g.standard_normal(300).astype(np.float32)
    o, gg = orc.sigmoid_gate(out, gate)
    assert np.array_equal(gg, orc.gate_sigmoid(gate))
    assert np.array_equal(o, (out * gg).astype(np.float32))


def test_norms_match_upstream_fixture():
    """ZCRMSNorm's divisor and RMSUnit against go-whistle's golden fixture
    (testdata/needle/zcrmsnorm.safetensors, upstream at float32; extracted
    into tests/golden/zcrmsnorm_fixture.npz): within 4e-7 relative, the
    reference's own figure for this fixture (its README lists 3.9e-7). The
    mean square here sums in float64, upstream in float32."""
    import os

    f = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "zcrmsnorm_fixture.npz"))
    x = f["x"].reshape(-1, 512)
    rows = x.shape[0]
    ru = orc.rms_unit(x, rows, 512).reshape(rows, 512)
    want = f["rms_unit"].reshape(rows, 512)
    assert np.max(np.abs(ru - want)) <= 4e-7 * np.max(np.abs(want))
    y = orc.zc_rmsnorm(x.ravel(), np.ones(512, np.float32), 512).reshape(rows, 512)  # gain 1: x / rms
    ref = x / f["rms"].reshape(rows, 1)
    assert np.max(np.abs(y - ref)) <= 4e-7 * np.max(np.abs(ref))
