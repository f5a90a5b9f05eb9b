"""Pins the CPU oracle's int8 KV part: the reference's hand vectors and
invariants for QuantizeRow (internal/needle/int8_test.go:16-61), brute
force for the int8 dot products, float64 recomputation for the weighted
sums and the attention (int8_test.go:207-284), and the exponent kernel's
accuracy, flush and exact points (exp_test.go:21-145)."""

import math

import numpy as np
import pytest

from go_whistle_amd import synth
from oracle import binding as orc


def test_quantize_row_hand_vectors():
    q, s = orc.quantize_row([127, 2.5, -2.5, 3.5, -0.5, 1.4999])
    assert s == 1 and list(q) == [127, 2, -2, 4, 0, 1]  # ties to even
    q, s = orc.quantize_row([-6.35, 0.05, 3])
    assert s == np.float32(np.float32(6.35) / np.float32(127)) and list(q) == [-127, 1, 60]
    q, s = orc.quantize_row(np.zeros(4, np.float32))
    assert s == 1 and list(q) == [0, 0, 0, 0]


NAN, INF = np.float32("nan"), np.float32("inf")


@pytest.mark.parametrize("row,scale,codes", [
    # Go's max keeps a NaN (int8.go:40-42): the bound is NaN, m > 0 fails,
    # s = 1; codes are RNE(x) clamped by Go's NaN-propagating min/max, and
    # int8 of a NaN is 0 (amd64's integer indefinite 0x80000000, low byte 0)
    ([1, NAN, -2, 3.6, 200, -1000], 1, [1, 0, -2, 4, 127, -128]),
    ([NAN, INF, -INF, 0.4, 2.5], 1, [0, 127, -128, 0, 2]),
    # an infinite bound: s = Inf, x / Inf is +-0 for finite x and NaN for
    # +-Inf, so every code is 0
    ([INF, 1, -1, 1e30], INF, [0, 0, 0, 0]),
    ([-INF, 5], INF, [0, 0]),
    ([NAN], 1, [0]),
])
def test_quantize_row_nan_and_inf(row, scale, codes):
    q, s = orc.quantize_row(np.array(row, np.float32))
    assert (s == scale) and list(q) == codes


def test_fake_quant_nan_and_inf():
    # float32(q) * s: a NaN row comes back as its clamped codes (scale 1), an
    # infinite row as 0 * Inf = NaN everywhere
    got = orc.fake_quant(np.array([NAN, 2.5, -300, 1, INF, 0.5], np.float32), 6, 3)
    assert list(got[:3]) == [0, 2, -128]
    assert np.isnan(got[3:]).all()


def test_softmax_nan_and_inf():
    # softmaxInPlace (load.go:128-138): Go's max keeps a NaN, so one NaN logit
    # makes every weight NaN; a +Inf logit gives Inf - Inf = NaN at its key
    # and a NaN sum; -Inf logits beside finite ones weigh 0
    for variant in (0, 1):
        s = orc.softmax(np.array([0, -1, NAN, 2, 0.5, 1, 1, 1, 3], np.float32), variant)
        assert np.isnan(s).all()
        s = orc.softmax(np.array([0, INF, 2, 0.5, 1, 1, 1, 3, 4], np.float32), variant)
        assert np.isnan(s).all()
        s = orc.softmax(np.array([0, -INF, 0, -INF, 0, 0, 0, 0, 0], np.float32), variant)
        assert s[1] == 0 and s[3] == 0 and np.all(s[[0, 2, 4, 5, 6, 7, 8]] == np.float32(1 / 7))


@pytest.mark.parametrize("n", [1, 7, 48, 64, 2048])
@pytest.mark.parametrize("scale", [1e-6, 1, 1e4])
def test_quantize_row_invariants(n, scale):
    g = synth.rng(n)
    x = (g.standard_normal(n) * scale).astype(np.float32)
    x[g.integers(0, n)] *= 9
    q, s = orc.quantize_row(x)
    m = np.float32(np.abs(x).max())
    assert s == np.float32(m / np.float32(127))
    d = np.abs(x.astype(np.float64) - float(s) * q.astype(np.float64))
    # within half a step, plus the float32 rounding of x/s (|x/s| <= 127),
    # which can carry x/s across a half point: 127 * 2^-24 of a step
    assert np.all(d <= float(s) * (0.5 + 128 * 2.0 ** -24))
    assert q.min() >= -127


def test_quantize_rows_per_chunk():
    g = synth.rng(5)
    x = g.standard_normal(3 * 96).astype(np.float32)
    q, s = orc.quantize_rows(x, 96, 48)
    assert s.size == 6
    for c in range(6):
        qc, sc = orc.quantize_row(x[c * 48:(c + 1) * 48])
        assert np.array_equal(q[c * 48:(c + 1) * 48], qc) and s[c] == sc


def test_fake_quant_hand_vectors_and_bound():
    # fakeQuant (int8.go:57-75) is QuantizeRow and back, float32(q) * s:
    # the hand vectors of int8_test.go:19-34 give exact values, and any row
    # stays within half a step (plus the divide's rounding) of its input
    got = orc.fake_quant(np.array([127, 2.5, -2.5, 3.5, -0.5, 1.4999], np.float32), 6, 6)
    assert list(got) == [127, 2, -2, 4, 0, 1]
    s = np.float32(np.float32(6.35) / np.float32(127))
    got = orc.fake_quant(np.array([-6.35, 0.05, 3], np.float32), 3, 3)
    assert list(got) == [np.float32(-127) * s, np.float32(1) * s, np.float32(60) * s]
    assert list(orc.fake_quant(np.zeros(4, np.float32), 4, 4)) == [0, 0, 0, 0]
    g = synth.rng(31)
    x = (g.standard_normal(3 * 2048) * 3).astype(np.float32)
    fq = orc.fake_quant(x, 2048, 2048)
    for r in range(3):
        xr = x[r * 2048:(r + 1) * 2048]
        sr = float(np.float32(np.abs(xr).max() / np.float32(127)))
        d = np.abs(xr.astype(np.float64) - fq[r * 2048:(r + 1) * 2048].astype(np.float64))
        assert np.all(d <= sr * (0.5 + 128 * 2.0 ** -24) + abs(xr).max() * 2.0 ** -24)


@pytest.mark.parametrize("width", [16, 48, 64, 8, 17])
@pytest.mark.parametrize("n", [1, 5, 375])
def test_dots_i8_bruteforce(width, n):
    g = synth.rng(width * 1000 + n)
    stride = width + 16
    k = g.integers(-128, 128, size=(n - 1) * stride + width).astype(np.int8)
    q = g.integers(-128, 128, size=width).astype(np.int8)
    q[0], k[0] = -128, -128
    got = np.zeros(n, np.int32)
    orc.lib().orc_dots_i8(orc.i32p(got), n, orc.i8p(q), width, orc.i8p(k), stride)
    rows = np.stack([k[j * stride:j * stride + width] for j in range(n)]).astype(np.int64)
    assert np.array_equal(got, rows @ q.astype(np.int64))


def test_axpys_and_float_dots_vs_float64():
    g = synth.rng(11)
    n, width, stride = 375, 64, 128
    v = g.integers(-128, 128, size=(n - 1) * stride + width).astype(np.int8)
    w = g.standard_normal(n).astype(np.float32)
    out = g.standard_normal(width).astype(np.float32)
    ref = out.astype(np.float64) + sum(float(w[j]) * v[j * stride:j * stride + width].astype(np.float64)
                                       for j in range(n))
    orc.lib().orc_axpys_i8(orc.fp(out), width, orc.fp(w), n, orc.i8p(v), stride)
    mag = np.abs(w).sum() * 128 + 10
    assert np.max(np.abs(out - ref)) <= (n + 2) * 2 ** -24 * mag
    q = g.standard_normal(width).astype(np.float32)
    dst = np.zeros(n, np.float32)
    orc.lib().orc_dots_f32_i8(orc.fp(dst), n, orc.fp(q), width, orc.i8p(v), stride)
    for j in range(0, n, 17):
        exact = q.astype(np.float64) @ v[j * stride:j * stride + width].astype(np.float64)
        assert abs(dst[j] - exact) <= (width + 1) * 2 ** -24 * (np.abs(q).sum() * 128)


def _check_exp(s, m, variant):
    got, got_sum = orc.exp_sub_sum(s, m, variant)
    want = np.exp((np.asarray(s, np.float32) - np.float32(m)).astype(np.float64))
    flush = 1.2e-38
    ok = want > flush
    rel = np.abs(got[ok] - want[ok]) / (2.0 ** -23 * want[ok])
    assert np.all(rel <= 2), rel.max()
    assert np.all(got[~ok] <= flush)
    n = len(s)
    bound = (2 * (n + 1) * 2 ** -24 + 2 * 2 ** -23) * want.sum() + n * flush
    assert abs(float(got_sum) - want.sum()) <= bound
    return got, got_sum


@pytest.mark.parametrize("variant", [0, 1])
def test_exp_sub_sum_random(variant):
    g = synth.rng(21)
    for n in list(range(0, 70)) + [127, 128, 129, 375, 1000, 4099]:
        for scale in (0.1, 3, 30, 100):
            s = (g.standard_normal(n) * scale).astype(np.float32)
            m = s.max() if n else np.float32(0)
            _check_exp(s, m, variant)


def test_exp_kernel_sweep_flush_and_exact_points():
    steps = 1 << 16
    s = (-90 * np.arange(steps, dtype=np.float32) / np.float32(steps)).astype(np.float32)
    _check_exp(s, 0, 1)
    got, total = orc.exp_sub_sum(np.zeros(8, np.float32), 0, 1)
    assert total == 8 and np.all(got == 1)
    lanes = np.array([0, -90, -np.inf, -87.3, -1, -2, -3, -4], np.float32)
    got, _ = orc.exp_sub_sum(lanes, 0, 1)
    assert got[1] <= 1.2e-38 and got[2] == 0 and got[3] >= 1.2e-38


def test_exp_kernel_lane_sum_structure():
    # The kernel's sum is ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)) over lane
    # partials l_k (sums of elements k, k+8, ... in order), plus the tail in
    # order (exp_amd64.s:112-121, exp_amd64.go:19-24); it must equal that
    # restated sum of the oracle's own per-element values.
    g = synth.rng(3)
    for n in (8, 16, 37, 375):
        s = (g.standard_normal(n) * 3).astype(np.float32)
        e, total = orc.exp_sub_sum(s, s.max(), 1)
        n8 = n & ~7
        lanes = [np.float32(0)] * 8
        for i in range(n8):
            lanes[i % 8] = np.float32(lanes[i % 8] + e[i])
        x = [np.float32(lanes[k] + lanes[k + 4]) for k in range(4)]
        acc = np.float32(np.float32(x[0] + x[1]) + np.float32(x[2] + x[3]))
        if n8 != n:
            tail = np.float32(0)
            for i in range(n8, n):
                tail = np.float32(tail + e[i])
            acc = np.float32(acc + tail)
        assert acc == total


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("quant_q", [True, False])
@pytest.mark.parametrize("variant", [0, 1])
def test_attend_int8_vs_float64(causal, quant_q, variant):
    # TestAttendInt8MatchesFloat (int8_test.go:212-284)
    heads, kv_heads, qk, vd, n, rows = 8, 2, 48, 64, 37, 3
    g = synth.rng(9)
    q = g.standard_normal(rows * heads * qk).astype(np.float32)
    kq, ks = orc.quantize_rows(g.standard_normal(n * kv_heads * qk).astype(np.float32), kv_heads * qk, qk)
    vq, vs = orc.quantize_rows(g.standard_normal(n * kv_heads * vd).astype(np.float32), kv_heads * vd, vd)
    kf = (kq.astype(np.float32).reshape(n, kv_heads, qk) * ks.reshape(n, kv_heads, 1)).astype(np.float32)
    vf = (vq.astype(np.float32).reshape(n, kv_heads, vd) * vs.reshape(n, kv_heads, 1)).astype(np.float32)
    scale = np.float32(math.sqrt(qk))
    keys = [n - rows + i + 1 if causal else n for i in range(rows)]
    spans = np.array([[0, 0, 0, keys[i]] for i in range(rows)], np.int32)
    out, probs = orc.attend_int8_spans(q, rows, heads, kq, ks, kv_heads * qk, qk, vq, vs, kv_heads * vd, vd, n,
                                       spans, scale, quant_q, variant, want_probs=True)
    qq = q.copy()
    if quant_q:
        for c in range(rows * heads):
            qc, sc = orc.quantize_row(q[c * qk:(c + 1) * qk])
            qq[c * qk:(c + 1) * qk] = (qc.astype(np.float32) * sc).astype(np.float32)
    for i in range(rows):
        for h in range(heads):
            kv = h // (heads // kv_heads)
            qi = qq[(i * heads + h) * qk:(i * heads + h + 1) * qk].astype(np.float64)
            lg = kf[:keys[i], kv].astype(np.float64) @ qi / float(scale)
            p = np.exp(lg - lg.max())
            p /= p.sum()
            got_p = probs[(i * heads + h) * n:(i * heads + h) * n + keys[i]]
            assert np.max(np.abs(got_p - p)) <= 2e-6
            assert abs(got_p.astype(np.float64).sum() - 1) <= 1e-5
            want = p @ vf[:keys[i], kv].astype(np.float64)
            got = out[(i * heads + h) * vd:(i * heads + h + 1) * vd]
            assert np.max(np.abs(got - want)) <= 2e-6


def test_attend_int8_two_spans_are_the_union():
    # A sliding window with a sink (int8.go:202-207): spans [0, 2) and
    # [10, 30) see the same keys as one attention over those rows.
    heads, qk, vd, n = 4, 64, 64, 40
    g = synth.rng(13)
    q = g.standard_normal(heads * qk).astype(np.float32)
    kq, ks = orc.quantize_rows(g.standard_normal(n * heads * qk).astype(np.float32), heads * qk, qk)
    vq, vs = orc.quantize_rows(g.standard_normal(n * heads * vd).astype(np.float32), heads * vd, vd)
    two = orc.attend_int8_spans(q, 1, heads, kq, ks, heads * qk, qk, vq, vs, heads * vd, vd, n,
                                np.array([[0, 2, 10, 30]], np.int32), 8.0, True)
    sel = np.r_[0:2, 10:30]
    one = orc.attend_int8_spans(q, 1, heads, kq.reshape(n, -1)[sel].ravel(), ks.reshape(n, -1)[sel].ravel(),
                                heads * qk, qk, vq.reshape(n, -1)[sel].ravel(), vs.reshape(n, -1)[sel].ravel(),
                                heads * vd, vd, sel.size, np.array([[0, 0, 0, sel.size]], np.int32), 8.0, True)
    assert np.array_equal(one, two)
