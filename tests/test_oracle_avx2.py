"""The oracle's AVX2 form of the lut kernel (the reference's amd64 path,
internal/cq/lut_amd64.s) against the generic restatement, bit for bit, as
the reference's internal/cq/asm_test.go holds its assembly to the Go code;
and the products split over threads as gemmLUT splits them (lut.go:102-201)
against the serial ones, bit for bit, as parallel_test.go:45-168 holds them;
and the AVX2 forms of the int8 attention kernels (int8kernel_amd64.s,
exp_amd64.s) against the generic ones. The AVX2 forms and the threads are
what bench.py's CPU baseline times."""

import numpy as np
import pytest

from go_whistle_amd import synth
from oracle import binding as orc

pytestmark = pytest.mark.skipif(not orc.have_avx2(), reason="this CPU has no AVX2")


@pytest.fixture(autouse=True)
def _serial_generic():
    yield
    orc.set_cpu(False, 1)


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("n", [8, 16, 32, 64, 128, 256, 1024])
def test_fwht(n):
    g = synth.rng(n)
    x = (g.standard_normal(n) * 10).astype(np.float32)
    assert same(orc.fwht(x, avx2=True), orc.fwht(x))


@pytest.mark.parametrize("width", [2, 4])
@pytest.mark.parametrize("n", [8, 32, 128, 512])
def test_tables(width, n):
    g = synth.rng(10 * n + width)
    cb = np.sort(g.standard_normal(1 << width) * 0.05).astype(np.float32)
    cb_max = np.float32(np.abs(cb).max())
    for x in (g.standard_normal(n).astype(np.float32), (g.standard_normal(n) ** 3).astype(np.float32),
              np.zeros(n, np.float32)):
        t0, m0 = orc.lut_tables(x, cb, cb_max, width)
        t1, m1 = orc.lut_tables(x, cb, cb_max, width, avx2=True)
        assert np.array_equal(t0, t1) and same(m0, m1)


def test_tables_half_way_entries():
    # entries exactly half-way between integers round to even in both forms
    cb = np.array([0.5, -1.5, 2.5, -3.5] + [k + 0.5 for k in range(4, 16)], np.float32)
    x = np.zeros(8, np.float32)
    x[0] = 1.0  # with cbMax 8191: M = 8191, inv = 1, a = 1, so entry c of table 0 is cb[c] itself
    t0, _ = orc.lut_tables(x, cb, np.float32(8191), 4)
    t1, _ = orc.lut_tables(x, cb, np.float32(8191), 4, avx2=True)
    assert np.array_equal(t0, t1)
    v = np.array([0, -2, 2, -4] + [k if k % 2 == 0 else k + 1 for k in range(4, 16)])  # ties to even
    assert np.array_equal(t1[:16], v & 127) and np.array_equal(t1[16:32], (v >> 7) + 64)


@pytest.mark.parametrize("gb", [4, 8, 16, 32, 64, 128, 256])
def test_lookup(gb):
    g = synth.rng(gb)
    groups, blocks = 3, 2
    idx = g.integers(0, 256, size=blocks * groups * gb * 32, dtype=np.uint8)
    # tables as lutPut writes them: lo plane v & 127, hi plane (v >> 7) + 64
    v = g.integers(-8191, 8192, size=(groups * gb * 2, 16))
    tab = np.concatenate([np.concatenate([(t & 127), (t >> 7) + 64]) for t in v]).astype(np.uint8)
    norm = (2.0 ** g.uniform(-4, 4, size=blocks * groups * 32)).astype(np.float32)
    steps = (g.random(groups) * 1e-3).astype(np.float32)
    y0 = orc.lut_lookup(idx, tab, norm, steps, blocks, groups, gb)
    y1 = orc.lut_lookup(idx, tab, norm, steps, blocks, groups, gb, avx2=True)
    assert same(y0, y1)


def _products(ms, xs, rows):
    return [m.gemm(x, rows) for m, x in zip(ms, xs)]


@pytest.mark.parametrize("bits", [4, 2])
def test_gemv_sweep_avx2_and_threads(bits):
    # the sweep's shapes at batch 1: 2048x512, 512x2048 and 16384x512 split
    # their blocks over threads (>= 2 * 2^18 index bytes), 512x512 does not
    g = synth.rng(70 + bits)
    packs = [synth.random_packed(g, o, i, 128, bits, sigma=0.05)
             for o, i in [(512, 512), (2048, 512), (512, 2048), (16384, 512)]]
    ms = [orc.OMatrix.new(p) for p in packs]
    xs = [synth.activations(g, 1, p.In) for p in packs]
    want = _products(ms, xs, 1)
    for avx2, threads in ((True, 1), (False, 8), (True, 8), (True, 3)):
        orc.set_cpu(avx2, threads)
        for a, b in zip(_products(ms, xs, 1), want):
            assert same(a, b)


@pytest.mark.parametrize("rows", [2, 5, 16])
def test_gemm_activation_split(rows):
    # several activations split over threads (or, with fewer rows than
    # threads, a large product's blocks), on a Rows view and with GEMMs
    g = synth.rng(90 + rows)
    p = synth.random_packed(g, 1000, 640, 128, 4, sigma=0.05)
    m = orc.OMatrix.new(p)
    v = m.rows(37, 911)
    x = synth.activations(g, rows, 640)
    want = [m.gemm(x, rows), v.gemm(x, rows), orc.gemms([m, v], x, rows)]
    for threads in (2, 8):
        orc.set_cpu(True, threads)
        got = [m.gemm(x, rows), v.gemm(x, rows), orc.gemms([m, v], x, rows)]
        assert same(got[0], want[0]) and same(got[1], want[1])
        assert all(same(a, b) for a, b in zip(got[2], want[2]))


@pytest.mark.parametrize("width,n", [(16, 1), (64, 37), (128, 300), (48, 9)])
def test_dots_and_axpys_i8(width, n):
    # dotsI8 / axpysI8 AVX2 forms (int8kernel_amd64.s) against the generic
    # loops; stride wider than the row, as in a multi-head cache
    g = synth.rng(width + n)
    stride = width * 3
    q = g.integers(-128, 128, size=width, dtype=np.int8)
    k = g.integers(-128, 128, size=n * stride, dtype=np.int8)
    assert np.array_equal(orc.dots_i8(q, k, n, stride, avx2=True), orc.dots_i8(q, k, n, stride))
    out = g.standard_normal(width).astype(np.float32)
    w = (g.random(n) * 1e-2).astype(np.float32)
    assert same(orc.axpys_i8(out, w, k, stride, avx2=True), orc.axpys_i8(out, w, k, stride))


@pytest.mark.parametrize("n", [8, 64, 1504])
def test_exp_sub_sum(n):
    # expSubSumAVX2 against the lane-by-lane restatement (variant 1); the
    # inputs reach below the -87.33 flush and include the maximum itself
    g = synth.rng(n)
    s = (g.standard_normal(n) * 30).astype(np.float32)
    m = np.float32(s.max())
    e0, t0 = orc.exp_sub_sum(s, m, 1)
    e1, t1 = orc.exp_sub_sum_avx2(s, m)
    assert same(e0, e1) and same(t0, t1)


@pytest.mark.parametrize("quant_q", [True, False])
def test_attend_int8_avx2_mode(quant_q):
    # AttendInt8Spans in the AVX2 mode equals the generic run bit for bit:
    # cross attention over 1500 keys and a two-span self-attention band
    g = synth.rng(5 if quant_q else 6)
    heads, qk, nk = 8, 64, 1500
    cols = heads * qk
    q = g.standard_normal(2 * cols).astype(np.float32)
    kq = g.integers(-128, 128, size=nk * cols, dtype=np.int8)
    vq = g.integers(-128, 128, size=nk * cols, dtype=np.int8)
    ks = (g.random(nk * heads) * 0.05 + 1e-3).astype(np.float32)
    vs = (g.random(nk * heads) * 0.05 + 1e-3).astype(np.float32)
    spans = np.array([[0, 0, 0, nk], [0, 4, 600, 1203]], np.int32)
    args = (q, 2, heads, kq, ks, cols, qk, vq, vs, cols, qk, nk, spans, np.float32(8.0), quant_q)
    want = orc.attend_int8_spans(*args)
    orc.set_cpu(True, 1)
    assert same(orc.attend_int8_spans(*args), want)
