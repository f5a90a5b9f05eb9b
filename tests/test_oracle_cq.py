"""Pins the CPU oracle's CQ part against checks that do not come from the
oracle itself: exhaustive and brute-force definitions, the explicit
Sylvester matrix, the float64 product within the reference's error bounds
(internal/cq/cq_test.go), and closed-form known answers for the lut
kernel's rounding, nibble order and group order."""

from fractions import Fraction

import numpy as np
import pytest

import go_whistle_amd as gw
from go_whistle_amd import synth
from helpers import TEST_SHAPES, cosine, dequant64, indices, lut_bound, rotated_bound, sylvester
from oracle import binding as orc


def test_f16_widen_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    got = np.zeros(65536, dtype=np.float32)
    orc.lib().orc_f16_to_f32_n(orc.fp(got), h.ctypes.data_as(orc.POINTER(orc.c_uint16)), 65536)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(got.view(np.uint32)[~nan], want.view(np.uint32)[~nan])
    # NaN keeps its payload shifted into the float32 mantissa (half.go:29-31)
    gb = got.view(np.uint32)[nan]
    assert np.all((gb & 0x7F800000) == 0x7F800000)
    assert np.array_equal((gb >> 13) & 0x3FF, h[nan] & 0x3FF)


@pytest.mark.parametrize("width", [2, 4])
def test_unpack_lsb_bruteforce(width):
    g = synth.rng(1)
    n = 256
    packed = g.integers(0, 256, size=n * width // 8, dtype=np.uint8)
    got = np.zeros(n, dtype=np.uint8)
    orc.lib().orc_unpack_lsb(orc.u8p(got), orc.u8p(packed), n, width)
    bits = np.unpackbits(packed, bitorder="little").reshape(n, width)
    want = (bits * (1 << np.arange(width))).sum(axis=1)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n", [1, 2, 8, 128, 1024])
def test_fwht_explicit_matrix(n):
    # TestFWHT (cq_test.go:613-640): small integers, so every sum is exact.
    g = synth.rng(n)
    x = (g.integers(0, 17, size=n) - 8).astype(np.float32)
    want = (sylvester(n) @ x.astype(np.float64)).astype(np.float32)
    assert np.array_equal(orc.fwht(x), want)


@pytest.mark.parametrize("shape", TEST_SHAPES)
@pytest.mark.parametrize("bits", [2, 4])
def test_row_and_dequant_vs_float64(shape, bits):
    out, inp, group = shape
    g = synth.rng(100 + out * 7 + bits)
    p = synth.random_packed(g, out, inp, group, bits)
    w64 = dequant64(p)
    m = orc.OMatrix.new(p)
    w = orc.dequant(p)
    for r in range(out):
        row = m.row(r)
        assert np.array_equal(row, w[r]), "Row must equal cact.CQ bit for bit"
        assert cosine(row, w64[r]) >= 0.9999999
        # |Δ| per element: G-1 FWHT adds over G terms each within γ
        tol = 2.0 ** -20 * np.abs(w64[r]).max() + 1e-30
        assert np.max(np.abs(row - w64[r])) <= tol


@pytest.mark.parametrize("shape", TEST_SHAPES)
@pytest.mark.parametrize("bits", [2, 4])
def test_kernels_vs_float64(shape, bits):
    # TestKernels (cq_test.go:196-254)
    out, inp, group = shape
    g = synth.rng(200 + out * 7 + bits)
    p = synth.random_packed(g, out, inp, group, bits)
    m = orc.OMatrix.new(p)
    w = dequant64(p)
    rows = 6
    x = synth.activations(g, rows, inp)
    for k in (orc.GATHER, orc.NIBBLE, orc.NIBBLE4, orc.LUT):
        got = m.gemm(x, rows, k).reshape(rows, out)
        for i in range(rows):
            xi = x[i * inp:(i + 1) * inp]
            bound = rotated_bound(p, xi)
            min_cos = 0.999999
            if k == orc.LUT:
                bound = bound + lut_bound(p, xi)
                min_cos = 0.99999
            want = w @ xi.astype(np.float64)
            d = np.abs(got[i].astype(np.float64) - want)
            assert np.all(d <= bound), (k, i, d.max(), bound[np.argmax(d)])
            assert cosine(got[i], want) >= min_cos


def test_gemm_rows_independent():
    # TestGEMMRows (cq_test.go:260-300)
    g = synth.rng(3)
    p = synth.random_packed(g, 33, 256, 128, 2)
    m = orc.OMatrix.new(p)
    rows = 4
    x = synth.activations(g, rows, 256).reshape(rows, 256)
    for k in (orc.LUT, orc.NIBBLE4, orc.NIBBLE):
        a = m.gemm(x, rows, k).reshape(rows, 33)
        b = m.gemm(x[::-1].copy(), rows, k).reshape(rows, 33)
        assert np.array_equal(a, b[::-1])
    one = m.gemm(x[0], 1, orc.LUT)
    assert np.array_equal(one, m.gemm(x, rows, orc.LUT)[:33])


@pytest.mark.parametrize("bits", [2, 4])
def test_rows_views_equal_slices(bits):
    # TestRow's view part and TestLUTKernelMatchesGeneric's views
    g = synth.rng(5 + bits)
    p = synth.random_packed(g, 70, 384, 128, bits)
    m = orc.OMatrix.new(p)
    x = synth.activations(g, 3, 384)
    for k in (orc.LUT, orc.NIBBLE4, orc.NIBBLE, orc.GATHER):
        full = m.gemm(x, 3, k).reshape(3, 70)
        for lo, hi in [(0, 70), (5, 40), (33, 70), (64, 66), (32, 32), (31, 33)]:
            v = m.rows(lo, hi)
            part = v.gemm(x, 3, k).reshape(3, hi - lo)
            assert np.array_equal(part, full[:, lo:hi]), (k, lo, hi)
            for r in range(lo, hi, 7):
                assert np.array_equal(v.row(r - lo), m.row(r))


def test_gemms_matches_gemm():
    # TestGEMMsMatchesGEMM (parallel_test.go:101-168)
    g = synth.rng(38)
    base = synth.random_packed(g, 384, 512, 128, 2)
    mats = []
    for out in (384, 96, 96, 384):
        p = synth.random_packed(g, out, 512, 128, 2)
        p.Codebook = base.Codebook
        mats.append(orc.OMatrix.new(p))
    for rows in (0, 1, 3, 37):
        x = synth.activations(g, rows, 512)
        got = orc.gemms(mats, x, rows)
        for m, y in zip(mats, got):
            assert np.array_equal(y, m.gemm(x, rows)) if rows else y.size == 0


def test_new_errors():
    # TestNewErrors (cq_test.go:561-585)
    g = synth.rng(7)
    good = synth.random_packed(g, 2, 128, 128, 2)

    def edit(**kw):
        q = gw.cq.Packed(**{**good.__dict__, **kw})
        with pytest.raises(orc.OracleError) as e:
            orc.OMatrix.new(q)
        return str(e.value)

    assert "not supported" in edit(Bits=3, Width=3)
    assert "not supported" in edit(Bits=5)
    assert "power of two" in edit(Group=24)
    assert "codebook" in edit(Codebook=good.Codebook[:3])
    assert "index" in edit(Index=good.Index[1:])
    assert "norm" in edit(Norms=good.Norms[2:])


# ---- closed-form known answers for the lut kernel --------------------------

ONE_F16 = np.array([0x3C00], dtype="<u2").view(np.uint8)  # FP16 1.0


def _packed(out, inp, group, bits, cb, index, norms):
    return gw.cq.Packed(Out=out, In=inp, Group=group, Bits=bits, Width=bits, Codebook=np.asarray(cb, np.float32),
                        Index=np.asarray(index, np.uint8), Norms=np.asarray(norms, np.uint8))


def _rne(v):
    """Round half to even of an exact rational: Python's round()."""
    return round(Fraction(float(v)))


def _find_tie(a, cb_max=1.0):
    """A float32 codebook level c in (0, cb_max) with c*a an exact tie
    2m + 0.5 (even m): round half to even and half away differ there."""
    a = np.float32(a)
    for m in range(1000, 4000):
        c = np.float32((2 * m + 0.5) / float(a))
        if c < cb_max and np.float32(c * a) == np.float32(2 * m + 0.5):
            return c
    raise AssertionError("no tie found")


def test_lut4_ties_round_half_even_and_planes():
    # x = e0 in one group of 8: x̂ = all ones, M = cbMax = 1, a = 8191.
    tie = _find_tie(8191.0)
    cb = np.sort(np.array([-1, -tie, -0.5, -0.25, -0.125, 0, 0.03, 0.06, 0.125, 0.25, 0.3, 0.5, 0.6, 0.7, tie, 1],
                          dtype=np.float32))
    code = int(np.nonzero(cb == tie)[0][0])
    ncode = int(np.nonzero(cb == -tie)[0][0])
    x = np.zeros(8, np.float32)
    x[0] = 1
    lut_step = np.float32(1 / (8191 * np.sqrt(8.0)))
    for c, sign in ((code, 1), (ncode, -1)):
        index = np.full(4, c | (c << 4), np.uint8)  # every nibble = c
        m = orc.OMatrix.new(_packed(1, 8, 8, 4, cb, index, ONE_F16))
        e = np.float32(cb[c] * np.float32(8191))
        v = _rne(e)
        assert abs(float(e)) % 2 == 0.5 and abs(v) % 2 == 0  # a tie, rounded to the even neighbour
        s = 8 * v
        step = np.float32(np.float32(1) * lut_step)
        coef = np.float32(np.float32(1) * step)
        want = np.float32(np.float32(0) + np.float32(np.float32(s) * coef))
        got = m.gemm(x, 1, orc.LUT)
        assert got.view(np.uint32)[0] == want.view(np.uint32), (c, got, want)


def test_lut2_ties_round_half_even():
    # 2 bits: pair tables cb[lo]*a + cb[hi]*b, x = e0: x̂ = all ones,
    # M = cbMax * 2, a = b = 8191/2.
    a = np.float32(np.float32(8191) / np.float32(2))
    half = None
    for m in range(500, 2000, 2):  # c*a = m + 1/4 with m even: the pair sum 2m + 1/2 is a tie
        c = np.float32((m + 0.25) / float(a))
        if np.float32(c * a) == np.float32(m + 0.25):
            half = c
            break
    assert half is not None
    cb = np.sort(np.array([-1, 0, half, 1], dtype=np.float32))
    c = int(np.nonzero(cb == half)[0][0])
    code = c | (c << 2)  # both indices of the pair address `half`
    e = np.float32(np.float32(half * a) + np.float32(half * a))
    v = _rne(e)
    assert float(e) - int(np.floor(float(e))) == 0.5 and v % 2 == 0
    x = np.zeros(8, np.float32)
    x[0] = 1
    index = np.full(2, code | (code << 4), np.uint8)
    m = orc.OMatrix.new(_packed(1, 8, 8, 2, cb, index, ONE_F16))
    lut_step = np.float32(1 / (8191 * np.sqrt(8.0)))
    step = np.float32(np.float32(2) * lut_step)
    want = np.float32(np.float32(4 * v) * np.float32(np.float32(1) * step))
    got = m.gemm(x, 1, orc.LUT)
    assert got.view(np.uint32)[0] == want.view(np.uint32)


@pytest.mark.parametrize("bits", [2, 4])
def test_lut_index_order_lsb_first(bits):
    # x = all ones: x̂ = (8, 0, ..., 0), so only index position 0 has a
    # non-zero table; position 0 is the low nibble (4 bits) or the low crumb
    # (2 bits) of byte 0 (matrix.go:185-189).
    cb = np.sort(np.array([-0.9, -0.3, 0.2, 1.0] if bits == 2 else np.linspace(-1, 1, 16), dtype=np.float32))
    x = np.ones(8, np.float32)
    first, other = 1, 2
    if bits == 4:
        index = np.array([first | (other << 4), other | (other << 4), 0x22, 0x22], np.uint8)
    else:
        index = np.array([first | (other << 2) | (other << 4) | (other << 6), 0xAA], np.uint8)
    m = orc.OMatrix.new(_packed(1, 8, 8, bits, cb, index, ONE_F16))
    cb_max = np.float32(np.abs(cb).max())
    mx = np.float32(8)
    mm = np.float32(cb_max * mx)
    inv = np.float32(np.float32(8191) / mm)
    av = np.float32(np.float32(8) * inv)
    if bits == 4:
        e = np.float32(cb[first] * av)
    else:  # pair (x̂0, x̂1) = (8, 0): code = other<<2 | first
        e = np.float32(np.float32(cb[first] * av) + np.float32(cb[other] * np.float32(0)))
    s = _rne(e)
    step = np.float32(mm * np.float32(1 / (8191 * np.sqrt(8.0))))
    want = np.float32(np.float32(s) * np.float32(np.float32(1) * step))
    got = m.gemm(x, 1, orc.LUT)
    assert got.view(np.uint32)[0] == want.view(np.uint32)


def test_lut_groups_accumulate_in_order():
    # Three groups of 8; group g's x is s_g * ones, so x̂_g = (8 s_g, 0, ...)
    # and the group's integer sum is v(code at position 0) = 8191 for the
    # level cbMax. Group 0's product is large and groups 1, 2 are each 0.3
    # of its ulp: ascending order (lut.go:297-310) absorbs them, the
    # reverse order would not.
    cb = np.sort(np.array([-1, -0.5, 0.5, 1], dtype=np.float32))
    top = 3  # cb[3] = 1 = cbMax
    x = np.concatenate([np.full(8, s, np.float32) for s in (1.0, 2.0 ** -25, 2.0 ** -25)])
    index = np.zeros(3 * 2, np.uint8)
    for g in range(3):
        index[2 * g] = top | (0 << 2)  # position 0 of group g: code `top`, pair partner 0
    # 2 bits: pairs (x̂0, x̂1) = (8 s, 0); the pair code is hi<<2 | lo with lo = top
    norms = np.array([0x3C00] * 3, dtype="<u2").view(np.uint8)
    m = orc.OMatrix.new(_packed(1, 24, 8, 2, cb, index, norms))
    lut_step = np.float32(1 / (8191 * np.sqrt(8.0)))
    prods = []
    for g, s in enumerate((1.0, 2.0 ** -25, 2.0 ** -25)):
        mx = np.float32(np.float32(8 * s))  # |x̂0| + |x̂1|
        mm = np.float32(np.float32(1) * mx)
        inv = np.float32(np.float32(8191) / mm)
        av = np.float32(np.float32(8 * s) * inv)
        # pair tables of group g: position 0 (code top | cb[0]*0), other pairs 0;
        # the row's other three pair nibbles hit code 0 of zero tables
        e0 = np.float32(np.float32(cb[top] * av) + np.float32(cb[0] * np.float32(0)))
        v0 = _rne(e0)
        ssum = v0  # the remaining 3 nibbles of the group address zero tables
        step = np.float32(mm * lut_step)
        prods.append(np.float32(np.float32(ssum) * np.float32(np.float32(1) * step)))
    asc = np.float32(0)
    for p_ in prods:
        asc = np.float32(asc + p_)
    desc = np.float32(0)
    for p_ in prods[::-1]:
        desc = np.float32(desc + p_)
    assert asc != desc, "the case must tell the orders apart"
    got = m.gemm(x, 1, orc.LUT)
    assert got.view(np.uint32)[0] == asc.view(np.uint32)


def test_lut_tables_byte_planes():
    # lutPut (lut.go:229-233): lo = v & 127, hi = v>>7 + 64, both in [0, 127],
    # and 128*(hi-64) + lo = v for every entry of random tables.
    g = synth.rng(23)
    for bits in (2, 4):
        for n in (8, 16, 128, 256):
            cb = np.sort(g.standard_normal(1 << bits).astype(np.float32))
            cb_max = np.float32(np.abs(cb).max())
            x = synth.heavy_vector(g, n)
            size = 32 * n * bits // 4
            tab = np.full(size + 4, 0xAA, np.uint8)
            f = orc.lib().orc_lut_tables2 if bits == 2 else orc.lib().orc_lut_tables4
            mm = f(orc.u8p(tab), orc.fp(x), n, orc.fp(cb), cb_max)
            assert np.all(tab[size:] == 0xAA), "bytes past the tables untouched"
            t = tab[:size].reshape(-1, 2, 16).astype(np.int64)
            assert t.max() <= 127 and t.min() >= 0
            v = 128 * (t[:, 1] - 64) + t[:, 0]
            # each entry within half a step of its exact value
            if bits == 4:
                exact = np.outer(x.astype(np.float64), cb.astype(np.float64))
            else:
                xa, xb = x[0::2].astype(np.float64), x[1::2].astype(np.float64)
                codes = np.arange(16)
                exact = np.outer(xa, cb[codes & 3]) + np.outer(xb, cb[codes >> 2])
            scale = 8191 / float(mm) if mm > 0 else 0
            assert np.all(np.abs(v - exact * scale) <= 0.5 + 1e-3 * np.abs(exact * scale) + 1e-6)
            assert np.abs(v).max() <= 8191


def _f32_of_exact(q):
    """float32 nearest (ties to even) to an exact rational."""
    q = Fraction(q)
    f = np.float32(float(q))  # may double-round: step to the true nearest
    best = f
    for cand in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        d, db = abs(Fraction(float(cand)) - q), abs(Fraction(float(best)) - q)
        if d < db or (d == db and (cand.view(np.uint32) & 1) == 0 and cand != best):
            best = cand
    return np.float32(best)


def test_lut_accumulate_is_unfused():
    # Two groups of 8 (4 bits), x̂_g = (8 s_g, 0, ...) so S_g = v(cbMax) =
    # 8191. y = (0 + S0*c0) + S1*c1 with each product rounded (Go on amd64
    # never fuses): find a group-1 scale where a fused multiply-add would
    # round differently, and require the unfused result.
    cb = np.linspace(-1, 1, 16).astype(np.float32)
    top = 15
    lut_step = np.float32(1 / (8191 * np.sqrt(8.0)))
    norms = np.array([0x3C00, 0x3C00], dtype="<u2").view(np.uint8)
    index = np.array([top, 0, 0, 0, top, 0, 0, 0], np.uint8)
    g = synth.rng(99)
    for _ in range(2000):
        s1 = np.float32(g.uniform(0.3, 0.9))
        prods, coefs = [], []
        for s in (np.float32(1), s1):
            mm = np.float32(np.float32(1) * np.float32(np.float32(8) * s))
            inv = np.float32(np.float32(8191) / mm)
            v = _rne(np.float32(cb[top] * np.float32(np.float32(8) * s * inv)))
            coef = np.float32(np.float32(1) * np.float32(mm * lut_step))
            coefs.append((v, coef))
            prods.append(np.float32(np.float32(v) * coef))
        y0 = np.float32(np.float32(0) + prods[0])
        unfused = np.float32(y0 + prods[1])
        fused = _f32_of_exact(Fraction(float(y0)) + Fraction(coefs[1][0]) * Fraction(float(coefs[1][1])))
        if fused != unfused:
            break
    else:
        raise AssertionError("no discriminating case")
    x = np.concatenate([np.full(8, 1, np.float32), np.full(8, s1, np.float32)])
    m = orc.OMatrix.new(_packed(1, 16, 8, 4, cb, index, norms))
    got = m.gemm(x, 1, orc.LUT)
    assert got.view(np.uint32)[0] == unfused.view(np.uint32)


def test_lut2_table_entry_is_unfused():
    # A 2-bit entry is RNE(float32(cb[lo]*a) + float32(cb[hi]*b)) (lut.go:253);
    # find a pair where fusing either product would move the rounded entry.
    g = synth.rng(7)
    cb = np.sort(g.standard_normal(4).astype(np.float32))
    cb_max = np.float32(np.abs(cb).max())
    for _ in range(20000):
        x = g.standard_normal(8).astype(np.float32)
        xh = orc.fwht(x)
        mx = np.float32(0)
        for q in range(0, 8, 2):
            mx = max(mx, np.float32(abs(xh[q]) + abs(xh[q + 1])))
        mm = np.float32(cb_max * mx)
        inv = np.float32(np.float32(8191) / mm)
        a, b = np.float32(xh[0] * inv), np.float32(xh[1] * inv)
        hit = None
        for c in range(16):
            lo, hi = np.float32(cb[c & 3] * a), np.float32(cb[c >> 2] * b)
            unfused = np.float32(lo + hi)
            f1 = _f32_of_exact(Fraction(float(cb[c & 3])) * Fraction(float(a)) + Fraction(float(hi)))
            f2 = _f32_of_exact(Fraction(float(lo)) + Fraction(float(cb[c >> 2])) * Fraction(float(b)))
            if _rne(unfused) != _rne(f1) or _rne(unfused) != _rne(f2):
                hit = (c, _rne(unfused))
                break
        if hit:
            break
    else:
        raise AssertionError("no discriminating case")
    tab = np.zeros(32 * 4, np.uint8)
    orc.lib().orc_lut_tables2(orc.u8p(tab), orc.fp(xh), 8, orc.fp(cb), cb_max)
    c, v = hit
    assert 128 * (int(tab[16 + c]) - 64) + int(tab[c]) == v


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("special", ["nan", "inf"])
def test_lut_nan_or_inf_input_gives_nan_rows(bits, special):
    # lutTables{2,4}Generic (lut.go:239-282) reduce the group bound with Go's
    # max, which keeps a NaN: a group holding one has M = NaN, lutInv gives 0
    # (NaN > 0 fails) and the step is NaN, so every row's y is NaN. +Inf
    # spreads through the rotation to every value of its group: M = Inf,
    # lutInv 8191/Inf = 0, each entry Inf * 0 = NaN (an integer of 0 after
    # lutPut), the step Inf and y = 0 * Inf = NaN. (The amd64 kernel's
    # VMAXPS keeps or drops a NaN depending on its lane and chunk, an
    # artefact; arm64's FMAX keeps it, as the generic Go does.)
    g = synth.rng(bits)
    p = synth.random_packed(g, 70, 384, 128, bits, sigma=0.05)
    m = orc.OMatrix.new(p)
    x = g.standard_normal(384).astype(np.float32)
    x[200] = np.float32(special)
    y = m.gemm(x, 1, orc.LUT)
    assert np.isnan(y).all()
    x[200] = 1.0
    assert np.isfinite(m.gemm(x, 1, orc.LUT)).all()
