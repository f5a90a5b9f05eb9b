"""GPU parity of Dense views (cq_dense), the dense fp32 MFMA form of Exact's
semantics, through the C ABI.

Two checks per case:
- against the oracle's Exact GEMM (nibble and nibble4 kernels,
  internal/cq/kernel.go:160-374): per activation, max |y - exact| <= 1e-5 *
  max |exact| (the relative tolerance the batched path is held to), the
  max over the whole matrix's outputs for that activation (a Rows view of
  one row would otherwise hold a single output, near zero where its sum
  cancels);
- against the product computed in float64 from the same rotated inputs
  (rotate's float32 values, kernel.go:203-217) and dequantized weights
  norm * codebook[index]: per output element |y - y64| <= (K + 2) * 2^-24 *
  sum_k |w_k * xh_k|, the worst-case bound of a float32 dot product of K
  terms in any summation order plus one rounding of each weight, so a
  dropped term, a wrong index or a transposed operand fails it whatever
  order the MFMA sums in.
Covers the encoder's batched shapes (2048x512 and 512x2048 at 2 and 4 bits,
375 / 1500 / 12000 activations, the last sampled: each activation's product
is independent of the others), ragged activation counts, Rows views that
start and end mid-block, groups of 32 to 1024 with padded inputs, GEMMs over
shared inputs (one rotation), mixed GEMMs of Dense and lut views, and the
nibble fallback under 16 activations and outside groups 32..1024 (bit for
bit Exact), and NaN and Inf activations (non-finite outputs for those, the
bars for the activations that share their tiles)."""

import numpy as np
import pytest

import go_whistle_amd as gw
from go_whistle_amd import cq, synth
from oracle import binding as orc

pytestmark = pytest.mark.gpu

REL = 1e-5  # relative tolerance against Exact, per activation


def dense_gemm(m, x, rows):
    import torch

    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32).reshape(rows, -1)).cuda()
    y = torch.full((rows, m.Out()), np.nan, dtype=torch.float32, device="cuda")
    m.gemm_dev(y, xd, rows)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def rotated(x, inp, group):
    """rotate's float32 values: zero-padded to groups*G, FWHT stages h = 1,
    2, ..., G/2 (each butterfly one float32 add and subtract), times the
    float32 1/sqrt(G)."""
    rows = x.shape[0]
    groups = (inp + group - 1) // group
    xh = np.zeros((rows, groups * group), np.float32)
    xh[:, :inp] = x
    v = xh.reshape(rows, groups, group)
    h = 1
    while h < group:
        b = v.reshape(rows, groups, group // (2 * h), 2, h)
        u, w = b[:, :, :, 0, :].copy(), b[:, :, :, 1, :].copy()
        b[:, :, :, 0, :] = u + w
        b[:, :, :, 1, :] = u - w
        h *= 2
    return xh * np.float32(1.0 / np.sqrt(group))


def weights64(p):
    """norm[r][k / G] * codebook[index(r, k)] in float64 (LSB-first codes)."""
    groups = (p.In + p.Group - 1) // p.Group
    kin = groups * p.Group
    idx = np.frombuffer(bytes(p.Index), np.uint8).reshape(p.Out, -1)
    per = 8 // p.Width
    codes = np.zeros((p.Out, kin), np.int64)
    for s in range(per):
        codes[:, s::per] = (idx >> (p.Width * s)) & ((1 << p.Width) - 1)
    norms = np.frombuffer(bytes(p.Norms), "<u2").view(np.float16).astype(np.float64).reshape(p.Out, groups)
    cb = np.asarray(p.Codebook, np.float64)
    return cb[codes] * np.repeat(norms, p.Group, axis=1)


def check(got, x, p, o, pick, lo=0, hi=None, full=None):
    """got [len(pick)][hi - lo] against Exact and the float64 bound for
    activations `pick` of x and rows [lo, hi) (o is the oracle's view of
    those rows, full its whole matrix when o is a view)."""
    hi = p.Out if hi is None else hi
    xs = x[pick]
    want = o.gemm(xs.ravel(), len(pick), orc.NIBBLE4).reshape(len(pick), -1)
    whole = want if full is None else full.gemm(xs.ravel(), len(pick), orc.NIBBLE4).reshape(len(pick), -1)
    assert np.all(np.isfinite(got)), "unwritten outputs"
    err = np.abs(got - want).max(axis=1)
    scale = np.abs(whole).max(axis=1)
    assert np.all(err <= REL * scale), (float((err / scale).max()), int(np.argmax(err / scale)))
    xh = rotated(xs, p.In, p.Group).astype(np.float64)
    w = weights64(p)[lo:hi]
    y64 = xh @ w.T
    bound = (xh.shape[1] + 2) * 2.0**-24 * (np.abs(xh) @ np.abs(w).T)
    assert np.all(np.abs(got - y64) <= bound), float((np.abs(got - y64) / bound).max())


@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("shape", [(2048, 512), (512, 2048)])
@pytest.mark.parametrize("rows", [375, 1500])
def test_dense_encoder_shapes(bits, shape, rows):
    out, inp = shape
    g = synth.rng(rows * 7 + bits + out)
    p = synth.random_packed(g, out, inp, 128, bits, sigma=0.05)
    m, o = cq.New(p).Dense(), orc.OMatrix.new(p)
    assert m.gemm_path(rows) == "dense-f32" and m.Kernel() == "dense-f32"
    x = g.standard_normal((rows, inp)).astype(np.float32)
    got = dense_gemm(m, x, rows)
    pick = np.arange(rows) if rows <= 375 else np.sort(g.choice(rows, size=96, replace=False))
    check(got[pick], x, p, o, pick)


@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("shape", [(2048, 512), (512, 2048)])
def test_dense_12000_frames_sampled(bits, shape):
    out, inp = shape
    rows = 12000
    g = synth.rng(12000 + bits + out)
    p = synth.random_packed(g, out, inp, 128, bits, sigma=0.05)
    m, o = cq.New(p).Dense(), orc.OMatrix.new(p)
    x = g.standard_normal((rows, inp)).astype(np.float32)
    got = dense_gemm(m, x, rows)
    pick = np.sort(g.choice(rows, size=40, replace=False))
    pick[0], pick[-1] = 0, rows - 1
    check(got[pick], x, p, o, pick)


@pytest.mark.parametrize(
    "out,inp,group,bits,rows",
    [
        (200, 300, 32, 4, 131),  # 10 groups of 32: K = 320, not a multiple of 64; inputs padded
        (70, 96, 32, 2, 17),  # 3 groups of 32 at 2 bits; one partial row tile
        (333, 640, 64, 4, 129),  # two activation tiles, the second of one activation
        (129, 1000, 256, 2, 250),  # 4 groups of 256, 24 padded inputs
        (64, 512, 128, 4, 16),  # the smallest activation count of the form
        (1536, 512, 128, 2, 300),
        (100, 2048, 1024, 4, 40),  # the largest group of the form
        (90, 3000, 512, 2, 33),  # 6 groups of 512, 72 padded inputs
    ],
)
def test_dense_ragged_geometries(out, inp, group, bits, rows):
    g = synth.rng(out * 31 + inp + rows)
    p = synth.random_packed(g, out, inp, group, bits, sigma=0.05)
    m, o = cq.New(p).Dense(), orc.OMatrix.new(p)
    assert m.gemm_path(rows) == "dense-f32"
    x = g.standard_normal((rows, inp)).astype(np.float32)
    got = dense_gemm(m, x, rows)
    check(got, x, p, o, np.arange(rows))


@pytest.mark.parametrize("lo,hi", [(37, 301), (64, 192), (0, 1), (511, 512), (100, 100 + 130)])
def test_dense_rows_views(lo, hi):
    g = synth.rng(lo * 1000 + hi)
    p = synth.random_packed(g, 512, 512, 128, 4, sigma=0.05)
    m, o = cq.New(p), orc.OMatrix.new(p)
    rows = 200
    x = g.standard_normal((rows, 512)).astype(np.float32)
    for v in (m.Dense().Rows(lo, hi), m.Rows(lo, hi).Dense()):
        assert v.Out() == hi - lo and v.gemm_path(rows) == "dense-f32"
        got = dense_gemm(v, x, rows)
        check(got, x, p, o.rows(lo, hi), np.arange(rows), lo, hi, full=o)
    assert m.Dense().Exact().gemm_path(rows) == "nibble4"


def test_dense_gemms_shared_input_and_mixed():
    import torch

    g = synth.rng(77)
    ps = [synth.random_packed(g, out, 512, 128, 4, sigma=0.05) for out in (512, 128, 320)]
    ps.append(synth.random_packed(g, 256, 512, 128, 2, sigma=0.05))
    ms = [cq.New(p) for p in ps]
    os_ = [orc.OMatrix.new(p) for p in ps]
    rows = 300
    x = g.standard_normal((rows, 512)).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    # three Dense views on one input, then a lut view between Dense ones
    for views in ([m.Dense() for m in ms], [ms[0].Dense(), ms[1], ms[2].Dense(), ms[3].Dense()]):
        ys = [torch.full((rows, v.Out()), np.nan, device="cuda") for v in views]
        cq.gemms_dev(views, ys, xd, rows)
        torch.cuda.synchronize()
        for v, p, o, y in zip(views, ps, os_, ys):
            got = y.cpu().numpy()
            if v.Kernel() == "dense-f32":
                check(got, x, p, o, np.arange(rows))
            else:
                want = o.gemm(x.ravel(), rows, orc.LUT).reshape(rows, -1)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows", [1, 3, 4, 9, 15])
def test_dense_few_activations_run_exact(rows):
    # under 16 activations a Dense view runs Exact's nibble kernels: Exact's bits
    g = synth.rng(rows + 500)
    p = synth.random_packed(g, 300, 512, 128, 4, sigma=0.05)
    m, o = cq.New(p).Dense(), orc.OMatrix.new(p)
    assert m.gemm_path(rows) == "nibble4"
    x = g.standard_normal((rows, 512)).astype(np.float32)
    got = dense_gemm(m, x, rows)
    want = o.gemm(x.ravel(), rows, orc.NIBBLE4).reshape(rows, -1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dense_small_groups_and_misuse():
    import torch

    g = synth.rng(5)
    # outside 32..1024: the nibble kernels (which take up to 512 group bytes)
    for group, inp, bits in ((16, 256, 4), (2048, 2048, 2)):
        p = synth.random_packed(g, 128, inp, group, bits, sigma=0.05)
        m, o = cq.New(p).Dense(), orc.OMatrix.new(p)
        assert m.gemm_path(200) == "nibble4"
        x = g.standard_normal((200, inp)).astype(np.float32)
        got = dense_gemm(m, x, 200)
        want = o.gemm(x.ravel(), 200, orc.NIBBLE4).reshape(200, -1)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    z = torch.zeros(16, device="cuda")
    with pytest.raises(gw.CQPanic):
        m.gemm_dev(z, z, -1)
    with pytest.raises(gw.CQDeviceError):  # fused products run the lut kernel
        cq.gemms_fused_dev([cq.New(synth.random_packed(g, 128, 256, 128, 4)).Dense()], [z], z, 32, norm_gain=z)


def test_dense_non_finite_activations():
    # NaN and +-Inf activations (in both 128-activation tiles): the rotation
    # spreads them over their group, so every output of that activation is
    # non-finite, as in Exact (whose NaN and Inf may fall differently: the
    # sums run in another order); the activations beside them in the same
    # tiles keep the bar
    g = synth.rng(91)
    p = synth.random_packed(g, 512, 512, 128, 4, sigma=0.05)
    m, o = cq.New(p).Dense(), orc.OMatrix.new(p)
    rows = 200
    x = g.standard_normal((rows, 512)).astype(np.float32)
    bad = {3: (10, np.nan), 70: (300, np.inf), 150: (0, -np.inf), 199: (511, np.nan)}
    for t, (k, v) in bad.items():
        x[t, k] = v
    got = dense_gemm(m, x, rows)
    want = o.gemm(x.ravel(), rows, orc.NIBBLE4).reshape(rows, -1)
    for t in bad:
        assert not np.isfinite(got[t]).any() and not np.isfinite(want[t]).any(), t
    good = np.array([t for t in range(rows) if t not in bad])
    check(got[good], x, p, o, good)
