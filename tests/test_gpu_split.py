"""The MFMA form split over groups (lut_mfma_split_kernel, then the fold in
group order), through the C ABI: products at some hundreds of activations
(the encoder's 375 and 1500 frames), bit for bit the oracle's lut product
(internal/cq/lut.go), with row views, several matrices on one input,
activations that do not fill a 32-wide tile, and every fused prologue and
epilogue."""

import numpy as np
import pytest

from go_whistle_amd import cq, synth
from go_whistle_amd._lib import check, lib
from oracle import binding as orc

pytestmark = pytest.mark.gpu


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("out,inp,rows", [(512, 512, 375), (2048, 512, 375), (512, 2048, 375), (512, 2048, 1500),
                                          (700, 384, 333), (512, 512, 1000), (512, 2048, 100)])
def test_split_gemm_bit_exact(bits, out, inp, rows):
    import torch

    g = synth.rng(out + inp + rows + bits)
    p = synth.random_packed(g, out, inp, 128, bits, sigma=0.05)
    m = cq.New(p)
    x = (g.standard_normal((rows, inp)) * 2).astype(np.float32)
    y = torch.full((rows, out), float("nan"), device="cuda")
    m.gemm_dev(y, _t(x), rows)
    torch.cuda.synchronize()
    path = m.gemm_path(rows)
    want = orc.OMatrix.new(p).gemm(x.reshape(-1), rows, orc.LUT).reshape(rows, out)
    assert same(y.cpu().numpy(), want), path
    if (out, inp, rows) == (512, 2048, 375) and bits == 4:
        assert path == "lut-mfma-split"
    if (out, inp, rows) == (2048, 512, 375):
        assert path == "lut-mfma-tab"  # enough (block, tile) workgroups for the table form
    if rows == 100:
        assert path == "lut"


@pytest.mark.parametrize("bits", [2, 4])
def test_split_views_and_shared_input(bits):
    # four row views of one root (two of them not block-aligned) on one
    # input, 400 activations: one split launch, each output bit for bit its
    # own oracle product
    import torch

    g = synth.rng(70 + bits)
    D, rows = 512, 400
    proot = synth.random_packed(g, 4 * D, D, 128, bits, sigma=0.05)
    root, oroot = cq.New(proot), orc.OMatrix.new(proot)
    spans = [(0, D), (D, 2 * D), (2 * D, 3 * D - 40), (3 * D - 40, 4 * D)]  # the last two not block-aligned
    ms = [root.Rows(lo, hi) for lo, hi in spans]
    x = g.standard_normal((rows, D)).astype(np.float32)
    ys = [torch.zeros(rows, hi - lo, device="cuda") for lo, hi in spans]
    cq.gemms_dev(ms, ys, _t(x), rows)
    torch.cuda.synchronize()
    for (lo, hi), y in zip(spans, ys):
        want = oroot.rows(lo, hi).gemm(x.reshape(-1), rows, orc.LUT).reshape(rows, hi - lo)
        assert same(y.cpu().numpy(), want), (lo, hi)


@pytest.mark.parametrize("bits", [2, 4])
def test_split_fused_prologues_and_epilogues(bits):
    # ZCRMSNorm in front, the residual add or SiLU behind, and the gated
    # input, each against the oracle's separate steps
    import torch

    g = synth.rng(90 + bits)
    rows, D, F = 375, 512, 2048
    pu = synth.random_packed(g, F, D, 128, bits, sigma=0.05)
    pd = synth.random_packed(g, D, F, 128, bits, sigma=0.05)
    mu, md = cq.New(pu), cq.New(pd)
    assert md.gemm_path(rows) == "lut-mfma-split"
    assert mu.gemm_path(rows) == "lut-mfma-tab"
    x = (g.standard_normal((rows, D)) * 3).astype(np.float32)
    gain = (1 + g.standard_normal(D) * 0.1).astype(np.float32)
    u = torch.zeros(rows, F, device="cuda")
    cq.gemms_fused_dev([mu], [u], _t(x), rows, norm_gain=_t(gain), act=1)
    h = orc.zc_rmsnorm(x.reshape(-1), gain, D)
    want_u = orc.silu(orc.OMatrix.new(pu).gemm(h, rows, orc.LUT))
    torch.cuda.synchronize()
    assert same(u.cpu().numpy().reshape(-1), want_u)
    resid = g.standard_normal((rows, D)).astype(np.float32)
    yd = _t(resid)
    cq.gemms_fused_dev([md], [yd], u, rows, resid=yd)
    torch.cuda.synchronize()
    want_y = (resid.reshape(-1) + orc.OMatrix.new(pd).gemm(want_u, rows, orc.LUT)).astype(np.float32)
    assert same(yd.cpu().numpy().reshape(-1), want_y)
    # the gated out projection: (a * sigmoid(gate)) times wo, plus the residual
    po = synth.random_packed(g, D, D, 128, bits, sigma=0.05)
    mo = cq.New(po)
    att = g.standard_normal((rows, D)).astype(np.float32)
    gate = (g.standard_normal((rows, D)) * 2).astype(np.float32)
    xo = _t(resid)
    cq.gemms_gated_dev([mo], [xo], _t(att), _t(gate), rows, resid=xo)
    torch.cuda.synchronize()
    gated, _ = orc.sigmoid_gate(att.reshape(-1), gate.reshape(-1))
    want_o = (resid.reshape(-1) + orc.OMatrix.new(po).gemm(gated, rows, orc.LUT)).astype(np.float32)
    assert same(xo.cpu().numpy().reshape(-1), want_o)


def test_split_workspace_grows_and_is_reused():
    # a small split product, then a larger one (the workspace grows), then the
    # small one again: each bit for bit its oracle product
    import torch

    g = synth.rng(123)
    ps = [synth.random_packed(g, o, 512, 128, 4, sigma=0.05) for o in (512, 4096, 512)]
    for p, rows in zip(ps, (400, 1024, 350)):
        m = cq.New(p)
        x = g.standard_normal((rows, 512)).astype(np.float32)
        y = torch.zeros(rows, p.Out, device="cuda")
        m.gemm_dev(y, _t(x), rows)
        torch.cuda.synchronize()
        assert same(y.cpu().numpy().reshape(-1), orc.OMatrix.new(p).gemm(x.reshape(-1), rows, orc.LUT)), rows


@pytest.mark.parametrize("views", [False, True])
def test_split_append_epilogue(views):
    # the K/V appends (RoPE on K) in the fold, bit for bit the product
    # followed by the separate append kernels, at 400 streams each at its own
    # position (some outside the cache): three matrices of their own
    # codebooks take the split form, three views of one root (one pre-pass
    # serves them) the table form
    import torch

    from go_whistle_amd import decoder as dec
    from go_whistle_amd import needle

    heads, hd, cap, batch = 8, 64, 16, 400
    D = heads * hd
    g = synth.rng(500 + views)
    cos, sin = (_t(a) for a in dec.rope_tables(hd, cap, 1e4))
    if views:
        root = cq.New(synth.random_packed(g, 3 * D, D, 128, 4, sigma=0.05))
        ms = [root.Rows(0, D), root.Rows(D, 2 * D), root.Rows(2 * D, 3 * D)]
    else:
        ms = [cq.New(synth.random_packed(g, D, D, 128, 4, sigma=0.05)) for _ in range(3)]
    assert ms[0].gemm_path(batch) == "lut-mfma-split"
    x = _t((g.standard_normal((batch, D)) * 2).astype(np.float32))
    gain = _t((1 + g.standard_normal(D) * 0.1).astype(np.float32))
    p = g.integers(0, cap, size=batch).astype(np.int32)
    p[1::7] = -1
    p[4::11] = cap
    pos = _t(p)
    want_y = [torch.zeros(batch, D, device="cuda") for _ in ms]
    got_y = [torch.zeros(batch, D, device="cuda") for _ in ms]
    kq1 = _t(g.integers(-128, 128, size=(batch, cap, D), dtype=np.int8))
    ks1 = _t(g.random((batch, cap, heads)).astype(np.float32))
    vq1 = _t(g.integers(-128, 128, size=(batch, cap, D), dtype=np.int8))
    vs1 = _t(g.random((batch, cap, heads)).astype(np.float32))
    kq2, ks2, vq2, vs2 = kq1.clone(), ks1.clone(), vq1.clone(), vs1.clone()
    cq.gemms_fused_dev(ms, want_y, x, batch, norm_gain=gain)
    needle.append_dev(kq1, ks1, want_y[1], batch, D, hd, cap * D, cap * heads, pos, cap, rope=(cos, sin))
    needle.append_dev(vq1, vs1, want_y[2], batch, D, hd, cap * D, cap * heads, pos, cap)
    cq.gemms_append_dev(ms, got_y, x, batch, [None, (kq2, ks2, (cos, sin)), (vq2, vs2, None)], cap * D,
                        cap * heads, pos, cap, norm_gain=gain)
    torch.cuda.synchronize()
    for a, b in zip(got_y, want_y):
        assert same(a.cpu().numpy(), b.cpu().numpy())
    assert np.array_equal(kq2.cpu().numpy(), kq1.cpu().numpy())
    assert np.array_equal(vq2.cpu().numpy(), vq1.cpu().numpy())
    assert same(ks2.cpu().numpy(), ks1.cpu().numpy()) and same(vs2.cpu().numpy(), vs1.cpu().numpy())
