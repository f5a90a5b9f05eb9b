"""The table form of the MFMA product (lut_tables_kernel, then
lut_mfma_tab_kernel), through the C ABI: products of 16 to 3072 activations
of 256K row-activations or more (384K at 2 bits), or whose (64-row block,
32-activation tile) workgroups reach the CUs, and up to 12288 over 768 rows
or more or at 2 bits (6144 otherwise) (the decode step's
q/k/v/gate and FFN-up products and its head at batch 256, the encoder's
products at 375, 1500 and 12000 frames), bit for bit the
oracle's lut product (internal/cq/lut.go), with row views, several matrices
on one input, activations that do not fill a 32-wide tile, every fused
prologue and epilogue, and the K/V append."""

import numpy as np
import pytest

from go_whistle_amd import cq, synth
from oracle import binding as orc

pytestmark = pytest.mark.gpu


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("out,inp,rows", [(2048, 512, 256), (2048, 512, 193), (2048, 512, 230), (2048, 512, 319),
                                          (2100, 384, 200), (4096, 1024, 256), (2048, 128, 250), (2048, 512, 375),
                                          (1536, 512, 1500), (512, 512, 3000), (2048, 128, 2048), (2100, 384, 2040)])
def test_tab_gemm_bit_exact(bits, out, inp, rows):
    # the last two run slabs of four blocks: one group, and three groups over
    # 33 blocks (the last slab one block) with a partial activation tile
    import torch

    g = synth.rng(out + inp + rows + bits + 7)
    p = synth.random_packed(g, out, inp, 128, bits, sigma=0.05)
    m = cq.New(p)
    assert m.gemm_path(rows) == "lut-mfma-tab"
    x = (g.standard_normal((rows, inp)) * 2).astype(np.float32)
    y = torch.full((rows, out), float("nan"), device="cuda")
    m.gemm_dev(y, _t(x), rows)
    torch.cuda.synchronize()
    want = orc.OMatrix.new(p).gemm(x.reshape(-1), rows, orc.LUT).reshape(rows, out)
    assert same(y.cpu().numpy(), want)


def test_tab_path_bounds():
    # the form runs from 16 activations to 3072 at 256K row-activations (384K
    # at 2 bits) or when its (block, tile) workgroups reach the CUs, and to
    # 12288 over 768 rows or more or at 2 bits (6144 otherwise), at most 8
    # groups; fewer, more groups or more activations leave it
    g = synth.rng(3)
    m = cq.New(synth.random_packed(g, 2048, 512, 128, 4, sigma=0.05))
    assert m.gemm_path(127) == "lut" and m.gemm_path(128) == "lut-mfma-tab"
    m2 = cq.New(synth.random_packed(g, 2048, 512, 128, 2, sigma=0.05))
    assert m2.gemm_path(191) == "lut" and m2.gemm_path(192) == "lut-mfma-tab"
    assert m.gemm_path(375) == "lut-mfma-tab" and m.gemm_path(3072) == "lut-mfma-tab"
    assert m.gemm_path(3073) == "lut-mfma-tab" and m.gemm_path(12288) == "lut-mfma-tab"
    assert m.gemm_path(12289) == "lut-mfma"
    m512 = cq.New(synth.random_packed(g, 512, 512, 128, 4, sigma=0.05))
    assert m512.gemm_path(6144) == "lut-mfma-tab" and m512.gemm_path(6145) != "lut-mfma-tab"
    m512b = cq.New(synth.random_packed(g, 512, 512, 128, 2, sigma=0.05))
    assert m512b.gemm_path(12288) == "lut-mfma-tab"
    m1 = cq.New(synth.random_packed(g, 1024, 512, 128, 4, sigma=0.05))
    assert m1.gemm_path(255) == "lut" and m1.gemm_path(256) == "lut-mfma-tab"
    mh = cq.New(synth.random_packed(g, 16384, 512, 128, 4, sigma=0.05))
    assert mh.gemm_path(15) == "lut" and mh.gemm_path(16) == "lut-mfma-tab"
    assert cq.New(synth.random_packed(g, 2048, 2048, 128, 2, sigma=0.05)).gemm_path(256) == "lut"
    # small matrices past 3072 activations: the table form at 2 bits (64x512
    # CQ2 at 3500 / 12000 activations measured 23.5 / 40.8 us against the
    # 512-row MFMA form's 40.5 / 77.3 us) and at 4 bits up to 6144
    # (64x512 CQ4 at 6000: 40.2 against 62.4 us); at 4 bits beyond, the
    # MFMA form (the two measured within 1%)
    for o in (64, 128, 256, 384):
        s2 = cq.New(synth.random_packed(g, o, 512, 128, 2, sigma=0.05))
        s4 = cq.New(synth.random_packed(g, o, 512, 128, 4, sigma=0.05))
        assert s2.gemm_path(3500) == s2.gemm_path(12000) == "lut-mfma-tab"
        assert s4.gemm_path(6000) == "lut-mfma-tab" and s4.gemm_path(12000) == "lut-mfma"


@pytest.mark.parametrize("bits,rows", [(2, 256), (4, 256), (4, 2000)])
def test_tab_views_and_shared_input(bits, rows):
    # four row views of one root (two not block-aligned) on one input: one
    # pre-pass and one product launch, each output bit for bit its own oracle
    # product; at 2000 activations the product runs slabs of four blocks (the
    # last view's third slab partial, its block starting mid-view)
    import torch

    g = synth.rng(170 + bits + rows)
    D = 512
    proot = synth.random_packed(g, 4 * D, D, 128, bits, sigma=0.05)
    root, oroot = cq.New(proot), orc.OMatrix.new(proot)
    spans = [(0, D), (D, 2 * D), (2 * D, 3 * D - 40), (3 * D - 40, 4 * D)]
    ms = [root.Rows(lo, hi) for lo, hi in spans]
    x = g.standard_normal((rows, D)).astype(np.float32)
    ys = [torch.full((rows, hi - lo), float("nan"), device="cuda") for lo, hi in spans]
    cq.gemms_dev(ms, ys, _t(x), rows)
    torch.cuda.synchronize()
    for (lo, hi), y in zip(spans, ys):
        want = oroot.rows(lo, hi).gemm(x.reshape(-1), rows, orc.LUT).reshape(rows, hi - lo)
        assert same(y.cpu().numpy(), want), (lo, hi)


@pytest.mark.parametrize("bits,rows", [(2, 256), (4, 256), (2, 2048)])
def test_tab_fused_prologues_and_epilogues(bits, rows):
    # ZCRMSNorm in front and SiLU behind (FFN-up), the gated input and the
    # residual add, each against the oracle's separate steps, over 2048 rows
    # (at 2048 activations the product runs slabs of four blocks)
    import torch

    g = synth.rng(190 + bits + rows)
    D, F = 512, 2048
    pu = synth.random_packed(g, F, D, 128, bits, sigma=0.05)
    mu = cq.New(pu)
    assert mu.gemm_path(rows) == "lut-mfma-tab"
    x = (g.standard_normal((rows, D)) * 3).astype(np.float32)
    gain = (1 + g.standard_normal(D) * 0.1).astype(np.float32)
    u = torch.zeros(rows, F, device="cuda")
    cq.gemms_fused_dev([mu], [u], _t(x), rows, norm_gain=_t(gain), act=1)
    h = orc.zc_rmsnorm(x.reshape(-1), gain, D)
    torch.cuda.synchronize()
    assert same(u.cpu().numpy().reshape(-1), orc.silu(orc.OMatrix.new(pu).gemm(h, rows, orc.LUT)))
    # the gated product with the residual add: (a * sigmoid(gate)) times w, plus resid
    att = g.standard_normal((rows, D)).astype(np.float32)
    gate = (g.standard_normal((rows, D)) * 2).astype(np.float32)
    resid = g.standard_normal((rows, F)).astype(np.float32)
    yo = _t(resid)
    cq.gemms_gated_dev([mu], [yo], _t(att), _t(gate), rows, resid=yo)
    torch.cuda.synchronize()
    gated, _ = orc.sigmoid_gate(att.reshape(-1), gate.reshape(-1))
    want = (resid.reshape(-1) + orc.OMatrix.new(pu).gemm(gated, rows, orc.LUT)).astype(np.float32)
    assert same(yo.cpu().numpy().reshape(-1), want)


@pytest.mark.parametrize("batch", [256, 3000])
def test_tab_append_epilogue(batch):
    # the q/k/v/gate launch of the decode step at 256 streams: the norm in
    # front, the K/V int8 appends (RoPE on K) in the fold, each stream at its
    # own position (some outside the cache); y bit for bit the oracle's
    # products and the caches those of the separate append kernels; at 3000
    # streams the product runs slabs of four blocks
    import torch

    from go_whistle_amd import decoder as dec
    from go_whistle_amd import needle

    heads, hd, cap = 8, 64, 16
    D = heads * hd
    g = synth.rng(600)
    cos, sin = (_t(a) for a in dec.rope_tables(hd, cap, 1e4))
    ps = [synth.random_packed(g, D, D, 128, 4, sigma=0.05) for _ in range(4)]
    for p in ps[1:]:
        p.Codebook = ps[0].Codebook
    ms = [cq.New(p) for p in ps]
    x = (g.standard_normal((batch, D)) * 2).astype(np.float32)
    gain = (1 + g.standard_normal(D) * 0.1).astype(np.float32)
    pp = g.integers(0, cap, size=batch).astype(np.int32)
    pp[1::7] = -1
    pp[4::11] = cap
    pos = _t(pp)
    h = orc.zc_rmsnorm(x.reshape(-1), gain, D)
    want_y = [orc.OMatrix.new(p).gemm(h, batch, orc.LUT).reshape(batch, D) for p in ps]
    kq1 = _t(g.integers(-128, 128, size=(batch, cap, D), dtype=np.int8))
    ks1 = _t(g.random((batch, cap, heads)).astype(np.float32))
    vq1 = _t(g.integers(-128, 128, size=(batch, cap, D), dtype=np.int8))
    vs1 = _t(g.random((batch, cap, heads)).astype(np.float32))
    kq2, ks2, vq2, vs2 = kq1.clone(), ks1.clone(), vq1.clone(), vs1.clone()
    needle.append_dev(kq1, ks1, _t(want_y[1]), batch, D, hd, cap * D, cap * heads, pos, cap, rope=(cos, sin))
    needle.append_dev(vq1, vs1, _t(want_y[2]), batch, D, hd, cap * D, cap * heads, pos, cap)
    got_y = [torch.zeros(batch, D, device="cuda") for _ in ms]
    cq.gemms_append_dev(ms, got_y, _t(x), batch, [None, (kq2, ks2, (cos, sin)), (vq2, vs2, None), None],
                        cap * D, cap * heads, pos, cap, norm_gain=_t(gain))
    torch.cuda.synchronize()
    for a, b in zip(got_y, want_y):
        assert same(a.cpu().numpy(), b)
    assert np.array_equal(kq2.cpu().numpy(), kq1.cpu().numpy())
    assert np.array_equal(vq2.cpu().numpy(), vq1.cpu().numpy())
    assert same(ks2.cpu().numpy(), ks1.cpu().numpy()) and same(vs2.cpu().numpy(), vs1.cpu().numpy())


def test_tab_head_rows_sampled():
    # the batch-256 decode head (16384x512 CQ4) on the table form: the first
    # and last 384 rows against the oracle's views
    import torch

    g = synth.rng(77)
    rows = 256
    p = synth.random_packed(g, 16384, 512, 128, 4, sigma=0.05)
    m = cq.New(p)
    assert m.gemm_path(rows) == "lut-mfma-tab"
    x = g.standard_normal((rows, 512)).astype(np.float32)
    y = torch.full((rows, 16384), float("nan"), device="cuda")
    m.gemm_dev(y, _t(x), rows)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    om = orc.OMatrix.new(p)
    for lo, hi in ((0, 384), (16000, 16384)):
        want = om.rows(lo, hi).gemm(x.reshape(-1), rows, orc.LUT).reshape(rows, hi - lo)
        assert same(got[:, lo:hi], want), (lo, hi)


def test_tab_workspace_shared_with_split():
    # a table-form product, a split-form product (the workspace grows), and
    # the table form again: each bit for bit its oracle product
    import torch

    g = synth.rng(321)
    cases = [(synth.random_packed(g, 2048, 512, 128, 4, sigma=0.05), 256),
             (synth.random_packed(g, 512, 2048, 128, 4, sigma=0.05), 1024),
             (synth.random_packed(g, 2048, 512, 128, 2, sigma=0.05), 200)]
    for (p, rows), path in zip(cases, ("lut-mfma-tab", "lut-mfma-split", "lut-mfma-tab")):
        m = cq.New(p)
        assert m.gemm_path(rows) == path
        x = g.standard_normal((rows, p.In)).astype(np.float32)
        y = torch.zeros(rows, p.Out, device="cuda")
        m.gemm_dev(y, _t(x), rows)
        torch.cuda.synchronize()
        assert same(y.cpu().numpy().reshape(-1), orc.OMatrix.new(p).gemm(x.reshape(-1), rows, orc.LUT)), rows


@pytest.mark.parametrize("out,bits,rows", [(1024, 4, 6000), (2048, 2, 12288), (1536, 4, 3100), (512, 4, 5000),
                                           (512, 2, 9000), (768, 4, 7000)])
def test_tab_many_activations_sampled(out, bits, rows):
    # past 3072 activations (over 768 rows or more, at 2 bits, or to 6144):
    # 48 sampled activations
    # (the first and last tiles, a tile edge mid-way, random ones) against
    # the oracle, each activation's product being its own
    import torch

    g = synth.rng(out + bits + rows)
    p = synth.random_packed(g, out, 512, 128, bits, sigma=0.05)
    m = cq.New(p)
    assert m.gemm_path(rows) == "lut-mfma-tab"
    x = g.standard_normal((rows, 512)).astype(np.float32)
    y = torch.full((rows, out), float("nan"), device="cuda")
    m.gemm_dev(y, _t(x), rows)
    torch.cuda.synchronize()
    mid = (rows // 64) * 32
    pick = np.unique(np.concatenate([[0, 1, 31, 32, mid - 1, mid, rows - 33, rows - 32, rows - 1],
                                     g.choice(rows, size=39, replace=False)]))
    got = y.cpu().numpy()[pick]
    want = orc.OMatrix.new(p).gemm(x[pick].reshape(-1), len(pick), orc.LUT).reshape(len(pick), out)
    assert same(got, want)


def test_tab_norm_many_activations_sampled():
    # ZCRMSNorm in front and SiLU behind at 3100 activations (the pre-pass
    # takes 8 activations a workgroup past 3072): 40 sampled activations
    # against the oracle's separate steps
    import torch

    g = synth.rng(3100)
    rows, D, F = 3100, 512, 2048
    p = synth.random_packed(g, F, D, 128, 2, sigma=0.05)
    m = cq.New(p)
    assert m.gemm_path(rows) == "lut-mfma-tab"
    x = (g.standard_normal((rows, D)) * 3).astype(np.float32)
    gain = (1 + g.standard_normal(D) * 0.1).astype(np.float32)
    u = torch.full((rows, F), float("nan"), device="cuda")
    cq.gemms_fused_dev([m], [u], _t(x), rows, norm_gain=_t(gain), act=1)
    torch.cuda.synchronize()
    pick = np.unique(np.concatenate([[0, 7, 8, 3071, 3072, 3099], g.choice(rows, size=34, replace=False)]))
    h = orc.zc_rmsnorm(x[pick].reshape(-1), gain, D)
    want = orc.silu(orc.OMatrix.new(p).gemm(h, len(pick), orc.LUT)).reshape(len(pick), F)
    assert same(u.cpu().numpy()[pick], want)


@pytest.mark.parametrize("bits,rows", [(4, 16), (4, 40), (2, 33)])
def test_tab_tall_few_activations(bits, rows):
    # a 16384-row matrix (the head of a beam search) at 16 to 40 activations,
    # one or two partial tiles spread over the XCDs: every activation against
    # the oracle on the first and last 512 rows
    import torch

    g = synth.rng(900 + rows + bits)
    p = synth.random_packed(g, 16384, 512, 128, bits, sigma=0.05)
    m = cq.New(p)
    assert m.gemm_path(rows) == "lut-mfma-tab"
    x = g.standard_normal((rows, 512)).astype(np.float32)
    y = torch.full((rows, 16384), float("nan"), device="cuda")
    m.gemm_dev(y, _t(x), rows)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    om = orc.OMatrix.new(p)
    for lo, hi in ((0, 512), (15872, 16384)):
        want = om.rows(lo, hi).gemm(x.reshape(-1), rows, orc.LUT).reshape(rows, hi - lo)
        assert same(got[:, lo:hi], want), (lo, hi)
