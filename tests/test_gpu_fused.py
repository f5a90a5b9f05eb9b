"""The fused forms of the decode step's neighbours, through the C ABI: each
bit for bit the separate steps it replaces (which the other GPU tests pin
to the oracle). ZCRMSNorm in front of a CQ product (lut kernel and its MFMA
form), the residual add and SiLU behind it, RoPE in front of the int8
append and of the query's attention, and the whole synthetic decoder with
and without fusion."""

import math

import numpy as np
import pytest

from go_whistle_amd import cq, decoder as dec, needle, synth
from go_whistle_amd._lib import check, lib

pytestmark = pytest.mark.gpu


def same(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _p(t):
    from ctypes import c_void_p

    return c_void_p(t.data_ptr())


def _s():
    return cq._stream()


def _norm(x, gain, rows, dim):
    import torch

    h = torch.empty_like(x)
    check(lib().nd_zcrmsnorm_dev(_p(h), _p(x), _p(gain), rows, dim, _s()))
    return h


@pytest.mark.parametrize("rows,shape,bits", [(1, (512, 512), 4), (5, (2048, 512), 2), (256, (16384, 512), 4),
                                             (3, (300, 640), 4), (2048, (16384, 512), 2), (64, (512, 2048), 4)])
def test_norm_prologue(rows, shape, bits):
    import torch

    out, inp = shape
    g = synth.rng(rows + out + bits)
    ms = [cq.New(synth.random_packed(g, out, inp, 128, bits, sigma=0.05)) for _ in range(2)]
    x = _t((g.standard_normal((rows, inp)) * 3).astype(np.float32))
    gain = _t((1 + g.standard_normal(inp) * 0.1).astype(np.float32))
    want = [torch.zeros(rows, out, device="cuda") for _ in ms]
    got = [torch.zeros(rows, out, device="cuda") for _ in ms]
    cq.gemms_dev(ms, want, _norm(x, gain, rows, inp), rows)
    cq.gemms_fused_dev(ms, got, x, rows, norm_gain=gain)
    torch.cuda.synchronize()
    for a, b in zip(got, want):
        assert same(a.cpu().numpy(), b.cpu().numpy())
    if rows >= 256:  # the table form up to 3072 activations
        assert ms[0].gemm_path(rows) == "lut-mfma-tab"


@pytest.mark.parametrize("rows,bits", [(1, 4), (7, 2), (48, 4), (40, 2), (256, 4)])
def test_residual_and_silu_epilogues(rows, bits):
    import torch

    g = synth.rng(70 + rows + bits)
    out, inp = (2048, 512) if rows < 256 else (16384, 512)
    m = cq.New(synth.random_packed(g, out, inp, 128, bits, sigma=0.05))
    a = _t(g.standard_normal((rows, inp)).astype(np.float32))
    x0 = g.standard_normal((rows, out)).astype(np.float32)
    y = torch.zeros(rows, out, device="cuda")
    m.gemm_dev(y, a, rows)
    # residual: x += W a, in place
    x = _t(x0)
    want = x.clone()
    check(lib().nd_add_dev(_p(want), _p(y), rows * out, _s()))
    cq.gemms_fused_dev([m], [x], a, rows, resid=x)
    # SiLU: u = silu(W a)
    u = torch.zeros(rows, out, device="cuda")
    cq.gemms_fused_dev([m], [u], a, rows, act=1)
    want_u = y.clone()
    check(lib().nd_silu_dev(_p(want_u), rows * out, _s()))
    torch.cuda.synchronize()
    assert same(x.cpu().numpy(), want.cpu().numpy())
    assert same(u.cpu().numpy(), want_u.cpu().numpy())


def test_fused_misuse():
    import torch

    from go_whistle_amd import CQPanic, CQDeviceError

    g = synth.rng(5)
    m = cq.New(synth.random_packed(g, 64, 128, 128, 4))
    z = torch.zeros(64 * 128, device="cuda")
    with pytest.raises(CQPanic):
        cq.gemms_fused_dev([m, m], [z, z], z, 1, resid=z)
    with pytest.raises(CQPanic):
        cq.gemms_fused_dev([m], [z], z, 1, resid=z, act=1)
    with pytest.raises(CQDeviceError):
        cq.gemms_fused_dev([m.Exact()], [z], z, 1, act=1)


def test_append_with_rope():
    import torch

    B, heads, hd, cap = 3, 8, 64, 16
    D = heads * hd
    cos, sin = dec.rope_tables(hd, cap, 1e5)
    cos, sin = _t(cos), _t(sin)
    g = synth.rng(11)
    x = _t(g.standard_normal((B, D)).astype(np.float32))
    pos = _t(np.array([0, 5, 15], np.int32))
    q1 = torch.zeros(B, cap, D, dtype=torch.int8, device="cuda")
    s1 = torch.zeros(B, cap, heads, device="cuda")
    q2, s2 = q1.clone(), s1.clone()
    xr = x.clone()
    check(lib().nd_rope_dev(_p(xr), B, heads, hd, _p(cos), _p(sin), cos.shape[0], _p(pos), 1, _s()))
    needle.append_dev(q1, s1, xr, B, D, hd, cap * D, cap * heads, pos, cap)
    needle.append_dev(q2, s2, x, B, D, hd, cap * D, cap * heads, pos, cap, rope=(cos, sin))
    torch.cuda.synchronize()
    assert np.array_equal(q1.cpu().numpy(), q2.cpu().numpy())
    assert same(s1.cpu().numpy(), s2.cpu().numpy())


@pytest.mark.parametrize("batch,bits,views", [(1, 4, False), (3, 2, False), (100, 4, False), (256, 4, False),
                                              (5, 4, True), (300, 2, True), (64, 4, False), (80, 2, True)])
def test_append_epilogue(batch, bits, views):
    # The K/V appends riding on the qkv product, bit for bit the product
    # followed by the separate append kernels; batch 1, 100 and 256 cover
    # the kernel's shared-block (4 and 2 wavefronts a block) and one-wavefront
    # write paths, 64 and 80 its wide form on 8-block units (two wavefronts a
    # block); views: q, k, v as row views of one fused root.
    import torch

    heads, hd, cap = 8, 64, 16
    D = heads * hd
    g = synth.rng(300 + batch + bits)
    cos, sin = dec.rope_tables(hd, cap, 1e4)
    cos, sin = _t(cos), _t(sin)
    if views:
        root = cq.New(synth.random_packed(g, 3 * D, D, 128, bits, sigma=0.05))
        ms = [root.Rows(0, D), root.Rows(D, 2 * D), root.Rows(2 * D, 3 * D)]
    else:
        ms = [cq.New(synth.random_packed(g, D, D, 128, bits, sigma=0.05)) for _ in range(3)]
    x = _t((g.standard_normal((batch, D)) * 2).astype(np.float32))
    gain = _t((1 + g.standard_normal(D) * 0.1).astype(np.float32))
    # every stream at its own position, some outside the cache (no append)
    p = g.integers(0, cap, size=batch).astype(np.int32)
    p[1::7] = -1
    p[4::11] = cap
    pos = _t(p)
    want_y = [torch.zeros(batch, D, device="cuda") for _ in ms]
    got_y = [torch.zeros(batch, D, device="cuda") for _ in ms]
    caches = []
    for _ in range(2):
        kq = _t(g.integers(-128, 128, size=(batch, cap, D), dtype=np.int8))
        ks = _t(g.random((batch, cap, heads)).astype(np.float32))
        vq = _t(g.integers(-128, 128, size=(batch, cap, D), dtype=np.int8))
        vs = _t(g.random((batch, cap, heads)).astype(np.float32))
        caches.append((kq, ks, vq, vs))
    (kq1, ks1, vq1, vs1), (kq2, ks2, vq2, vs2) = caches
    kq2.copy_(kq1), ks2.copy_(ks1), vq2.copy_(vq1), vs2.copy_(vs1)
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
    assert same(ks2.cpu().numpy(), ks1.cpu().numpy())
    assert same(vs2.cpu().numpy(), vs1.cpu().numpy())


def test_append_epilogue_misuse():
    import torch

    from go_whistle_amd import CQPanic, CQDeviceError

    g = synth.rng(6)
    D, cap = 512, 4
    root = cq.New(synth.random_packed(g, 2 * D, D, 128, 4))
    z = torch.zeros(D, device="cuda")
    q8 = torch.zeros(cap * D, dtype=torch.int8, device="cuda")
    s8 = torch.zeros(cap * 8, device="cuda")
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    with pytest.raises(CQPanic):  # heads cut by the view
        cq.gemms_append_dev([root.Rows(32, D + 32)], [z], z, 1, [(q8, s8, None)], cap * D, cap * 8, pos, cap)
    with pytest.raises(CQPanic):  # no positions
        cq.gemms_append_dev([root.Rows(0, D)], [z], z, 1, [(q8, s8, None)], cap * D, cap * 8, None, cap)
    with pytest.raises(CQDeviceError):  # an Exact view runs no lut kernel
        cq.gemms_append_dev([root.Rows(0, D).Exact()], [z], z, 1, [(q8, s8, None)], cap * D, cap * 8, pos, cap)


@pytest.mark.parametrize("batch,n,vd", [(1, 37, 64), (4, 300, 64), (80, 100, 64), (3, 50, 128), (2, 20, 40)])
def test_attention_with_query_rope(batch, n, vd):
    # the chain kernel (vd 64, both layouts), the streamed kernel (vd 128)
    # and the general kernel (vd 40, qk 20)
    import torch

    heads = 8
    qk = 64 if vd != 40 else 20
    g = synth.rng(batch * 1000 + n + vd)
    cap = 64
    cos, sin = dec.rope_tables(qk, cap, 1e5)
    cos, sin = _t(cos), _t(sin)
    stride = n * heads * max(qk, vd)
    kq = _t(g.integers(-128, 128, size=batch * stride, dtype=np.int8))
    vq = _t(g.integers(-128, 128, size=batch * stride, dtype=np.int8))
    ks = _t((g.random(batch * n * heads) * 0.05 + 1e-4).astype(np.float32))
    vs = _t((g.random(batch * n * heads) * 0.05 + 1e-4).astype(np.float32))
    q = _t(g.standard_normal(batch * heads * qk).astype(np.float32))
    qpos = _t(g.integers(0, cap, size=batch).astype(np.int32))
    spans = _t(np.array([[0, 0, 0, n - (b % 3)] for b in range(batch)], np.int32))
    kw = dict(batch=batch, q_stride=heads * qk, kv_stride=stride, s_stride=n * heads, out_stride=heads * vd)
    args = (1, heads, kq, ks, heads * qk, qk, vq, vs, heads * vd, vd, spans, n, np.float32(math.sqrt(qk)), True)
    qr = q.clone()
    check(lib().nd_rope_dev(_p(qr), batch, heads, qk, _p(cos), _p(sin), cos.shape[0], _p(qpos), 1, _s()))
    want = torch.zeros(batch * heads * vd, device="cuda")
    got = torch.zeros_like(want)
    needle.attend_int8_dev(want, qr, *args, **kw)
    needle.attend_int8_dev(got, q, *args, **kw, rope=(cos, sin, qpos))
    torch.cuda.synchronize()
    assert same(got.cpu().numpy(), want.cpu().numpy())


def test_decoder_fused_equals_plain():
    cfg = dec.DecoderConfig(vocab=4096, layers=2, frames=100, max_pos=64)
    model = dec.make_model(3, cfg)
    out = []
    for fused in (False, True):
        d = dec.Decoder(model, 4, fused=fused)
        d.set_memory(3)
        toks = d.decode([1, 2, 3, 4], 20).cpu().numpy()
        out.append((toks, d.logits.cpu().numpy()))
    assert np.array_equal(out[0][0], out[1][0])
    assert same(out[0][1], out[1][1])


def test_sigmoid_gate_vs_oracle():
    """nd_sigmoid_gate_dev against the oracle's Attention.output gate
    (attention.go:245-249), bit for bit, tails and zeros included."""
    import torch

    from oracle import binding as orc

    g = synth.rng(91)
    out = (g.standard_normal(70001) * 3).astype(np.float32)
    gate = (g.standard_normal(70001) * 8).astype(np.float32)
    gate[:6] = [0.0, -0.0, 120.0, -120.0, -103.5, 30.0]
    wo, wg = orc.sigmoid_gate(out, gate)
    o, gg = _t(out), _t(gate)
    check(lib().nd_sigmoid_gate_dev(_p(o), _p(gg), out.size, _s()))
    torch.cuda.synchronize()
    assert same(gg.cpu().numpy(), wg) and same(o.cpu().numpy(), wo)


@pytest.mark.parametrize("rows,shape,bits,resid", [(1, (512, 512), 4, True), (6, (512, 2048), 2, True),
                                                   (4, (1024, 512), 4, False), (300, (16384, 512), 4, False),
                                                   (2048, (16384, 512), 4, True), (256, (512, 512), 4, True),
                                                   (128, (512, 2048), 2, True)])
def test_gated_product(rows, shape, bits, resid):
    """cq_gemms_gated_dev (x * sigmoid(gate) inside the product, then the
    residual add) bit for bit the separate gate, product and add; at 300
    and 2048 activations of a 16384-row matrix the table form's pre-pass
    carries the gate."""
    import torch

    out, inp = shape
    g = synth.rng(92 + rows + out)
    m = cq.New(synth.random_packed(g, out, inp, 128, bits, sigma=0.05))
    x = _t((g.standard_normal((rows, inp)) * 2).astype(np.float32))
    gate = _t((g.standard_normal((rows, inp)) * 4).astype(np.float32))
    r0 = _t(g.standard_normal((rows, out)).astype(np.float32))
    xw, gw_ = x.clone(), gate.clone()
    check(lib().nd_sigmoid_gate_dev(_p(xw), _p(gw_), rows * inp, _s()))
    want = torch.zeros(rows, out, device="cuda")
    m.gemm_dev(want, xw, rows)
    if resid:
        want = r0 + want
    got = r0.clone() if resid else torch.zeros(rows, out, device="cuda")
    gate_before = gate.clone()
    cq.gemms_gated_dev([m], [got], x, gate, rows, resid=got if resid else None)
    torch.cuda.synchronize()
    assert same(got.cpu().numpy(), want.cpu().numpy())
    assert torch.equal(gate, gate_before)  # the gate is only read
    if rows >= 300:
        assert m.gemm_path(rows) == "lut-mfma-tab"


def test_gated_product_vs_oracle():
    """The gated product against the oracle: gate, then the lut product."""
    import torch

    from oracle import binding as orc

    g = synth.rng(95)
    p = synth.random_packed(g, 512, 512, 128, 4, sigma=0.05)
    m, om = cq.New(p), orc.OMatrix.new(p)
    x = (g.standard_normal((3, 512)) * 2).astype(np.float32)
    gate = (g.standard_normal((3, 512)) * 4).astype(np.float32)
    xw, _ = orc.sigmoid_gate(x, gate)
    want = om.gemm(xw, 3)
    got = torch.zeros(3, 512, device="cuda")
    cq.gemms_gated_dev([m], [got], _t(x), _t(gate), 3)
    torch.cuda.synchronize()
    assert same(got.cpu().numpy().ravel(), want)


def test_gated_misuse():
    import torch

    from go_whistle_amd import CQPanic

    g = synth.rng(96)
    ms = [cq.New(synth.random_packed(g, 512, 512, 128, 4, sigma=0.05)) for _ in range(2)]
    x = torch.zeros(2, 512, device="cuda")
    ys = [torch.zeros(2, 512, device="cuda") for _ in ms]
    with pytest.raises(CQPanic):  # no gate
        cq.gemms_gated_dev(ms, ys, x, None, 2)
    with pytest.raises(CQPanic):  # a residual add takes one matrix
        cq.gemms_gated_dev(ms, ys, x, x, 2, resid=ys[0])
