"""Chained products through the C ABI (cq_tables_bytes, cq_gemm_tables_dev,
cq_gemms_tables_dev): a product whose launch runs a workgroup per
activation over all of its rows also builds the next product's table-form
tables from its output row (ZCRMSNorm, rotation, bound, int8 planes,
lut.go:158-282), and the next product runs on them without its pre-pass.
Every output is bit for bit the oracle's separate steps (the gated input or
plain input, the residual add, the norm, the lut product of
internal/cq/lut.go, SiLU, the K/V int8 appends), with the table buffer
filled with garbage first (slots past the activations are never written and
their results dropped), at full and ragged activation tiles, and where the
producer cannot build them (more activations than one round of workgroups)
the next product runs unchained."""

import numpy as np
import pytest

from go_whistle_amd import cq, synth
from go_whistle_amd._lib import CQPanic
from oracle import binding as orc

pytestmark = pytest.mark.gpu


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _shared(g, n, out, inp, bits):
    ps = [synth.random_packed(g, out, inp, 128, bits, sigma=0.05) for _ in range(n)]
    for p in ps[1:]:
        p.Codebook = ps[0].Codebook
    return ps


def _produce(g, kind, rows, D=512):
    """The producer: wo / cross-wo (512x512 CQ4, gated input, residual) or
    FFN-down (512x2048 CQ2, residual). Returns (packed, x, gate, resid, the
    oracle's output rows)."""
    if kind == "gated":
        p = synth.random_packed(g, D, D, 128, 4, sigma=0.05)
        x = g.standard_normal((rows, D)).astype(np.float32)
        gate = (g.standard_normal((rows, D)) * 2).astype(np.float32)
        xin, _ = orc.sigmoid_gate(x.reshape(-1), gate.reshape(-1))
    else:
        p = synth.random_packed(g, D, 4 * D, 128, 2, sigma=0.05)
        x = (g.standard_normal((rows, 4 * D)) * 0.5).astype(np.float32)
        gate, xin = None, x.reshape(-1)
    resid = (g.standard_normal((rows, D)) * 3).astype(np.float32)
    want = (resid.reshape(-1) + orc.OMatrix.new(p).gemm(xin, rows, orc.LUT)).astype(np.float32)
    return p, x, gate, resid, want.reshape(rows, D)


def _chain(m, x, gate, resid, rows, nxt, gain):
    import torch

    nb = cq.tables_bytes(nxt, rows)
    tables = torch.full((max(nb, 1),), 0x5A, dtype=torch.uint8, device="cuda")[:nb] if nb else None
    y = _t(resid)
    built = cq.gemm_tables_dev(m, y, _t(x), rows, nxt, tables, gate=None if gate is None else _t(gate), resid=y,
                               next_gain=_t(gain))
    return y, tables, built


@pytest.mark.parametrize("kind,nbits,nout,act,rows,built", [
    ("gated", 4, [512, 512], 0, 256, True),   # wo -> cross q/gate
    ("gated", 2, [2048], 1, 256, True),       # cross-wo -> FFN up, SiLU
    ("gated", 2, [2048], 1, 200, True),       # a ragged last tile
    ("down", 4, [16384], 0, 256, True),       # FFN-down -> the head
    ("down", 4, [16384], 0, 137, True),
    ("down", 4, [16384], 0, 64, False),       # the producer's workgroups take a quarter of the rows each
])
def test_chain_bit_exact(kind, nbits, nout, act, rows, built):
    # the producer builds the tables where it runs a workgroup per activation
    # over its 512 rows (from 129 activations to one round of workgroups);
    # otherwise the next product runs unchained on the producer's output
    import torch

    g = synth.rng(7000 + rows + nbits + len(nout))
    D = 512
    p, x, gate, resid, want_y = _produce(g, kind, rows)
    ps = _shared(g, len(nout), nout[0], D, nbits)
    nxt = [cq.New(q) for q in ps]
    gain = (1 + g.standard_normal(D) * 0.1).astype(np.float32)
    assert cq.tables_bytes(nxt, rows) > 0
    y, tables, got_built = _chain(cq.New(p), x, gate, resid, rows, nxt, gain)
    assert got_built == built
    outs = [torch.full((rows, o), float("nan"), device="cuda") for o in nout]
    if got_built:
        cq.gemms_tables_dev(nxt, outs, rows, tables, act=act)
    else:
        cq.gemms_fused_dev(nxt, outs, y, rows, norm_gain=_t(gain), act=act)
    torch.cuda.synchronize()
    assert same(y.cpu().numpy(), want_y)
    h = orc.zc_rmsnorm(want_y.reshape(-1), gain, D)
    for q, o in zip(ps, outs):
        w = orc.OMatrix.new(q).gemm(h, rows, orc.LUT)
        if act:
            w = orc.silu(w)
        assert same(o.cpu().numpy().reshape(-1), w)


@pytest.mark.parametrize("rows", [256, 130])
def test_chain_append(rows):
    # FFN-down -> the next layer's q/k/v/gate with the K/V int8 appends (RoPE
    # on K) in the fold, each stream at its own position (some outside the
    # cache); caches bit for bit those of the separate append kernels
    import torch

    from go_whistle_amd import decoder as dec
    from go_whistle_amd import needle

    heads, hd, cap = 8, 64, 16
    D = heads * hd
    g = synth.rng(7100 + rows)
    p, x, gate, resid, want_y = _produce(g, "down", rows)
    ps = _shared(g, 4, D, D, 4)
    ms = [cq.New(q) for q in ps]
    gain = (1 + g.standard_normal(D) * 0.1).astype(np.float32)
    cos, sin = (_t(a) for a in dec.rope_tables(hd, cap, 1e4))
    pp = g.integers(0, cap, size=rows).astype(np.int32)
    pp[1::7] = -1
    pp[4::11] = cap
    pos = _t(pp)
    h = orc.zc_rmsnorm(want_y.reshape(-1), gain, D)
    want = [orc.OMatrix.new(q).gemm(h, rows, orc.LUT).reshape(rows, D) for q in ps]
    kq1 = _t(g.integers(-128, 128, size=(rows, cap, D), dtype=np.int8))
    ks1 = _t(g.random((rows, cap, heads)).astype(np.float32))
    vq1 = _t(g.integers(-128, 128, size=(rows, cap, D), dtype=np.int8))
    vs1 = _t(g.random((rows, cap, heads)).astype(np.float32))
    kq2, ks2, vq2, vs2 = kq1.clone(), ks1.clone(), vq1.clone(), vs1.clone()
    needle.append_dev(kq1, ks1, _t(want[1]), rows, D, hd, cap * D, cap * heads, pos, cap, rope=(cos, sin))
    needle.append_dev(vq1, vs1, _t(want[2]), rows, D, hd, cap * D, cap * heads, pos, cap)
    y, tables, built = _chain(cq.New(p), x, gate, resid, rows, ms, gain)
    assert built
    got = [torch.zeros(rows, D, device="cuda") for _ in ms]
    cq.gemms_tables_dev(ms, got, rows, tables, caches=[None, (kq2, ks2, (cos, sin)), (vq2, vs2, None), None],
                        q_stride=cap * D, s_stride=cap * heads, pos=pos, cap=cap)
    torch.cuda.synchronize()
    assert same(y.cpu().numpy(), want_y)
    for a, b in zip(got, want):
        assert same(a.cpu().numpy(), b)
    assert np.array_equal(kq2.cpu().numpy(), kq1.cpu().numpy())
    assert np.array_equal(vq2.cpu().numpy(), vq1.cpu().numpy())
    assert same(ks2.cpu().numpy(), ks1.cpu().numpy()) and same(vs2.cpu().numpy(), vs1.cpu().numpy())


def test_chain_unbuilt_and_misuse():
    # more activations than one round of the producer's workgroups: no
    # tables (the product is still right); a next product without the table
    # form needs none; a wrong buffer size or a consumer without the form is
    # refused
    import torch

    D = 512
    g = synth.rng(7200)
    rows = 300
    p, x, gate, resid, want_y = _produce(g, "down", rows)
    head = [cq.New(synth.random_packed(g, 16384, D, 128, 4, sigma=0.05))]
    gain = (1 + g.standard_normal(D) * 0.1).astype(np.float32)
    assert cq.tables_bytes(head, rows) > 0
    y, tables, built = _chain(cq.New(p), x, gate, resid, rows, head, gain)
    torch.cuda.synchronize()
    assert not built and same(y.cpu().numpy(), want_y)
    small = [cq.New(synth.random_packed(g, D, D, 128, 4, sigma=0.05))]
    assert cq.tables_bytes(small, 256) == 0
    p2, x2, _, resid2, want2 = _produce(g, "down", 256)
    y2, t2, built2 = _chain(cq.New(p2), x2, None, resid2, 256, small, gain)
    torch.cuda.synchronize()
    assert t2 is None and not built2 and same(y2.cpu().numpy(), want2)
    nb = cq.tables_bytes(head, 256)
    buf = torch.zeros(nb + 256, dtype=torch.uint8, device="cuda")
    out, out2 = torch.zeros(256, 16384, device="cuda"), torch.zeros(256, D, device="cuda")
    with pytest.raises(CQPanic):
        cq.gemms_tables_dev(head, [out], 256, buf)  # the wrong size
    with pytest.raises(CQPanic):
        cq.gemms_tables_dev(small, [out2], 256, buf[:nb])  # no table form
    with pytest.raises(CQPanic):
        cq.gemm_tables_dev(cq.New(p2), y2, _t(x2), 256, head, buf, resid=y2)  # the wrong size


def test_decoder_chained_equals_unchained():
    # the synthetic decoder at 256 streams: wo, cross-wo and FFN-down build
    # the next products' tables (cross q/gate, FFN up, the next q/k/v/gate
    # and the head); tokens and logits bit for bit the unchained step's
    from go_whistle_amd import decoder as dec

    cfg = dec.DecoderConfig(layers=2, frames=100, max_pos=64)
    model = dec.make_model(11, cfg)
    runs = []
    for chain in (True, False):
        d = dec.Decoder(model, 256)
        d.chain = chain
        d.set_memory(11, "device")
        toks = d.decode(list(range(256)), 12).cpu().numpy()
        runs.append((toks, d.logits.cpu().numpy(), d.n_chained))
    assert runs[0][2] == 3 * cfg.layers and runs[1][2] == 0
    assert np.array_equal(runs[0][0], runs[1][0])
    assert same(runs[0][1], runs[1][1])
