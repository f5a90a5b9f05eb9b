"""GPU parity with the CPU oracle on NaN and infinite inputs, through the C
ABI. The reference reduces every bound with Go's max, which keeps a NaN
(QuantizeRow, int8.go:36-55; softmaxInPlace, load.go:128-138; the lut
tables, lut.go:239-282), and converts a NaN code to int8 0. Each quantiser
(QuantizeRows, fakeQuant, the append, the fused append, the attention's
query), each attention kernel, and the lut product and its MFMA form are
held to the oracle here with NaN and +-Inf in rows, queries, keys and
values: bit for bit where a value is a number, NaN where the oracle has
NaN. Also the stream counts that are not a multiple of 8 (the remainder
of the XCD-aware stream mapping) and 256 streams of self-attention over
1..448 keys."""

import math

import numpy as np
import pytest

from go_whistle_amd import cq, needle, synth
from go_whistle_amd._lib import check, lib
from oracle import binding as orc

pytestmark = pytest.mark.gpu

NAN, INF = np.float32("nan"), np.float32("inf")


def same_nan(a, b):
    """Equal bits where b is a number, NaN exactly where b is NaN."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    if a.shape != b.shape:
        return False
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~nb].view(np.uint32), b[~nb].view(np.uint32))


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _p(t):
    from ctypes import c_void_p

    return c_void_p(t.data_ptr())


def _special_rows(g, rows, width, every=3):
    """rows x width of N(0, 1) where every `every`-th row carries a NaN, a
    +Inf, a -Inf, both infinities, or a NaN beside infinities."""
    x = g.standard_normal((rows, width)).astype(np.float32)
    kinds = [(NAN,), (INF,), (-INF,), (INF, -INF), (NAN, INF, -INF)]
    for r in range(0, rows, every):
        vals = kinds[(r // every) % len(kinds)]
        cols = g.choice(width, size=len(vals), replace=False)
        x[r, cols] = vals
    return x


@pytest.mark.parametrize("width", [64, 17, 512])
def test_quantize_rows_nan_inf(width):
    g = synth.rng(width + 1)
    x = _special_rows(g, 40, width)
    q, s = needle.QuantizeRows(x.reshape(-1), width, width)
    wq, ws = orc.quantize_rows(x.reshape(-1), width, width)
    assert np.array_equal(q, wq)
    assert same_nan(s, ws)
    assert (ws[::3] == 1).any() and np.isinf(ws).any()  # both kinds of special bound occur


def test_fake_quant_nan_inf():
    import torch

    g = synth.rng(77)
    x = _special_rows(g, 30, 96, every=2)
    want = orc.fake_quant(x.reshape(-1), 96, 48)
    xd = _t(x.reshape(-1))
    out = torch.empty_like(xd)
    needle.fake_quant_dev(out, xd, 30, 96, 48)
    torch.cuda.synchronize()
    assert same_nan(out.cpu().numpy(), want)


@pytest.mark.parametrize("rope", [False, True])
def test_append_nan_inf(rope):
    import torch

    from go_whistle_amd import decoder as dec

    g = synth.rng(5 + rope)
    B, cap, heads, hd = 6, 8, 8, 64
    D = heads * hd
    x = _special_rows(g, B * heads, hd, every=2).reshape(B, D)
    pos = np.array([0, 3, 7, 1, 2, 5], np.int32)
    cos, sin = dec.rope_tables(hd, cap, 1e5)
    q = torch.zeros(B, cap, D, dtype=torch.int8, device="cuda")
    s = torch.zeros(B, cap, heads, device="cuda")
    xd, pd, cd, sd = _t(x), _t(pos), _t(cos), _t(sin)
    needle.append_dev(q, s, xd, B, D, hd, cap * D, cap * heads, pd, cap, rope=(cd, sd) if rope else None)
    torch.cuda.synchronize()
    qh, sh = q.cpu().numpy(), s.cpu().numpy()
    for b in range(B):
        row = orc.rope(x[b], heads, hd, cos, sin, pos[b:b + 1]) if rope else x[b]
        wq, ws = orc.quantize_rows(row, D, hd)
        assert np.array_equal(qh[b, pos[b]], wq), b
        assert same_nan(sh[b, pos[b]], ws), b


def test_fused_append_nan_activation():
    # cq_gemms_append_dev: an activation row holding a NaN gives NaN product
    # rows (the lut bound keeps it), whose heads quantise to scale 1 and
    # codes 0; the other activations' appends are bit for bit the separate
    # append of their products
    import torch

    from go_whistle_amd import decoder as dec

    g = synth.rng(31)
    B, cap, D, hd = 4, 6, 512, 64
    heads = D // hd
    mk, mv = (cq.New(synth.random_packed(g, D, D, 128, 4, sigma=0.05)) for _ in range(2))
    x = g.standard_normal((B, D)).astype(np.float32)
    x[1, 300] = NAN
    x[3, 7] = INF
    pos = _t(np.array([0, 2, 5, 1], np.int32))
    cos, sin = (_t(a) for a in dec.rope_tables(hd, cap, 1e5))
    xd = _t(x)
    k, v = torch.zeros(B, D, device="cuda"), torch.zeros(B, D, device="cuda")
    caches = [[torch.zeros(B, cap, D, dtype=torch.int8, device="cuda"), torch.zeros(B, cap, heads, device="cuda")]
              for _ in range(4)]
    cq.gemms_append_dev([mk, mv], [k, v], xd, B, [(caches[0][0], caches[0][1], (cos, sin)),
                                                  (caches[1][0], caches[1][1], None)], cap * D, cap * heads, pos,
                        cap)
    k2, v2 = torch.zeros(B, D, device="cuda"), torch.zeros(B, D, device="cuda")
    cq.gemms_dev([mk, mv], [k2, v2], xd, B)
    needle.append_dev(caches[2][0], caches[2][1], k2, B, D, hd, cap * D, cap * heads, pos, cap, rope=(cos, sin))
    needle.append_dev(caches[3][0], caches[3][1], v2, B, D, hd, cap * D, cap * heads, pos, cap)
    torch.cuda.synchronize()
    assert same_nan(k.cpu().numpy(), k2.cpu().numpy()) and same_nan(v.cpu().numpy(), v2.cpu().numpy())
    kn = k.cpu().numpy()
    assert np.isnan(kn[1]).all() and np.isnan(kn[3]).all() and np.isfinite(kn[[0, 2]]).all()
    p = pos.cpu().numpy()
    for a, b in ((0, 2), (1, 3)):
        qa, sa = caches[a][0].cpu().numpy(), caches[a][1].cpu().numpy()
        assert np.array_equal(qa, caches[b][0].cpu().numpy()) and same_nan(sa, caches[b][1].cpu().numpy())
        for r in (1, 3):
            assert not qa[r, p[r]].any() and np.all(sa[r, p[r]] == 1)


def test_gemv_and_mfma_nan_inf():
    # the lut product (batch 1) and its MFMA form (many activations): a NaN
    # or Inf anywhere in an activation makes that activation's whole output
    # NaN (lut.go:239-282 with Go's max); the other activations stay bit for
    # bit the oracle's
    import torch

    g = synth.rng(12)
    for bits in (2, 4):
        p = synth.random_packed(g, 2048, 512, 128, bits, sigma=0.05)
        m, om = cq.New(p), orc.OMatrix.new(p)
        x = g.standard_normal(512).astype(np.float32)
        x[100] = NAN
        y = np.zeros(2048, np.float32)
        m.GEMV(y, x)
        assert np.isnan(y).all()
        rows = 128
        xs = g.standard_normal((rows, 512)).astype(np.float32)
        xs[5, 9], xs[64, 500], xs[100, 0] = NAN, INF, -INF
        want = om.gemm(xs.reshape(-1), rows).reshape(rows, 2048)
        assert np.isnan(want[[5, 64, 100]]).all()
        xd, yd = _t(xs), torch.zeros(rows, 2048, device="cuda")
        check(lib().cq_gemm_mfma_dev(m.handle, _p(yd), _p(xd), rows, cq._stream()))
        yl = torch.zeros(rows, 2048, device="cuda")
        m.gemm_dev(yl, xd, rows)
        torch.cuda.synchronize()
        assert same_nan(yd.cpu().numpy(), want)
        assert same_nan(yl.cpu().numpy(), want)


@pytest.mark.parametrize("form", ["tab2", "tab4", "split"])
def test_batched_forms_nan_inf_prologues(form):
    # NaN and +-Inf activations through the table form (2 and 4 bits) and
    # the split form, plain, behind the fused ZCRMSNorm prologue and behind
    # the gated input: each activation holding one gives NaN rows (Go's max
    # keeps the NaN bound, lut.go:239-282; the norm's and the gate's NaN
    # reach the bound the same way), the others the oracle's bits
    import torch

    if form == "split":
        out, inp, bits, rows = 512, 2048, 4, 1024
        path = "lut-mfma-split"
    else:
        out, inp, bits, rows = 2048, 512, int(form[-1]), 400
        path = "lut-mfma-tab"
    g = synth.rng(60 + len(form) + bits)
    p = synth.random_packed(g, out, inp, 128, bits, sigma=0.05)
    m, om = cq.New(p), orc.OMatrix.new(p)
    assert m.gemm_path(rows) == path
    x = _special_rows(g, rows, inp, every=7)
    gain = (1 + g.standard_normal(inp) * 0.1).astype(np.float32)
    gate = (g.standard_normal((rows, inp)) * 2).astype(np.float32)
    gate[3, 11], gate[10, 0] = NAN, -INF  # rows 3 and 10 hold no special x
    xd, gd = _t(x), _t(gate)
    y = torch.zeros(rows, out, device="cuda")
    m.gemm_dev(y, xd, rows)
    torch.cuda.synchronize()
    want = om.gemm(x.reshape(-1), rows).reshape(rows, out)
    assert np.isnan(want[0]).all() and np.isfinite(want[1]).all()
    assert same_nan(y.cpu().numpy(), want)
    cq.gemms_fused_dev([m], [y], xd, rows, norm_gain=_t(gain))
    torch.cuda.synchronize()
    want = om.gemm(orc.zc_rmsnorm(x.reshape(-1), gain, inp), rows).reshape(rows, out)
    assert same_nan(y.cpu().numpy(), want)
    cq.gemms_gated_dev([m], [y], xd, gd, rows)
    torch.cuda.synchronize()
    xs, _ = orc.sigmoid_gate(x.reshape(-1), gate.reshape(-1))
    want = om.gemm(xs, rows).reshape(rows, out)
    assert np.isnan(want[3]).all()
    assert same_nan(y.cpu().numpy(), want)


def _attend(q, t, heads, kq, ks, k_cols, qk, vq, vs, v_cols, vd, spans, nk, quant_q, batch, kv_stride, s_stride):
    import torch

    out = torch.zeros(batch * t * heads * vd, device="cuda")
    spd = _t(spans.astype(np.int32))
    needle.attend_int8_dev(out, _t(q), t, heads, _t(kq), _t(ks), k_cols, qk, _t(vq), _t(vs), v_cols, vd, spd, nk,
                           np.float32(math.sqrt(qk)), quant_q, batch=batch, q_stride=t * heads * qk,
                           kv_stride=kv_stride, s_stride=s_stride, out_stride=t * heads * vd)
    torch.cuda.synchronize()
    return out.cpu().numpy()


# (batch, heads, kv_heads, qk, vd, nk): the resident chain kernel (few
# streams), the ring (many streams of 64-code heads), the one-wavefront
# chain (48-code keys), the streamed kernel (128-code values), the general
# kernel (widths 20/40)
KERNEL_CASES = [(4, 8, 8, 64, 64, 300), (72, 8, 8, 64, 64, 200), (72, 8, 8, 48, 64, 120), (5, 4, 2, 64, 128, 150),
                (3, 4, 4, 20, 40, 90)]


@pytest.mark.parametrize("case", KERNEL_CASES, ids=["chain", "ring", "chain1", "stream128", "general"])
@pytest.mark.parametrize("quant_q", [True, False])
def test_attention_nan_inf(case, quant_q):
    # keys and values quantised from float rows with NaN and Inf (scale 1
    # and codes, or scale Inf and codes 0), queries with NaN and Inf; each
    # stream's output against the oracle's AttendInt8Spans
    batch, heads, kv_heads, qk, vd, nk = case
    g = synth.rng(batch * 10 + qk + quant_q)
    kf = _special_rows(g, batch * nk * kv_heads, qk, every=37)
    vf = _special_rows(g, batch * nk * kv_heads, vd, every=41)
    kq, ks = orc.quantize_rows(kf.reshape(-1), kv_heads * qk, qk)
    vq, vs = orc.quantize_rows(vf.reshape(-1), kv_heads * vd, vd)
    qf = g.standard_normal((batch, heads, qk)).astype(np.float32)
    for b in range(0, batch, 3):
        qf[b, b % heads, (b * 7) % qk] = [NAN, INF, -INF][(b // 3) % 3]
    spans = np.array([[0, 0, 0, 1 + (b * 53) % nk] for b in range(batch)], np.int32)
    kvs, ss = nk * kv_heads * qk, nk * kv_heads
    stride = nk * kv_heads * max(qk, vd)  # one stream stride for the keys and the values
    kpad = np.zeros(batch * stride, np.int8)
    vpad = np.zeros(batch * stride, np.int8)
    for b in range(batch):
        kpad[b * stride:b * stride + kvs] = kq[b * kvs:(b + 1) * kvs]
        vpad[b * stride:b * stride + nk * kv_heads * vd] = vq[b * nk * kv_heads * vd:(b + 1) * nk * kv_heads * vd]
    got = _attend(qf.reshape(-1), 1, heads, kpad, ks, kv_heads * qk, qk, vpad, vs, kv_heads * vd, vd, spans, nk,
                  quant_q, batch, stride, ss)
    nans = 0
    for b in range(batch):
        sl = slice(b * ss, (b + 1) * ss)
        want = orc.attend_int8_spans(qf[b].reshape(-1), 1, heads, kq[b * kvs:(b + 1) * kvs], ks[sl], kv_heads * qk,
                                     qk, vq[b * nk * kv_heads * vd:(b + 1) * nk * kv_heads * vd], vs[sl],
                                     kv_heads * vd, vd, nk, spans[b:b + 1], np.float32(math.sqrt(qk)), quant_q, 1)
        assert same_nan(got[b * heads * vd:(b + 1) * heads * vd], want), b
        nans += int(np.isnan(want).any())
    assert nans > 0  # the special values reach the outputs


def _streams(seed, batch, nk, heads, qk, vd, lengths, quant_q):
    g = synth.rng(seed)
    stride = nk * heads * max(qk, vd)
    kq = g.integers(-128, 128, size=batch * stride, dtype=np.int8)
    vq = g.integers(-128, 128, size=batch * stride, dtype=np.int8)
    ks = (g.random(batch * nk * heads) * 0.05 + 1e-4).astype(np.float32)
    vs = (g.random(batch * nk * heads) * 0.05 + 1e-4).astype(np.float32)
    q = g.standard_normal(batch * heads * qk).astype(np.float32)
    spans = np.array([[0, 0, 0, n] for n in lengths], np.int32)
    got = _attend(q, 1, heads, kq, ks, heads * qk, qk, vq, vs, heads * vd, vd, spans, nk, quant_q, batch, stride,
                  nk * heads)
    for b in range(batch):
        sl = slice(b * nk * heads, (b + 1) * nk * heads)
        want = orc.attend_int8_spans(q[b * heads * qk:(b + 1) * heads * qk], 1, heads,
                                     kq[b * stride:b * stride + nk * heads * qk], ks[sl], heads * qk, qk,
                                     vq[b * stride:b * stride + nk * heads * vd], vs[sl], heads * vd, vd, nk,
                                     spans[b:b + 1], np.float32(math.sqrt(qk)), quant_q, 1)
        assert np.array_equal(got[b * heads * vd:(b + 1) * heads * vd].view(np.uint32), want.view(np.uint32)), b


@pytest.mark.parametrize("batch", [9, 13, 250])
@pytest.mark.parametrize("vd", [64, 128])
def test_stream_counts_not_a_multiple_of_8(batch, vd):
    # the XCD-aware mapping serves streams in groups of 8; the last batch % 8
    # streams take its remainder branch. 9 and 13 streams run the resident
    # chain (or streamed) kernel, 250 the ring (or streamed ring) kernel.
    nk = 160 if vd == 64 else 96
    lengths = [1 + (b * 29) % nk for b in range(batch)]
    _streams(batch + vd, batch, nk, 8 if vd == 64 else 4, 64, vd, lengths, True)


def test_256_streams_self_attention_to_448():
    # config 4 at batch 256: each stream's causal self-attention over its own
    # length, spread over 1..448 (the ring kernel)
    batch, nk = 256, 448
    lengths = [1 + (b * 447) // (batch - 1) for b in range(batch)]
    assert lengths[0] == 1 and lengths[-1] == 448
    _streams(448, batch, nk, 8, 64, 64, lengths, True)


def test_shared_caches_read_through_the_index():
    # kv_attend_int8_shared_dev: stream b reads cache idx[b]; the output
    # equals the plain call on caches gathered per stream, and an index
    # outside the caches leaves the output untouched
    import torch

    g = synth.rng(99)
    caches, batch, heads, qk, nk = 5, 12, 8, 64, 300
    stride = nk * heads * qk
    kq = g.integers(-128, 128, size=caches * stride, dtype=np.int8)
    vq = g.integers(-128, 128, size=caches * stride, dtype=np.int8)
    ks = (g.random(caches * nk * heads) * 0.05 + 1e-4).astype(np.float32)
    vs = (g.random(caches * nk * heads) * 0.05 + 1e-4).astype(np.float32)
    q = g.standard_normal(batch * heads * qk).astype(np.float32)
    idx = np.array([3, 3, 0, 4, 1, 2, 2, 2, 0, 4, 7, -1], np.int32)  # the last two: outside the caches
    spans = np.array([[0, 0, 0, 1 + (b * 37) % nk] for b in range(batch)], np.int32)
    out = torch.full((batch * heads * qk,), 5.0, device="cuda")
    # every operand held until the kernel has run: a freed temporary's block
    # is handed to the next allocation
    held = [_t(a) for a in (q, kq, ks, vq, vs, spans, idx)]
    qd, kd, ksd, vd, vsd, spd, idd = held
    args = [_p(out), heads * qk, _p(qd), heads * qk, 1, heads, _p(kd), _p(ksd), heads * qk, qk, _p(vd), _p(vsd),
            heads * qk, qk, stride, nk * heads, _p(spd), nk, float(np.float32(8.0)), 1, batch]
    check(lib().kv_attend_int8_shared_dev(*args, _p(idd), caches, cq._stream()))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    del held
    for b in range(batch):
        o = got[b * heads * qk:(b + 1) * heads * qk]
        c = int(idx[b])
        if not 0 <= c < caches:
            assert np.all(o == 5.0), b
            continue
        sl = slice(c * nk * heads, (c + 1) * nk * heads)
        want = orc.attend_int8_spans(q[b * heads * qk:(b + 1) * heads * qk], 1, heads,
                                     kq[c * stride:(c + 1) * stride], ks[sl], heads * qk, qk,
                                     vq[c * stride:(c + 1) * stride], vs[sl], heads * qk, qk, nk, spans[b:b + 1],
                                     np.float32(8.0), True, 1)
        assert np.array_equal(o.view(np.uint32), want.view(np.uint32)), b
