"""GPU parity of the int8 KV numerics with the CPU oracle, through the C
ABI: QuantizeRows codes and scales bit for bit, and AttendInt8Spans bit for
bit with amd64's softmax exponent, for decode self-attention over a causal
KV cache (1..448 keys), cross-attention over 1500 frames, GQA, windows with
a sink, and many streams at once. The launch picks between a kernel that
streams 16-byte-aligned value heads of 64 or 128 codes through LDS (all of
a stream's rows at once for small launches, a ring of chunks for large
ones) and a general kernel for other widths and alignments; every case
below names the path it reaches."""

import math

import numpy as np
import pytest

import go_whistle_amd as gw
from go_whistle_amd import needle, synth
from oracle import binding as orc

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("width", [48, 64, 17, 2048])
def test_quantize_rows_bit_exact(width):
    g = synth.rng(width)
    cols = width * 4
    rows = 37
    x = (g.standard_normal(rows * cols) * g.choice([1e-6, 1, 1e4], size=rows * cols)).astype(np.float32)
    x[: cols // 2] = 0  # zero chunks: scale 1
    x[cols * 3 + 5] = 127.0
    q, s = needle.QuantizeRows(x, cols, width)
    wq, ws = orc.quantize_rows(x, cols, width)
    assert np.array_equal(q, wq)
    assert same_bits(s, ws)


def test_quantize_hand_vectors():
    q, s = needle.QuantizeRow(np.array([127, 2.5, -2.5, 3.5, -0.5, 1.4999], np.float32))
    assert s == 1 and list(q) == [127, 2, -2, 4, 0, 1]
    q, s = needle.QuantizeRow(np.array([-6.35, 0.05, 3], np.float32))
    assert list(q) == [-127, 1, 60]


def _cache(g, n, kv_heads, qk, vd):
    kq, ks = orc.quantize_rows(g.standard_normal(n * kv_heads * qk).astype(np.float32), kv_heads * qk, qk)
    vq, vs = orc.quantize_rows(g.standard_normal(n * kv_heads * vd).astype(np.float32), kv_heads * vd, vd)
    return kq, ks, vq, vs


def _attend_gpu(q, t, heads, kq, ks, k_cols, qk, vq, vs, v_cols, vd, spans, nk_max, scale, quant_q, batch=1,
                q_stride=0, kv_stride=0, s_stride=0, out_stride=0):
    import torch

    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    out = torch.zeros(max(1, batch * (out_stride or t * heads * vd)), dtype=torch.float32, device="cuda")
    needle.attend_int8_dev(out, dev(q), t, heads, dev(kq), dev(ks), k_cols, qk, dev(vq), dev(vs), v_cols, vd,
                           dev(spans.astype(np.int32)), nk_max, scale, quant_q, batch=batch, out_stride=out_stride,
                           q_stride=q_stride, kv_stride=kv_stride, s_stride=s_stride)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("quant_q", [True, False])
@pytest.mark.parametrize("n", [1, 5, 8, 9, 37, 64, 447, 448])
def test_self_attention_decode_bit_exact(quant_q, n):
    heads, qk, vd = 8, 64, 64
    g = synth.rng(n + 7 * quant_q)
    kq, ks, vq, vs = _cache(g, n, heads, qk, vd)
    q = g.standard_normal(heads * qk).astype(np.float32)
    spans = np.array([[0, 0, 0, n]], np.int32)
    scale = np.float32(math.sqrt(qk))
    got = _attend_gpu(q, 1, heads, kq, ks, heads * qk, qk, vq, vs, heads * vd, vd, spans, n, scale, quant_q)
    want = orc.attend_int8_spans(q, 1, heads, kq, ks, heads * qk, qk, vq, vs, heads * vd, vd, n, spans, scale,
                                 quant_q, 1)
    assert same_bits(got[:want.size], want)


@pytest.mark.parametrize("quant_q", [True, False])
def test_cross_attention_1500_and_block_rows(quant_q):
    heads, qk, vd, n, t = 8, 64, 64, 1500, 3
    g = synth.rng(1500)
    kq, ks, vq, vs = _cache(g, n, heads, qk, vd)
    q = g.standard_normal(t * heads * qk).astype(np.float32)
    spans = np.array([[0, 0, 0, n]] * t, np.int32)
    got = _attend_gpu(q, t, heads, kq, ks, heads * qk, qk, vq, vs, heads * vd, vd, spans, n, 8.0, quant_q)
    want = orc.attend_int8_spans(q, t, heads, kq, ks, heads * qk, qk, vq, vs, heads * vd, vd, n, spans, 8.0,
                                 quant_q, 1)
    assert same_bits(got[:want.size], want)


def test_gqa_causal_and_windows():
    # Whistle's self-attention geometry: 8 query heads of 48 over 2 KV heads
    # (int8_test.go:212-284), causal rows, and a window with a sink.
    heads, kv_heads, qk, vd, n, t = 8, 2, 48, 64, 37, 3
    g = synth.rng(9)
    kq, ks, vq, vs = _cache(g, n, kv_heads, qk, vd)
    q = g.standard_normal(t * heads * qk).astype(np.float32)
    scale = np.float32(math.sqrt(qk))
    for spans in (np.array([[0, 0, 0, n - t + i + 1] for i in range(t)], np.int32),
                  np.array([[0, 2, 10 + i, 30 + i] for i in range(t)], np.int32)):
        for quant_q in (True, False):
            got = _attend_gpu(q, t, heads, kq, ks, kv_heads * qk, qk, vq, vs, kv_heads * vd, vd, spans, n, scale,
                              quant_q)
            want = orc.attend_int8_spans(q, t, heads, kq, ks, kv_heads * qk, qk, vq, vs, kv_heads * vd, vd, n, spans,
                                         scale, quant_q, 1)
            assert same_bits(got[:want.size], want)


def test_many_streams():
    # 16 independent streams (beam hypotheses), each its own cache length.
    heads, qk, vd, nk, batch = 8, 64, 64, 300, 16
    g = synth.rng(256)
    kqs, kss, vqs, vss, qs, spans = [], [], [], [], [], []
    for b in range(batch):
        kq, ks, vq, vs = _cache(g, nk, heads, qk, vd)
        kqs.append(kq); kss.append(ks); vqs.append(vq); vss.append(vs)
        qs.append(g.standard_normal(heads * qk).astype(np.float32))
        spans.append([0, 0, 0, 1 + (b * 37) % nk])
    spans = np.array(spans, np.int32)
    got = _attend_gpu(np.concatenate(qs), 1, heads, np.concatenate(kqs), np.concatenate(kss), heads * qk, qk,
                      np.concatenate(vqs), np.concatenate(vss), heads * vd, vd, spans, nk, 8.0, True, batch=batch,
                      q_stride=heads * qk, kv_stride=nk * heads * qk, s_stride=nk * heads, out_stride=heads * vd)
    for b in range(batch):
        want = orc.attend_int8_spans(qs[b], 1, heads, kqs[b], kss[b], heads * qk, qk, vqs[b], vss[b], heads * vd, vd,
                                     nk, spans[b:b + 1], 8.0, True, 1)
        assert same_bits(got[b * heads * vd:(b + 1) * heads * vd], want), b


def _streams_case(seed, batch, nk, heads, kv_heads, qk, vd, spans, quant_q, pad=0):
    """`batch` independent caches of nk rows with random codes and scales,
    in one device buffer per operand with a stream stride of
    nk * kv_heads * max(qk, vd) + pad codes; each stream's output is checked
    against the oracle bit for bit."""
    g = synth.rng(seed)
    width = max(qk, vd)
    stride = nk * kv_heads * width + pad
    kq = g.integers(-128, 128, size=batch * stride, dtype=np.int8)
    vq = g.integers(-128, 128, size=batch * stride, dtype=np.int8)
    ks = (g.random(batch * nk * kv_heads) * 0.05 + 1e-4).astype(np.float32)
    vs = (g.random(batch * nk * kv_heads) * 0.05 + 1e-4).astype(np.float32)
    q = g.standard_normal(batch * heads * qk).astype(np.float32)
    spans = np.asarray(spans, np.int32).reshape(batch, 4)
    got = _attend_gpu(q, 1, heads, kq, ks, kv_heads * qk, qk, vq, vs, kv_heads * vd, vd, spans, nk,
                      np.float32(math.sqrt(qk)), quant_q, batch=batch, q_stride=heads * qk, kv_stride=stride,
                      s_stride=nk * kv_heads, out_stride=heads * vd)
    for b in range(batch):
        kb = kq[b * stride: b * stride + nk * kv_heads * qk]
        vb = vq[b * stride: b * stride + nk * kv_heads * vd]
        sl = slice(b * nk * kv_heads, (b + 1) * nk * kv_heads)
        want = orc.attend_int8_spans(q[b * heads * qk:(b + 1) * heads * qk], 1, heads, kb, ks[sl], kv_heads * qk, qk,
                                     vb, vs[sl], kv_heads * vd, vd, nk, spans[b:b + 1], np.float32(math.sqrt(qk)),
                                     quant_q, 1)
        assert same_bits(got[b * heads * vd:(b + 1) * heads * vd], want), (b, spans[b])


def _lengths(nk, batch, seed):
    # chunk edges of the streamed kernel (48 and 64 keys), empty and full streams
    edge = [0, 1, 7, 8, 9, 47, 48, 49, 63, 64, 65, 95, 96, 97, 191, 192, 193, nk - 1, nk]
    g = synth.rng(seed)
    return [edge[b] if b < len(edge) else int(g.integers(0, nk + 1)) for b in range(batch)]


@pytest.mark.parametrize("quant_q", [True, False])
def test_streamed_ring_of_chunks(quant_q):
    # 72 streams x 8 heads = 576 workgroups: value rows go through a ring
    # of chunks, refilled ahead of the products (cross-attention shape).
    batch, nk, heads = 72, 1500, 8
    spans = []
    for b, n in enumerate(_lengths(nk, batch, 5)):
        if b % 5 == 4 and n > 120:  # attention sink plus a window
            spans.append([0, 4, n - 100, n])
        else:
            spans.append([0, 0, 0, n])
    _streams_case(72, batch, nk, heads, heads, 64, 64, spans, quant_q)


def test_streamed_all_rows_resident():
    # 16 streams x 8 heads: every value row of a stream in LDS at once.
    batch, nk = 16, 1500
    spans = [[0, 0, 0, n] for n in _lengths(nk, batch, 6)]
    _streams_case(16, batch, nk, 8, 8, 64, 64, spans, True)


@pytest.mark.parametrize("batch", [3, 160])
def test_streamed_value_heads_of_128(batch):
    # vd 128 (two chain wavefronts), GQA 4 heads over 2 KV heads; 3 streams
    # keep every row resident, 160 streams use the ring.
    nk = 300
    spans = [[0, 0, 0, n] for n in _lengths(nk, batch, 7)]
    _streams_case(128 + batch, batch, nk, 4, 2, 64, 128, spans, True)


@pytest.mark.parametrize("qk,vd,pad", [(20, 40, 0), (64, 64, 8), (48, 96, 0)])
def test_general_kernel_shapes(qk, vd, pad):
    # widths other than 64/128 codes, or streams off 16-byte alignment,
    # take the general kernel
    batch, nk = 5, 200
    spans = [[0, 0, 0, n] for n in _lengths(nk, batch, 8)]
    _streams_case(qk + vd + pad, batch, nk, 4, 4, qk, vd, spans, True, pad=pad)


def test_attend_misuse():
    import torch

    z = torch.zeros(64, dtype=torch.float32, device="cuda")
    with pytest.raises(gw.CQPanic):
        needle.attend_int8_dev(z, z, 1, 8, z, z, 100, 64, z, z, 512, 64, z, 1, 8.0, True)


@pytest.mark.parametrize("rows,cols,width", [(1, 512, 512), (37, 2048, 2048), (1500, 512, 64), (5, 96, 48)])
def test_fake_quant_bit_exact(rows, cols, width):
    # fakeQuant (int8.go:57-75) on the device against the oracle, in place
    # and out of place, with zero chunks (scale 1) and wide dynamic range
    import torch

    g = synth.rng(rows + cols + width)
    x = (g.standard_normal(rows * cols) * g.choice([1e-6, 1, 1e4], size=rows * cols)).astype(np.float32)
    x[:width] = 0
    want = orc.fake_quant(x, cols, width)
    xd = torch.from_numpy(x).cuda()
    out = torch.empty_like(xd)
    needle.fake_quant_dev(out, xd, rows, cols, width)
    needle.fake_quant_dev(xd, xd, rows, cols, width)
    torch.cuda.synchronize()
    assert same_bits(out.cpu().numpy(), want)
    assert same_bits(xd.cpu().numpy(), want)


@pytest.mark.parametrize("rows", [1, 375, 1500])
def test_linear_int8_input(rows):
    # needle.Linear WithInt8Input (linear.go:82-95): the mHC phi shape
    # (CQ4 128x2048) and a 512x512 CQ4, each input row fake-quantised, then
    # the lut product (its MFMA form when the grid is large), bit for bit
    # the oracle's; ApplyShared over quantising and plain linears equals
    # one Apply each (linear.go:97-145)
    import torch

    g = synth.rng(900 + rows)
    phi = gw.cq.New(synth.random_packed(g, 128, 2048, 128, 4, sigma=0.05))
    p2 = synth.random_packed(g, 512, 2048, 128, 4, sigma=0.05)
    m2 = gw.cq.New(p2)
    x = (g.standard_normal(rows * 2048) * 2).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    lin_q = needle.Linear(phi).WithInt8Input(True)
    lin_q2 = needle.Linear(m2, act8=True)
    lin_p = needle.Linear(m2)
    assert lin_q.Int8Input() and not lin_p.Int8Input()
    y = torch.zeros(rows * 128, device="cuda")
    lin_q.Apply(y, xd, rows)
    ys = [torch.zeros(rows * 128, device="cuda"), torch.zeros(rows * 512, device="cuda"),
          torch.zeros(rows * 512, device="cuda")]
    needle.ApplyShared(ys, xd, rows, lin_q, lin_p, lin_q2)
    y2q, y2p = torch.zeros(rows * 512, device="cuda"), torch.zeros(rows * 512, device="cuda")
    lin_q2.Apply(y2q, xd, rows)
    lin_p.Apply(y2p, xd, rows)
    torch.cuda.synchronize()
    xq = orc.fake_quant(x, 2048, 2048)
    o1 = orc.OMatrix.new(synth.random_packed(synth.rng(900 + rows), 128, 2048, 128, 4, sigma=0.05))
    want = o1.gemm(xq[: rows * 2048], rows)
    assert same_bits(y.cpu().numpy(), want)
    assert same_bits(ys[0].cpu().numpy(), want)
    assert same_bits(ys[1].cpu().numpy(), y2p.cpu().numpy())
    assert same_bits(ys[2].cpu().numpy(), y2q.cpu().numpy())
    o2 = orc.OMatrix.new(p2)
    assert same_bits(y2q.cpu().numpy(), o2.gemm(xq, rows))
    assert same_bits(y2p.cpu().numpy(), o2.gemm(x, rows))
