"""GPU parity of the MFMA form of the lut product (many activations,
group 128) with the CPU oracle's lut GEMM, bit for bit, through the C ABI.
cq_gemm_mfma_dev runs it whatever the size; cq_gemm_dev picks it when the
grid is large. Covers the encoder's batched shapes (FFN up/down at 2 and 4
bits), rows that do not fill a workgroup, activation counts that do not fill
a tile, Rows views that start mid-block, GEMMs over shared inputs, edge
values, and the full 12000-frame batch, checked on sampled activations
(each activation's product is independent of the others)."""

import numpy as np
import pytest

import go_whistle_amd as gw
from go_whistle_amd import cq, synth
from oracle import binding as orc

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def first_diff(a, b):
    d = np.nonzero(np.asarray(a, np.float32).view(np.uint32) != np.asarray(b, np.float32).view(np.uint32))[0]
    return (int(d[0]), float(a[d[0]]), float(b[d[0]]), d.size) if d.size else None


def mfma_gemm(m, x, rows):
    import torch

    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32).reshape(rows, -1)).cuda()
    y = torch.zeros(rows, m.Out(), dtype=torch.float32, device="cuda")
    m.gemm_mfma_dev(y, xd, rows)
    torch.cuda.synchronize()
    return y.cpu().numpy().ravel()


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("out,inp,rows", [(2048, 512, 64), (512, 2048, 130), (700, 384, 97), (200, 512, 300),
                                          (64, 128, 65), (16384, 512, 256), (512, 512, 1)])
def test_mfma_gemm_bit_exact(bits, out, inp, rows):
    print(f"mfma gemm CQ{bits} {out}x{inp} rows {rows}", flush=True)
    g = synth.rng(out + inp + rows + bits)
    p = synth.random_packed(g, out, inp, 128, bits, sigma=0.05)
    m, o = cq.New(p), orc.OMatrix.new(p)
    x = synth.activations(g, rows, inp)
    got, want = mfma_gemm(m, x, rows), o.gemm(x, rows, orc.LUT)
    assert same_bits(got, want), first_diff(got, want)


@pytest.mark.parametrize("bits", [2, 4])
def test_mfma_edge_values(bits):
    # all-zero groups (M = 0), exact zeros, heavy tails, subnormal and huge
    # FP16 norms, codebooks with repeated and extreme levels
    g = synth.rng(77 + bits)
    p = synth.random_packed(g, 330, 640, 128, bits)
    nb = p.Norms.view("<u2").copy()
    nb[::7] = g.integers(1, 0x3FF, size=nb[::7].size)
    nb[3::11] = 0x7BFF
    p.Norms = nb.view(np.uint8)
    cb = p.Codebook.copy()
    cb[1] = cb[0]
    cb[-1] = np.float32(3.5)
    p.Codebook = np.sort(cb).astype(np.float32)
    m, o = cq.New(p), orc.OMatrix.new(p)
    rows = 90
    x = np.concatenate([synth.heavy_vector(g, 640) for _ in range(rows)]).astype(np.float32)
    x[5 * 640 + 128: 5 * 640 + 256] = 0      # one activation's group all zero
    x[7 * 640: 8 * 640] = 0                   # one activation all zero
    x[::13] = 0
    got, want = mfma_gemm(m, x, rows), o.gemm(x, rows, orc.LUT)
    assert same_bits(got, want), first_diff(got, want)


@pytest.mark.parametrize("bits", [2, 4])
def test_mfma_rows_views(bits):
    g = synth.rng(500 + bits)
    p = synth.random_packed(g, 600, 512, 128, bits)
    m, o = cq.New(p), orc.OMatrix.new(p)
    rows = 80
    x = synth.activations(g, rows, 512)
    for lo, hi in ((0, 600), (37, 301), (64, 128), (250, 600), (599, 600)):
        got = mfma_gemm(m.Rows(lo, hi), x, rows)
        want = o.rows(lo, hi).gemm(x, rows, orc.LUT)
        assert same_bits(got, want), (lo, hi, first_diff(got, want))


def test_mfma_gemms_shared_input():
    # q, k, v over one input (ApplyShared) at 13000 frames (past the table
    # form): one MFMA launch for the three matrices, each bit for bit its own
    # GEMM (sampled frames).
    import torch

    g = synth.rng(808)
    ps = [synth.random_packed(g, out, 512, 128, 4, sigma=0.05) for out in (2048, 1024, 1536)]
    for p in ps[1:]:
        p.Codebook = ps[0].Codebook.copy()
    ms = [cq.New(p) for p in ps]
    rows = 13000
    assert ms[0].gemm_path(rows) == "lut-mfma"
    x = g.standard_normal((rows, 512)).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    ys = [torch.zeros(rows, p.Out, dtype=torch.float32, device="cuda") for p in ps]
    cq.gemms_dev(ms, ys, xd, rows)
    torch.cuda.synchronize()
    pick = np.array([0, 1, 63, 64, 700, 1437, 1499, 2048, 3999, 12287, 12999])
    for p, y in zip(ps, ys):
        want = orc.OMatrix.new(p).gemm(x[pick].ravel(), len(pick), orc.LUT).reshape(len(pick), p.Out)
        got = y.cpu().numpy()[pick]
        assert same_bits(got, want), first_diff(got.ravel(), want.ravel())


def test_mfma_path_choice_and_misuse():
    import torch

    g = synth.rng(9)
    m = cq.New(synth.random_packed(g, 2048, 512, 128, 4))
    # the lut kernel per activation for few activations, the table form at
    # some hundred to 12288 over 2048 rows, the 512-row form beyond
    assert m.gemm_path(1) == "lut" and m.gemm_path(256) == "lut-mfma-tab"
    assert m.gemm_path(375) == "lut-mfma-tab" and m.gemm_path(12000) == "lut-mfma-tab"
    assert m.gemm_path(12289) == "lut-mfma"
    assert m.Exact().gemm_path(12000) == "nibble4"
    z = torch.zeros(64 * 2048, dtype=torch.float32, device="cuda")
    with pytest.raises(gw.CQDeviceError):  # not a lut view
        m.Exact().gemm_mfma_dev(z, z, 1)
    m64 = cq.New(synth.random_packed(g, 64, 256, 64, 4))
    with pytest.raises(gw.CQDeviceError):  # group 64
        m64.gemm_mfma_dev(z, z, 1)
    with pytest.raises(gw.CQPanic):
        m.gemm_mfma_dev(z, z, -1)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("rows,path", [(12000, "lut-mfma-tab"), (12800, "lut-mfma")])
def test_mfma_12000_frames_sampled(bits, rows, path):
    # The encoder's 8-utterance batch: 12000 activations through the device
    # pointer API (the table form), and 12800 (the 512-row MFMA form); 40
    # sampled activations against the oracle.
    import torch

    g = synth.rng(rows + bits)
    p = synth.random_packed(g, 2048, 512, 128, bits, sigma=0.05)
    m, o = cq.New(p), orc.OMatrix.new(p)
    assert m.gemm_path(rows) == path
    x = g.standard_normal((rows, 512)).astype(np.float32)
    y = torch.zeros(rows, 2048, dtype=torch.float32, device="cuda")
    m.gemm_dev(y, torch.from_numpy(x).cuda(), rows)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    pick = np.sort(g.choice(rows, size=40, replace=False))
    pick[0], pick[-1] = 0, rows - 1
    want = o.gemm(x[pick].ravel(), len(pick), orc.LUT).reshape(len(pick), 2048)
    assert same_bits(got[pick], want), first_diff(got[pick].ravel(), want.ravel())
