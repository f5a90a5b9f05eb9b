"""GPU parity of the CQ products with the CPU oracle, through the C ABI:
bit for bit for the lut kernel (Matrix.GEMM/GEMV), the Exact views'
nibble4/nibble kernels, Row, Rows views and GEMMs; the reference's panics,
the Bytes accounting and concurrent use (internal/cq/cq_test.go,
parallel_test.go, asm_test.go)."""

import threading

import numpy as np
import pytest

import go_whistle_amd as gw
from go_whistle_amd import cq, synth
from helpers import TEST_SHAPES
from oracle import binding as orc

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def gemm(m, x, rows):
    y = np.zeros(rows * m.Out(), np.float32)
    m.GEMM(y, x, rows)
    return y


def first_diff(a, b):
    d = np.nonzero(a.view(np.uint32) != b.view(np.uint32))[0]
    return (int(d[0]), float(a[d[0]]), float(b[d[0]]), d.size) if d.size else None


# The baseline sweep's matrices (4 and 16 levels ~N(0, 0.05)) at batch 1.
SWEEP = [(512, 512), (2048, 512), (512, 2048), (16384, 512)]


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("shape", SWEEP)
def test_lut_gemv_sweep_bit_exact(shape, bits):
    out, inp = shape
    print(f"lut GEMV {out}x{inp} CQ{bits}", flush=True)
    g = synth.rng(1000 + out + inp + bits)
    p = synth.random_packed(g, out, inp, 128, bits, sigma=0.05)
    m, o = cq.New(p), orc.OMatrix.new(p)
    assert m.Kernel() == "lut"
    for trial in range(3):
        x = synth.activations(g, 1, inp) if trial < 2 else synth.heavy_vector(g, inp)
        got = np.zeros(out, np.float32)
        m.GEMV(got, x)
        want = o.gemm(x, 1, orc.LUT)
        assert same_bits(got, want), first_diff(got, want)


@pytest.mark.parametrize("out,inp,bits", [(300, 4096, 4), (200, 4096, 2), (130, 384, 4), (130, 256, 2),
                                          (512, 2048, 4)])
def test_batch1_wide_units(out, inp, bits):
    """Few activations of a small matrix take the lut kernel's wide form (a
    wavefront per group, or two per group on half its units each, up to 16
    per workgroup); wide rows also run several chunks of groups. Bit for
    bit the oracle, also for views that cut blocks."""
    print(f"wide lut units {out}x{inp} CQ{bits}", flush=True)
    g = synth.rng(2000 + out + inp + bits)
    p = synth.random_packed(g, out, inp, 128, bits, sigma=0.05)
    m, o = cq.New(p), orc.OMatrix.new(p)
    for rows in (1, 2):
        x = synth.activations(g, rows, inp)
        got, want = gemm(m, x, rows), o.gemm(x, rows, orc.LUT)
        assert same_bits(got, want), (rows, first_diff(got, want))
        got = gemm(m.Rows(5, 69), x, rows)
        assert same_bits(got, o.rows(5, 69).gemm(x, rows, orc.LUT)), rows


@pytest.mark.parametrize("out,inp,bits,rows", [(512, 2048, 2, 256), (512, 512, 4, 128), (512, 512, 4, 48),
                                               (24, 2048, 4, 200), (2048, 512, 4, 48), (1536, 512, 2, 64),
                                               (600, 1024, 4, 40), (384, 512, 4, 100)])
def test_one_round_wide_units(out, inp, bits, rows):
    """Grids of at most one workgroup per CU take the wide form with units
    of 1-8 blocks: 16 wavefronts on 8 blocks two to a block (512x2048 at
    256), four or eight to a block, one per group of one block (24x2048),
    12 wavefronts on units of 3 blocks (384 rows at 100). Bit for bit the
    oracle, also for a view that cuts blocks."""
    print(f"one-round wide units {out}x{inp} CQ{bits} rows {rows}", flush=True)
    g = synth.rng(2500 + out + inp + bits + rows)
    p = synth.random_packed(g, out, inp, 128, bits, sigma=0.05)
    m, o = cq.New(p), orc.OMatrix.new(p)
    assert m.gemm_path(rows) == "lut"
    x = synth.activations(g, rows, inp)
    got, want = gemm(m, x, rows), o.gemm(x, rows, orc.LUT)
    assert same_bits(got, want), first_diff(got, want)
    lo, hi = 5, min(out, 5 + 300)
    got = gemm(m.Rows(lo, hi), x, rows)
    want = o.rows(lo, hi).gemm(x, rows, orc.LUT)
    assert same_bits(got, want), first_diff(got, want)


@pytest.mark.parametrize("shape", TEST_SHAPES)
@pytest.mark.parametrize("bits", [2, 4])
def test_small_shapes_all_kernels_bit_exact(shape, bits):
    # TestKernels' shapes: groups 8..128, padding to one real column; six
    # rows so that Exact runs nibble4 on four and nibble on two.
    out, inp, group = shape
    print(f"kernels {shape} CQ{bits}", flush=True)
    g = synth.rng(200 + out * 7 + bits)
    p = synth.random_packed(g, out, inp, group, bits)
    m, o = cq.New(p), orc.OMatrix.new(p)
    rows = 6
    x = synth.activations(g, rows, inp)
    assert same_bits(gemm(m, x, rows), o.gemm(x, rows, orc.LUT))
    e = m.Exact()
    assert e.Kernel() == "nibble4"
    got, want = gemm(e, x, rows), o.gemm(x, rows, orc.NIBBLE4)
    assert same_bits(got, want), first_diff(got, want)
    for r in range(out):
        row = np.zeros(inp, np.float32)
        m.Row(row, r)
        assert same_bits(row, o.row(r))


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("rows", [1, 3, 4, 5, 37])
def test_gemm_rows_and_exact(bits, rows):
    g = synth.rng(300 + rows + bits)
    p = synth.random_packed(g, 200, 512, 128, bits)
    m, o = cq.New(p), orc.OMatrix.new(p)
    x = synth.activations(g, rows, 512)
    assert same_bits(gemm(m, x, rows), o.gemm(x, rows, orc.LUT))
    assert same_bits(gemm(m.Exact(), x, rows), o.gemm(x, rows, orc.NIBBLE4))


def test_gemm_375_frames_and_wide_inputs():
    # q_proj over a 30 s clip and the 2048-wide φ input (cq/bench_test.go:23-38).
    g = synth.rng(375)
    # small launches take wide rows in chunks of 8 (4-bit) or 16 (2-bit) groups:
    # 1000 (8 groups, the last padded), 1280 (10: a chunk of 8, then 2) and
    # 2600 (21: 16, then 5) cover the last chunk's tail
    for out, inp, bits, rows in [(384, 512, 2, 375), (128, 2048, 4, 64), (96, 4096, 4, 3), (64, 8192, 2, 2),
                                 (33, 1000, 4, 1), (70, 1280, 4, 2), (200, 1280, 2, 1), (50, 2600, 2, 1)]:
        print(f"gemm {out}x{inp} CQ{bits} rows {rows}", flush=True)
        p = synth.random_packed(g, out, inp, 128, bits)
        m, o = cq.New(p), orc.OMatrix.new(p)
        x = synth.activations(g, rows, inp)
        got, want = gemm(m, x, rows), o.gemm(x, rows, orc.LUT)
        assert same_bits(got, want), first_diff(got, want)


def test_edge_values():
    # An all-zero group (M = 0), exact zeros, heavy tails and subnormal and
    # huge FP16 norms.
    g = synth.rng(41)
    p = synth.random_packed(g, 130, 384, 128, 4)
    nb = p.Norms.view("<u2").copy()
    nb[::7] = g.integers(1, 0x3FF, size=nb[::7].size)  # subnormal halves
    nb[3::11] = 0x7BFF  # 65504
    p.Norms = nb.view(np.uint8)
    m, o = cq.New(p), orc.OMatrix.new(p)
    x = synth.heavy_vector(g, 384)
    x[128:256] = 0
    for k, mm in ((orc.LUT, m), (orc.NIBBLE4, m.Exact())):
        got, want = gemm(mm, x, 1), o.gemm(x, 1, k)
        assert same_bits(got, want), (k, first_diff(got, want))


@pytest.mark.parametrize("bits", [2, 4])
def test_rows_views(bits):
    g = synth.rng(5 + bits)
    p = synth.random_packed(g, 170, 384, 128, bits)
    m, o = cq.New(p), orc.OMatrix.new(p)
    x = synth.activations(g, 3, 384)
    full = gemm(m, x, 3).reshape(3, 170)
    for lo, hi in [(0, 170), (5, 40), (33, 70), (64, 66), (63, 129), (100, 170)]:
        v = m.Rows(lo, hi)
        assert v.Out() == hi - lo
        part = gemm(v, x, 3).reshape(3, hi - lo)
        assert same_bits(part, full[:, lo:hi])
        assert same_bits(part, o.rows(lo, hi).gemm(x, 3, orc.LUT).reshape(3, hi - lo))
        ve = v.Exact()
        assert same_bits(gemm(ve, x, 3), o.rows(lo, hi).gemm(x, 3, orc.NIBBLE4))
        row = np.zeros(384, np.float32)
        v.Row(row, hi - lo - 1)
        assert same_bits(row, o.row(hi - 1))


def test_no_rows():
    # TestGEMMNoRows (cq_test.go:304-331)
    g = synth.rng(5)
    empty = cq.New(synth.random_packed(g, 0, 256, 128, 2))
    m = cq.New(synth.random_packed(g, 64, 256, 128, 4))
    x = synth.activations(g, 2, 256)
    for v in (empty, m.Rows(32, 32), m.Rows(5, 5)):
        v.GEMM(np.zeros(0, np.float32), x, 2)
        v.GEMV(np.zeros(0, np.float32), x[:256])
        v.Exact().GEMM(np.zeros(0, np.float32), x, 2)
    m.GEMM(np.zeros(0, np.float32), np.zeros(0, np.float32), 0)


def test_panics():
    # TestGEMMPanics (cq_test.go:587-610)
    m = cq.New(synth.random_packed(synth.rng(9), 4, 128, 128, 4))
    cases = [
        lambda: m.GEMV(np.zeros(4, np.float32), np.zeros(127, np.float32)),
        lambda: m.GEMV(np.zeros(3, np.float32), np.zeros(128, np.float32)),
        lambda: m.GEMM(np.zeros(8, np.float32), np.zeros(128, np.float32), 2),
        lambda: m.Row(np.zeros(128, np.float32), 4),
        lambda: m.Rows(3, 5),
    ]
    for c in cases:
        with pytest.raises(gw.CQPanic):
            c()


def test_gemms_matches_gemm():
    # TestGEMMsMatchesGEMM (parallel_test.go:101-168)
    g = synth.rng(382)
    cb = None
    mats = []
    for out in (384, 96, 96, 384):
        p = synth.random_packed(g, out, 512, 128, 2)
        if cb is None:
            cb = p.Codebook
        p.Codebook = cb
        mats.append(cq.New(p))
    other = cq.New(synth.random_packed(g, 64, 512, 128, 2))
    phi = cq.New(synth.random_packed(g, 72, 2048, 128, 4))
    sets = {"qkvg": mats, "phi": [phi.Rows(24, 28), phi.Rows(28, 32), phi.Rows(32, 48)],
            "mixed": [mats[0], other, mats[1]], "one": [mats[0]],
            "exact": [mats[0].Exact(), mats[1].Exact()]}
    for name, ms in sets.items():
        for rows in (0, 1, 3, 375):
            x = synth.activations(g, rows, ms[0].In())
            want = [gemm(m, x, rows) for m in ms]
            got = [np.zeros(rows * m.Out(), np.float32) for m in ms]
            cq.GEMMs(ms, got, x, rows)
            for a, b in zip(got, want):
                assert same_bits(a, b), (name, rows)


def test_new_gather_bytes_and_prepare():
    # TestNewGather / TestExact accounting (cq_test.go:446-559)
    g = synth.rng(17)
    p = synth.random_packed(g, 70, 384, 128, 2)
    eager = cq.New(p)
    packed = p.Index.size + 4 * 70 * 3 + 4 * 4
    for prepare in (False, True):
        lazy = cq.NewGather(p)
        assert lazy.Bytes() == packed
        r1, r2 = np.zeros(384, np.float32), np.zeros(384, np.float32)
        lazy.Row(r1, 41)
        eager.Row(r2, 41)
        assert same_bits(r1, r2)
        view = lazy.Rows(33, 63)
        if prepare:
            lazy.Prepare()
        x = synth.activations(g, 3, 384)
        assert same_bits(gemm(view, x, 3), gemm(eager.Rows(33, 63), x, 3))
        assert lazy.Bytes() == eager.Bytes()
    exact = cq.NewGather(p).Exact()
    exact.Prepare()
    assert exact.Bytes() == packed


def test_concurrent_views():
    # TestGEMMConcurrent (cq_test.go:393-444): 8 threads on shared views.
    g = synth.rng(15)
    p = synth.random_packed(g, 70, 384, 128, 4)
    shared = cq.New(p)
    views = [(0, 70), (5, 40), (33, 70), (64, 66)]
    x = synth.activations(g, 3, 384)
    want = {}
    for lo, hi in views:
        for ex in (False, True):
            v = shared.Rows(lo, hi)
            want[(lo, hi, ex)] = gemm(v.Exact() if ex else v, x, 3)
    errors = []

    def work(t):
        for n in range(20):
            lo, hi = views[(t + n) % len(views)]
            ex = n % 2 == 1
            v = shared.Rows(lo, hi)
            got = gemm(v.Exact() if ex else v, x, 3)
            if not same_bits(got, want[(lo, hi, ex)]):
                errors.append((t, lo, hi, ex))
                return

    threads = [threading.Thread(target=work, args=(t,)) for t in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors


def test_device_pointer_api_and_row_gather():
    import torch

    g = synth.rng(77)
    p = synth.random_packed(g, 1000, 512, 128, 4, sigma=0.05)
    m, o = cq.New(p), orc.OMatrix.new(p)
    x = synth.activations(g, 5, 512)
    xd = torch.from_numpy(x).cuda()
    yd = torch.zeros(5 * 1000, dtype=torch.float32, device="cuda")
    m.gemm_dev(yd, xd, 5)
    torch.cuda.synchronize()
    assert same_bits(yd.cpu().numpy(), o.gemm(x, 5, orc.LUT))
    rows = torch.tensor([3, 999, 0, 512, 3], dtype=torch.int32, device="cuda")
    dst = torch.zeros(5 * 512, dtype=torch.float32, device="cuda")
    m.row_gather_dev(dst, rows)
    torch.cuda.synchronize()
    got = dst.cpu().numpy().reshape(5, 512)
    for i, r in enumerate([3, 999, 0, 512, 3]):
        assert same_bits(got[i], o.row(r))


def test_batch_plan_matches_gemm():
    # Many independent products in one plan: every output equals the
    # matrix's own GEMM bit for bit, including Rows views and several rows.
    import torch

    g = synth.rng(4242)
    specs = [(512, 512, 4), (2048, 512, 4), (512, 2048, 4), (700, 512, 2), (130, 2048, 2), (64, 256, 4)]
    mats, os_, xs, ys, rows = [], [], [], [], []
    for k, (out, inp, bits) in enumerate(specs):
        p = synth.random_packed(g, out, inp, 128, bits, sigma=0.05)
        m = cq.New(p)
        if k == 3:
            m = m.Rows(33, 650)
        r = 1 if k % 2 == 0 else 3
        mats.append(m)
        os_.append(orc.OMatrix.new(p) if k != 3 else orc.OMatrix.new(p).rows(33, 650))
        xs.append(torch.from_numpy(synth.activations(g, r, inp)).cuda())
        ys.append(torch.full((r * m.Out(),), float("nan"), dtype=torch.float32, device="cuda"))
        rows.append(r)
    b = cq.Batch(mats, ys, xs, rows)
    assert b.launches() == 2  # one per (bits, group) geometry
    for rep in range(2):
        b.run()
        torch.cuda.synchronize()
        for k in range(len(specs)):
            want = os_[k].gemm(xs[k].cpu().numpy(), rows[k], orc.LUT)
            assert same_bits(ys[k].cpu().numpy(), want), (rep, k)


def test_batch_plan_many_units():
    # A plan larger than the resident grid: workgroups take byte-balanced
    # runs of blocks that cross job and activation boundaries (several units
    # per workgroup, tables rebuilt per unit, multi-chunk inputs). Every
    # output equals the matrix's own device GEMM bit for bit.
    import torch

    g = synth.rng(777)
    specs = [(16384, 512, 4), (2048, 512, 4), (512, 2048, 4), (512, 512, 4), (16384, 512, 2), (512, 2048, 2)]
    mats, xs, ys, rows = [], [], [], []
    for k in range(24):
        out, inp, bits = specs[k % len(specs)]
        m = cq.New(synth.random_packed(g, out, inp, 128, bits, sigma=0.05))
        r = 1 + (k % 3 == 1)
        mats.append(m)
        xs.append(torch.from_numpy(synth.activations(g, r, inp)).cuda())
        ys.append(torch.full((r * out,), float("nan"), dtype=torch.float32, device="cuda"))
        rows.append(r)
    b = cq.Batch(mats, ys, xs, rows)
    assert b.launches() == 2
    b.run()
    want = [torch.zeros_like(y) for y in ys]
    for m, w, x, r in zip(mats, want, xs, rows):
        m.gemm_dev(w, x, r)
    torch.cuda.synchronize()
    for k in range(len(mats)):
        assert torch.equal(ys[k].view(torch.int32), want[k].view(torch.int32)), k


def test_batch_plan_in_a_graph():
    import torch

    g = synth.rng(99)
    mats = [cq.New(synth.random_packed(g, 1024, 512, 128, 4, sigma=0.05)) for _ in range(3)]
    xs = [torch.from_numpy(synth.activations(g, 1, 512)).cuda() for _ in range(3)]
    ys = [torch.zeros(1024, dtype=torch.float32, device="cuda") for _ in range(3)]
    b = cq.Batch(mats, ys, xs)
    b.run()
    torch.cuda.synchronize()
    want = [y.clone() for y in ys]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        b.run()
    for rep in range(3):
        for y in ys:
            y.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for y, w in zip(ys, want):
            assert torch.equal(y.view(torch.int32), w.view(torch.int32)), rep
