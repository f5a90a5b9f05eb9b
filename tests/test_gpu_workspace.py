"""The table and split forms' device workspaces: products queued at the same
time on two streams of one thread, or from several threads, each bit for
bit the oracle's lut product (internal/cq/lut.go; a Matrix is safe for
concurrent use, internal/cq/matrix.go:22-24, and TestGEMMConcurrent runs
products side by side, internal/cq/cq_test.go:393-444); a product captured
into a graph before any product of its shape ran, replayed with other
products between the replays; and the pool's trim."""

import threading

import numpy as np
import pytest

from go_whistle_amd import cq, synth
from go_whistle_amd._lib import lib
from oracle import binding as orc

pytestmark = pytest.mark.gpu


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _case(seed, out, inp, bits, rows):
    g = synth.rng(seed)
    p = synth.random_packed(g, out, inp, 128, bits, sigma=0.05)
    x = g.standard_normal((rows, inp)).astype(np.float32)
    return p, x


@pytest.mark.parametrize("shape,path", [((2048, 512, 4, 1024), "lut-mfma-tab"),
                                        ((512, 2048, 4, 1024), "lut-mfma-split")])
def test_two_streams_one_thread(shape, path):
    # two products of one form, each on its own stream, queued back to back
    # from this thread without a wait between them, twice over: each output
    # equals its own oracle product
    import torch

    out, inp, bits, rows = shape
    cases = [_case(900 + k, out, inp, bits, rows) for k in range(2)]
    ms = [cq.New(p) for p, _ in cases]
    assert all(m.gemm_path(rows) == path for m in ms)
    xs = [torch.from_numpy(x).cuda() for _, x in cases]
    ys = [torch.full((rows, out), float("nan"), device="cuda") for _ in cases]
    streams = [torch.cuda.Stream() for _ in cases]
    torch.cuda.synchronize()
    for _ in range(2):
        for m, x, y, s in zip(ms, xs, ys, streams):
            with torch.cuda.stream(s):
                m.gemm_dev(y, x, rows)
    torch.cuda.synchronize()
    for (p, x), y in zip(cases, ys):
        want = orc.OMatrix.new(p).gemm(x.ravel(), rows, orc.LUT).reshape(rows, out)
        assert same(y.cpu().numpy(), want)


def test_threads_streams():
    # four threads, each with its own stream, each running table-form
    # products of its own matrix and input three times
    import torch

    rows, out, inp = 512, 2048, 512
    cases = [_case(950 + k, out, inp, 4 if k % 2 else 2, rows) for k in range(4)]
    ms = [cq.New(p) for p, _ in cases]
    assert all(m.gemm_path(rows) == "lut-mfma-tab" for m in ms)
    xs = [torch.from_numpy(x).cuda() for _, x in cases]
    ys = [torch.full((rows, out), float("nan"), device="cuda") for _ in cases]
    torch.cuda.synchronize()
    errors = []

    def run(k):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for _ in range(3):
                    ms[k].gemm_dev(ys[k], xs[k], rows)
            s.synchronize()
        except Exception as e:  # reported below
            errors.append(e)

    ts = [threading.Thread(target=run, args=(k,)) for k in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors
    torch.cuda.synchronize()
    for (p, x), y in zip(cases, ys):
        want = orc.OMatrix.new(p).gemm(x.ravel(), rows, orc.LUT).reshape(rows, out)
        assert same(y.cpu().numpy(), want)


def test_capture_first_product_and_trim():
    # a table-form product of a shape no product ran before (its workspace
    # is allocated during the capture), replayed three times with eager
    # products of other sizes queued between the replays; then the pool's
    # trim keeps the graph's workspace and the products still run
    import torch

    rows, out = 1777, 2048
    p, x = _case(977, out, 512, 2, rows)
    m = cq.New(p)
    assert m.gemm_path(rows) == "lut-mfma-tab"
    want = orc.OMatrix.new(p).gemm(x.ravel(), rows, orc.LUT).reshape(rows, out)
    p2, x2 = _case(978, out, 512, 4, 640)
    m2 = cq.New(p2)
    want2 = orc.OMatrix.new(p2).gemm(x2.ravel(), 640, orc.LUT).reshape(640, out)
    xd, x2d = torch.from_numpy(x).cuda(), torch.from_numpy(x2).cuda()
    y = torch.zeros(rows, out, device="cuda")
    y2 = torch.zeros(640, out, device="cuda")
    torch.cuda.synchronize()
    held0 = lib().cq_workspace_held()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        m.gemm_dev(y, xd, rows)
    assert lib().cq_workspace_held() > held0
    for k in range(3):
        y.fill_(float("nan"))
        g.replay()
        m2.gemm_dev(y2, x2d, 640)  # eager, on the current stream, between replays
        torch.cuda.synchronize()
        assert same(y.cpu().numpy(), want), k
        assert same(y2.cpu().numpy(), want2), k
    held = lib().cq_workspace_trim()
    assert 0 < held <= lib().cq_workspace_held()
    g.replay()
    m2.gemm_dev(y2, x2d, 640)
    torch.cuda.synchronize()
    assert same(y.cpu().numpy(), want) and same(y2.cpu().numpy(), want2)
