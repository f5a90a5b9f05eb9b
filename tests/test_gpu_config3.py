"""The batched products the benchmark times on encoder-frame activations,
at their own shapes, against the oracle's lut GEMM (internal/cq/lut.go:
88-156, the fold in group order at lut.go:289-313): 2048x512 at 1500
activations on the table form, compared in full; 512x2048 at 12000
activations on the 512-row MFMA form, compared on 48 sampled activations
that include the first and last 32- and 64-activation tiles."""

import numpy as np
import pytest

from go_whistle_amd import cq, synth
from oracle import binding as orc

pytestmark = pytest.mark.gpu


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def first_diff(a, b):
    bad = np.flatnonzero(a.view(np.uint32) != b.view(np.uint32))
    return (int(bad[0]), float(a[bad[0]]), float(b[bad[0]]), len(bad)) if len(bad) else None


@pytest.mark.parametrize("bits", [4, 2])
def test_ffn_up_1500_frames_full(bits):
    import torch

    rows = 1500
    g = synth.rng(31500 + bits)
    p = synth.random_packed(g, 2048, 512, 128, bits, sigma=0.05)
    m = cq.New(p)
    assert m.gemm_path(rows) == "lut-mfma-tab"
    x = g.standard_normal((rows, 512)).astype(np.float32)
    y = torch.full((rows, 2048), float("nan"), device="cuda")
    m.gemm_dev(y, torch.from_numpy(x).cuda(), rows)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    want = orc.OMatrix.new(p).gemm(x.ravel(), rows, orc.LUT).reshape(rows, 2048)
    assert same(got, want), first_diff(got.ravel(), want.ravel())


@pytest.mark.parametrize("bits", [4, 2])
def test_ffn_down_12000_frames_sampled(bits):
    import torch

    rows = 12000
    g = synth.rng(312000 + bits)
    p = synth.random_packed(g, 512, 2048, 128, bits, sigma=0.05)
    m = cq.New(p)
    assert m.gemm_path(rows) == "lut-mfma"
    x = g.standard_normal((rows, 2048)).astype(np.float32)
    y = torch.full((rows, 512), float("nan"), device="cuda")
    m.gemm_dev(y, torch.from_numpy(x).cuda(), rows)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    edges = [0, 1, 31, 32, 63, 64, rows - 65, rows - 64, rows - 33, rows - 32, rows - 1]
    rest = g.choice(np.setdiff1d(np.arange(rows), edges), size=48 - len(edges), replace=False)
    pick = np.sort(np.concatenate([edges, rest]))
    assert len(pick) == 48
    want = orc.OMatrix.new(p).gemm(x[pick].ravel(), len(pick), orc.LUT).reshape(len(pick), 512)
    assert same(got[pick], want), first_diff(got[pick].ravel(), want.ravel())
    assert not np.isnan(got).any()
