"""The mHC pieces on the device (nd_rms_unit_dev, nd_mhc_heads_dev and its
stacked-logits form, nd_mhc_mix_dev) bit for bit the oracle (float64 exp-domain Sinkhorn with the
same exp; the log domain of huge logits within 1e-6), and within 1e-5 of
upstream's golden fixture (tests/golden/mhc_fixture.npz)."""

import os

import numpy as np
import pytest

from go_whistle_amd import needle
from oracle import binding as orc

pytestmark = pytest.mark.gpu
FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "mhc_fixture.npz")


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def same(a, b):
    a, b = np.asarray(a, np.float32).ravel(), np.asarray(b, np.float32).ravel()
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def run_device(pre, post, res, stream, block_out, rows, n, dim, affine=None):
    import torch

    hp, hq = torch.zeros(rows * n, device="cuda"), torch.zeros(rows * n, device="cuda")
    hr, u = torch.zeros(rows * n * n, device="cuda"), torch.zeros(rows * dim, device="cuda")
    sd = _t(stream)
    needle.mhc_heads_dev(hp, hq, hr, u, _t(pre), _t(post), _t(res), sd, rows, n, dim,
                         None if affine is None else _t(affine))
    out = torch.zeros(rows * n * dim, device="cuda")
    needle.mhc_mix_dev(out, sd, hr, hq, _t(block_out), u, rows, n, dim)
    nx = torch.zeros(rows * n * dim, device="cuda")
    needle.rms_unit_dev(nx, sd, rows, n * dim)
    torch.cuda.synchronize()
    return [t.cpu().numpy() for t in (hp, hq, hr, u, out, nx)]


@pytest.mark.parametrize("l", [0, 1])
def test_fixture_rows(l):
    f = np.load(FIX)
    L = lambda k: f[f"layer{l}__{k}"]
    stream = np.repeat(f["x"][0][:, None, :], 4, axis=1) if l == 0 else f["layer1__stream_in"][0]
    hp, hq, hr, u, out, nx = run_device(L("h_pre_logits"), L("h_post_logits"), L("h_res_logits"), stream,
                                        L("block_out"), 8, 4, 512)
    ohp, ohq, ohr, ou = orc.mhc_heads(L("h_pre_logits"), L("h_post_logits"), L("h_res_logits"), stream, 8, 4, 512)
    oout = orc.mhc_mix(stream, ohr, ohq, L("block_out"), ou, 8, 4, 512)
    for got, want in ((hp, ohp), (hq, ohq), (hr, ohr), (u, ou), (out, oout),
                      (nx, orc.rms_unit(stream.reshape(8, 2048), 8, 2048))):
        assert same(got, want)
    rel = lambda a, b: np.max(np.abs(a.ravel() - b.ravel())) / max(1.0, np.max(np.abs(b)))
    assert rel(out, L("stream_out")) <= 1e-5 and rel(hr, L("h_res")) <= 1e-5


@pytest.mark.parametrize("rows,n,dim,scale", [(5, 4, 512, 1.0), (3, 8, 96, 2.0), (2, 4, 64, 1e4)])
def test_random_rows_with_affine(rows, n, dim, scale):
    g = np.random.default_rng(rows * 100 + n)
    pre, post = g.standard_normal((rows, n)).astype(np.float32), g.standard_normal((rows, n)).astype(np.float32)
    res = (g.standard_normal((rows, n * n)) * scale).astype(np.float32)
    stream = g.standard_normal((rows, n, dim)).astype(np.float32)
    block_out = g.standard_normal((rows, dim)).astype(np.float32)
    affine = np.concatenate([[0.7, 1.3, 0.9], g.standard_normal(4 * n + n * n) * 0.5]).astype(np.float32)
    got = run_device(pre, post, res, stream, block_out, rows, n, dim, affine)
    ohp, ohq, ohr, ou = orc.mhc_heads(pre, post, res, stream, rows, n, dim, affine)
    oout = orc.mhc_mix(stream, ohr, ohq, block_out, ou, rows, n, dim)
    assert same(got[0], ohp) and same(got[1], ohq) and same(got[3], ou)
    if scale < 100:  # float64 exp domain: the same operations
        assert same(got[2], ohr) and same(got[4], oout)
    else:  # float32 log domain: the GPU's and the C library's log may differ in the last place
        assert np.max(np.abs(got[2] - ohr)) <= 1e-6
        assert np.max(np.abs(got[2].reshape(rows, n, n).sum(1) - 1)) <= 4e-7


@pytest.mark.parametrize("rows,n,dim,affine", [(7, 4, 512, True), (3, 8, 96, False), (1, 2, 64, True)])
def test_stacked_logits_equal_separate(rows, n, dim, affine):
    # nd_mhc_heads_stacked_dev reads row r's logits at r * (2n + n^2): pre,
    # post, res; the outputs are the separate arrays' bit for bit
    import torch

    g = np.random.default_rng(rows * 10 + n)
    pre, post = g.standard_normal((rows, n)).astype(np.float32), g.standard_normal((rows, n)).astype(np.float32)
    res = g.standard_normal((rows, n * n)).astype(np.float32)
    stream = g.standard_normal((rows, n, dim)).astype(np.float32)
    aff = np.concatenate([[0.7, 1.3, 0.9], g.standard_normal(4 * n + n * n) * 0.5]).astype(np.float32) if affine else None
    want = run_device(pre, post, res, stream, np.zeros((rows, dim), np.float32), rows, n, dim, aff)
    hp, hq = torch.zeros(rows * n, device="cuda"), torch.zeros(rows * n, device="cuda")
    hr, u = torch.zeros(rows * n * n, device="cuda"), torch.zeros(rows * dim, device="cuda")
    stacked = np.concatenate([pre, post, res], axis=1)
    needle.mhc_heads_stacked_dev(hp, hq, hr, u, _t(stacked), _t(stream), rows, n, dim, None if aff is None else _t(aff))
    torch.cuda.synchronize()
    for got, w in zip((hp, hq, hr, u), want[:4]):
        assert same(got.cpu().numpy(), w)


def test_mhc_misuse():
    import torch

    from go_whistle_amd import CQPanic

    z = torch.zeros(64, device="cuda")
    with pytest.raises(CQPanic):
        needle.mhc_heads_dev(z, z, z, z, z, z, z, z, 1, 9, 4)  # more than 8 lanes
    with pytest.raises(CQPanic):
        needle.mhc_heads_stacked_dev(z, z, z, z, z, z, 1, 9, 4)
    with pytest.raises(CQPanic):
        needle.mhc_mix_dev(z, z, z, z, z, z, 1, 4, 4)  # in place
