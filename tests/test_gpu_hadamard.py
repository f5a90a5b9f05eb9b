"""HadamardMLP on the device (nd_hadamard_mlp_dev) against the float64
restatement, within the reference test's bar of 1e-5
(internal/needle/hadamard_test.go:152-191): the test's own tiny block
(blocks 2 x 4, rank 3), Whistle's (16 x 32, rank 8), a model width padded
to the mix width, and several rows per launch."""

import numpy as np
import pytest

from go_whistle_amd import needle
from oracle import hadamard_ref as hr

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("na,nb,rank,dim,rows", [(2, 4, 3, 8, 3), (16, 32, 8, 512, 1), (16, 32, 8, 512, 256),
                                                  (16, 32, 8, 300, 5), (32, 32, 8, 768, 2)])
def test_hadamard_mlp_within_1e5(na, nb, rank, dim, rows):
    import torch

    print(f"HadamardMLP {na}x{nb} rank {rank} dim {dim} rows {rows}", flush=True)
    g = np.random.default_rng(na * 1000 + nb + rank + dim + rows)
    w = hr.random_weights(g, na, nb, rank, dim)
    x = (g.standard_normal((rows, dim)) * 1.5).astype(np.float32)
    h = needle.HadamardMLP(w)
    xd = torch.from_numpy(x).cuda()
    out = torch.full((rows, dim), float("nan"), device="cuda")
    h.forward_dev(out, xd, rows)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    want = hr.forward(w, x, rows)
    assert np.all(np.isfinite(got))
    assert np.max(np.abs(got - want)) <= 1e-5 * max(1.0, np.max(np.abs(want)))


def test_hadamard_mlp_misuse():
    from go_whistle_amd import CQPanic

    g = np.random.default_rng(9)
    w = hr.random_weights(g, 4, 8, 3)
    bad = dict(w)
    bad["p1"] = np.zeros(32, np.int32)
    with pytest.raises(CQPanic):
        needle.HadamardMLP(bad)
    w2 = hr.random_weights(g, 4, 8, 40)  # rank above 32
    import torch

    h = needle.HadamardMLP(w2)
    x = torch.zeros(1, 32, device="cuda")
    with pytest.raises(CQPanic):
        h.forward_dev(x, x, 1)
