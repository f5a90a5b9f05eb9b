"""Pins the float64 HadamardMLP restatement (oracle/hadamard_ref.py) by
checks that do not restate it: the Kronecker product against np.kron's
dense matrix (internal/needle/hadamard_test.go:13-46), and closed forms of
the whole block (identity factors and permutations, a conditioning that
cancels, zero padding to the mix width)."""

import numpy as np
import pytest

from oracle import hadamard_ref as hr


@pytest.mark.parametrize("na,nb", [(2, 3), (4, 4), (16, 32)])
def test_kron_apply_matches_dense(na, nb):
    g = np.random.default_rng(na * 100 + nb)
    a, b, z = g.standard_normal((na, na)), g.standard_normal((nb, nb)), g.standard_normal(na * nb)
    got, want = hr.kron_apply(z, a, b), hr.kron_dense(z, a, b)
    assert np.max(np.abs(got - want)) <= 1e-12 * max(1.0, np.max(np.abs(want)))


def _identity_block(n, na, nb, rank, dim):
    w = {k: np.ones(n, np.float32) for k in ("d1", "d2", "d3", "d4")}
    w["b2"] = np.zeros(n, np.float32)
    for s in (1, 2, 3):
        w[f"w{s}a"], w[f"w{s}b"] = np.eye(na, dtype=np.float32), np.eye(nb, dtype=np.float32)
    w["cond_v"] = np.zeros((dim, rank), np.float32)
    w["cond_u"] = np.zeros((rank, n), np.float32)
    w["p1"] = w["p2"] = np.arange(n, dtype=np.int32)
    return w


def test_identity_block_is_silu():
    """Identity factors and permutations, unit scales, no bias, cond = 1:
    out = silu(x) exactly as a closed form."""
    n, na, nb = 32, 4, 8
    w = _identity_block(n, na, nb, 3, n)
    x = np.random.default_rng(1).standard_normal((2, n))
    got = hr.forward(w, x, 2)
    assert np.allclose(got, x / (1 + np.exp(-x)), rtol=0, atol=1e-15)


def test_conditioning_and_permutations():
    """cond_u with equal rows gives cond = 1 + that row whatever the
    logits; a reversed p1 reverses z1; d4 scales the output."""
    n, na, nb, rank = 24, 4, 6, 5
    w = _identity_block(n, na, nb, rank, n)
    g = np.random.default_rng(2)
    row = g.standard_normal(n) * 0.3
    w["cond_u"] = np.tile(row, (rank, 1)).astype(np.float32)
    w["cond_v"] = g.standard_normal((n, rank)).astype(np.float32)
    w["p1"] = np.arange(n)[::-1].astype(np.int32)
    w["d4"] = np.full(n, 2.0, np.float32)
    x = g.standard_normal((1, n))
    a = (1.0 + row.astype(np.float32).astype(np.float64)) * x[0][::-1]
    want = 2.0 * a / (1 + np.exp(-a))
    assert np.allclose(hr.forward(w, x, 1)[0], want, rtol=0, atol=1e-12)


def test_padding_to_the_mix_width():
    """dim < n: x zero-padded, the output the first dim values of the
    full-width block run on the padded row."""
    g = np.random.default_rng(3)
    na, nb, rank, dim = 4, 8, 3, 20
    w = hr.random_weights(g, na, nb, rank, dim)
    x = g.standard_normal((2, dim))
    wf = dict(w)
    wf["cond_v"] = np.zeros((na * nb, rank), np.float32)
    wf["cond_v"][:dim] = w["cond_v"]
    xf = np.zeros((2, na * nb))
    xf[:, :dim] = x
    assert np.allclose(hr.forward(w, x, 2), hr.forward(wf, xf, 2)[:, :dim], rtol=0, atol=1e-13)
