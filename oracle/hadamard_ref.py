"""HadamardMLP (Whistle's Monarch FFN) restated in float64 numpy, one row at
a time, as architecture.py writes it and as go-whistle's own test
transcribes it (internal/needle/hadamard_test.go:74-150 refHadamard; the
block: internal/needle/hadamard.go:12-24, 172-310):

  cond = 1 + softmax(x @ cond_v) @ cond_u
  z1   = kron(d1 * x; w1a, w1b)[p1]
  z2   = kron(silu(d2 * cond * z1 + b2); w2a, w2b)[p2]
  out  = d4 * kron(d3 * z2; w3a, w3b)

with kron(z; a, b)[k*nb + l] = sum_ij z[i*nb + j] a[i, k] b[j, l] and x
zero-padded from the model width dim to n = na*nb (the output cut back to
dim). The reference computes in float32 with github.com/cwbudde/algo-tensor
v0.4.0 GEMMs (absent here), whose summation order its tests bound only to
1e-5 of this float64 form (hadamard_test.go:152-191); that bound is the
parity bar for the device kernel.

TEST INFRASTRUCTURE ONLY: the checker for nd_hadamard_mlp_dev.
"""

import numpy as np


def kron_apply(z, a, b):
    """z (na*nb) times a kron b: (a^T Z b) flattened, Z = z as na x nb."""
    na, nb = a.shape[0], b.shape[0]
    Z = np.asarray(z, np.float64).reshape(na, nb)
    return (np.asarray(a, np.float64).T @ Z @ np.asarray(b, np.float64)).reshape(-1)


def kron_dense(z, a, b):
    """The same product through np.kron's dense matrix: (a kron b)[i*nb + j,
    k*nb + l] = a[i, k] b[j, l] (hadamard_test.go:13-46)."""
    return np.asarray(z, np.float64) @ np.kron(np.asarray(a, np.float64), np.asarray(b, np.float64))


def forward(w, x, rows):
    """w: dict of d1, d2, b2, d3, d4 (n), w1a..w3b (square factors), cond_v
    (dim x rank), cond_u (rank x n), p1, p2 (permutations of n). x: rows x
    dim. Returns rows x dim, float64."""
    d1, d2, b2, d3, d4 = (np.asarray(w[k], np.float64) for k in ("d1", "d2", "b2", "d3", "d4"))
    cv, cu = np.asarray(w["cond_v"], np.float64), np.asarray(w["cond_u"], np.float64)
    fac = [(np.asarray(w[f"w{s}a"], np.float64), np.asarray(w[f"w{s}b"], np.float64)) for s in (1, 2, 3)]
    p1, p2 = np.asarray(w["p1"], np.int64), np.asarray(w["p2"], np.int64)
    n, dim = d1.size, cv.shape[0]
    x = np.asarray(x, np.float64).reshape(rows, dim)
    out = np.zeros((rows, dim))
    for r in range(rows):
        xi = np.zeros(n)
        xi[:dim] = x[r]
        logits = xi[:dim] @ cv
        e = np.exp(logits - logits.max())
        cond = 1.0 + (e / e.sum()) @ cu
        z = kron_apply(d1 * xi, *fac[0])[p1]
        a = d2 * cond * z + b2
        z = a / (1.0 + np.exp(-a))
        z = kron_apply(z, *fac[1])[p2]
        z = kron_apply(d3 * z, *fac[2])
        out[r] = (d4 * z)[:dim]
    return out


def random_weights(g, na, nb, rank, dim=None, scale=0.5):
    """Seeded weights of the block's shapes (dim defaults to n)."""
    n = na * nb
    dim = n if dim is None else dim
    w = {k: (1.0 + g.standard_normal(n) * 0.2).astype(np.float32) for k in ("d1", "d2", "d3", "d4")}
    w["b2"] = (g.standard_normal(n) * 0.1).astype(np.float32)
    for s in (1, 2, 3):
        w[f"w{s}a"] = (g.standard_normal((na, na)) * scale / np.sqrt(na)).astype(np.float32)
        w[f"w{s}b"] = (g.standard_normal((nb, nb)) * scale / np.sqrt(nb)).astype(np.float32)
    w["cond_v"] = (g.standard_normal((dim, rank)) * 0.6 / np.sqrt(dim)).astype(np.float32)
    w["cond_u"] = (g.standard_normal((rank, n)) * 0.6).astype(np.float32)
    w["p1"] = g.permutation(n).astype(np.int32)
    w["p2"] = g.permutation(n).astype(np.int32)
    return w
