"""Independent float64 checks of the CQ product, after the reference's own
tests (internal/cq/cq_test.go:43-178): the explicit Sylvester Hadamard
dequantisation and the float32 error bounds of the rotated and the lut
products."""

import numpy as np

LUT_Q = 8191


def sylvester(n):
    """The ±1 Hadamard matrix of order n (cq_test.go:44-66)."""
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


def f16_norms(p):
    return p.Norms.view("<u2").astype(np.uint16).view(np.float16).astype(np.float64).reshape(p.Out, p.Groups())


def indices(p):
    """Every index of every row, LSB first, by numpy's bit unpacking."""
    bits = np.unpackbits(p.Index.reshape(p.Out, p.RowBytes()), axis=1, bitorder="little")
    bits = bits.reshape(p.Out, -1, p.Width)
    weights = (1 << np.arange(p.Width)).astype(np.int64)
    return (bits.astype(np.int64) * weights).sum(axis=2)  # [Out, Groups*Group]


def dequant64(p):
    """w[r, g] = H · cb[idx] · norm / √G cut to In, in float64 (cq_test.go:68-91)."""
    h = sylvester(p.Group)
    idx = indices(p)
    cb = p.Codebook.astype(np.float64)
    n = f16_norms(p)
    w = np.zeros((p.Out, p.Groups() * p.Group))
    for g in range(p.Groups()):
        c = cb[idx[:, g * p.Group:(g + 1) * p.Group]] * n[:, g:g + 1] / np.sqrt(p.Group)
        w[:, g * p.Group:(g + 1) * p.Group] = c @ h.T
    return w[:, :p.In]


def cosine(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(a @ b / np.sqrt((a @ a) * (b @ b)))


def rotated_bound(p, x):
    """cq_test.go:106-135."""
    k = p.Groups() * p.Group + np.log2(p.Group) + 8
    gamma = k * 2.0 ** -24 / (1 - k * 2.0 ** -24)
    idx = indices(p)
    cb = np.abs(p.Codebook.astype(np.float64))
    n = f16_norms(p)
    bound = np.zeros(p.Out)
    xa = np.abs(x.astype(np.float64))
    for g in range(p.Groups()):
        x_abs = xa[g * p.Group:min((g + 1) * p.Group, p.In)].sum()
        c_abs = cb[idx[:, g * p.Group:(g + 1) * p.Group]].sum(axis=1)
        bound += gamma * n[:, g] * c_abs * x_abs / np.sqrt(p.Group)
    return bound


def lut_bound(p, x):
    """cq_test.go:137-178."""
    h = sylvester(p.Group)
    cb_max = np.abs(p.Codebook.astype(np.float64)).max()
    n = f16_norms(p)
    bound = np.zeros(p.Out)
    per = p.Group * p.Bits / 4
    for g in range(p.Groups()):
        xg = np.zeros(p.Group)
        seg = x[g * p.Group:min((g + 1) * p.Group, p.In)].astype(np.float64)
        xg[:seg.size] = seg
        xt = h @ xg
        if p.Bits == 2:
            mx = np.max(np.abs(xt[0::2]) + np.abs(xt[1::2]))
        else:
            mx = np.max(np.abs(xt))
        bound += 1.01 * n[:, g] * per * cb_max * mx / (2 * LUT_Q * np.sqrt(p.Group))
    return bound


# Shapes of the reference's TestKernels (cq_test.go:183-191): one and several
# groups, padding down to one real column, groups 8 to 128.
TEST_SHAPES = [(1, 8, 8), (3, 16, 8), (4, 13, 8), (5, 40, 32), (7, 200, 128), (6, 384, 128), (9, 129, 128)]
