"""Seeded synthetic CQ matrices and activations.

random_packed follows the reference tests' recipe (internal/cq/cq_test.go:
20-41): uniform random index bytes, FP16 norms with exponents 11..19 (2^-4
.. 2^4) and random mantissas, and one sorted codebook per matrix. The
codebook is N(0, 1)/sqrt(G) as in the tests, or N(0, sigma) for the
benchmark shapes (one codebook of 2^bits levels per matrix: the .cact
layout, internal/cact/packed.go:18-29). Generators are numpy PCG64 streams.
"""

import numpy as np

from .cq import Packed


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def random_packed(g, out, inp, group, bits, sigma=None, width=None):
    width = bits if width is None else width
    groups = (inp + group - 1) // group
    row_bytes = groups * group * width // 8
    if sigma is None:
        cb = (g.standard_normal(1 << bits) / np.sqrt(group)).astype(np.float32)
    else:
        cb = (g.standard_normal(1 << bits) * sigma).astype(np.float32)
    cb = np.sort(cb)
    index = g.integers(0, 256, size=out * row_bytes, dtype=np.uint8)
    exp = g.integers(11, 20, size=out * groups).astype(np.uint16)
    man = g.integers(0, 1024, size=out * groups).astype(np.uint16)
    norms = ((exp << 10) | man).astype("<u2").view(np.uint8)
    return Packed(Out=out, In=inp, Group=group, Bits=bits, Width=width, Codebook=cb, Index=index, Norms=norms)


def activations(g, rows, inp, scale=1.0):
    return (g.standard_normal(rows * inp) * scale).astype(np.float32)


def heavy_vector(g, n):
    """Heavy tails (Gaussian cubed) and about one exact zero in 16, as the
    reference's asmVector (internal/cq/asm_test.go:19-38)."""
    v = g.standard_normal(n)
    v = v * v * v
    v[g.integers(0, 16, size=n) == 0] = 0
    return v.astype(np.float32)
