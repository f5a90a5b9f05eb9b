"""MI355X (gfx950) implementation of go-whistle's CQ quantized-matrix path.

The product is libcqhip.so (csrc/, C ABI in include/cqhip.h): the packed
2/4-bit CQ codebook-LUT GEMV/GEMM of internal/cq and the int8 KV numerics
of internal/needle, as hand-written HIP kernels. This package is the
Python mirror of the reference's Go API over that ABI (cq, needle), a
seeded synthetic-data generator (synth) and the build step (build).
"""

from ._lib import CQDeviceError, CQError, CQPanic, lib  # noqa: F401
from . import cq, needle, synth  # noqa: F401
