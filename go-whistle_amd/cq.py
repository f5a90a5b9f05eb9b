"""go-whistle's internal/cq Matrix API over libcqhip's C ABI.

Mirrors the Go surface (internal/cq/matrix.go:25-189, kernel.go:76-158):
New / NewGather, Out, In, Bits, Prepare, Bytes, Rows, Exact, Row, GEMV,
GEMM and GEMMs, with the same argument meaning. Construction errors raise
CQError (the Go error result), shape misuse raises CQPanic (the Go panic).
Host arrays are numpy float32; the *_dev methods take torch tensors that
live on the GPU and queue the work on torch's current stream.
"""

from dataclasses import dataclass
import ctypes
from ctypes import POINTER, c_float, c_size_t, c_uint8, c_void_p

import numpy as np

from ._lib import CQPanic, check, lib


@dataclass
class Packed:
    """cact.Packed (internal/cact/packed.go:18-29): a CQ tensor as stored."""

    Out: int
    In: int
    Group: int
    Bits: int
    Width: int
    Codebook: np.ndarray  # float32, 2^Bits levels
    Index: np.ndarray     # uint8, Out * RowBytes
    Norms: np.ndarray     # uint8, 2 * Out * Groups little-endian FP16

    def Groups(self):
        return (self.In + self.Group - 1) // self.Group

    def RowBytes(self):
        return self.Groups() * self.Group * self.Width // 8


def _fptr(a):
    return a.ctypes.data_as(POINTER(c_float))


def _f32(a):
    a = np.asarray(a)
    if a.dtype != np.float32 or not a.flags.c_contiguous:
        raise CQPanic("cq: float32 contiguous arrays expected")
    return a


def _stream():
    import torch

    return c_void_p(torch.cuda.current_stream().cuda_stream)


class Matrix:
    """A CQ matrix or view (internal/cq/matrix.go:25-41), on the device."""

    def __init__(self, handle):
        self._h = c_void_p(handle)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value and lib is not None:  # module globals are gone at interpreter exit
            lib().cq_free(h)
            self._h = None

    @property
    def handle(self):
        return self._h

    # --- construction (matrix.go:46-96) ---
    @staticmethod
    def _new(p: Packed, gather: bool):
        cb = np.ascontiguousarray(p.Codebook, dtype=np.float32)
        idx = np.ascontiguousarray(p.Index, dtype=np.uint8)
        nrm = np.ascontiguousarray(p.Norms, dtype=np.uint8)
        out = c_void_p()
        check(lib().cq_new(p.Out, p.In, p.Group, p.Bits, p.Width, _fptr(cb), cb.size,
                           idx.ctypes.data_as(POINTER(c_uint8)), idx.size, nrm.ctypes.data_as(POINTER(c_uint8)),
                           nrm.size, 1 if gather else 0, ctypes.byref(out)))
        return Matrix(out.value)

    def Out(self):
        return lib().cq_out(self._h)

    def In(self):
        return lib().cq_in(self._h)

    def Bits(self):
        return lib().cq_bits(self._h)

    def Prepare(self):
        check(lib().cq_prepare(self._h))

    def Bytes(self):
        return lib().cq_bytes(self._h)

    def DeviceBytes(self):
        return lib().cq_device_bytes(self._h)

    def Rows(self, lo, hi):
        v = c_void_p()
        check(lib().cq_rows(self._h, lo, hi, ctypes.byref(v)))
        return Matrix(v.value)

    def Exact(self):
        v = c_void_p()
        check(lib().cq_exact(self._h, ctypes.byref(v)))
        return Matrix(v.value)

    def Dense(self):
        """A view whose products of 16 or more activations run the dense fp32
        MFMA form of Exact's semantics (within float32 rounding of Exact,
        not bit for bit); fewer run Exact's nibble kernels. No counterpart
        in the reference."""
        v = c_void_p()
        check(lib().cq_dense(self._h, ctypes.byref(v)))
        return Matrix(v.value)

    def Kernel(self):
        return lib().cq_kernel_name(self._h).decode()

    # --- host-slice products ---
    def Row(self, dst, r):
        dst = _f32(dst)
        check(lib().cq_row(self._h, _fptr(dst), dst.size, r))

    def GEMV(self, dst, x):
        self.GEMM(dst, x, 1)

    def GEMM(self, dst, x, rows):
        dst, x = _f32(dst), _f32(x)
        check(lib().cq_gemm(self._h, _fptr(dst), dst.size, _fptr(x), x.size, rows))

    # --- device tensors (torch, on the GPU) ---
    def gemm_dev(self, y, x, rows):
        check(lib().cq_gemm_dev(self._h, c_void_p(y.data_ptr()), c_void_p(x.data_ptr()), rows, _stream()))

    def gemm_mfma_dev(self, y, x, rows):
        """The MFMA form of the lut product, whatever the grid size."""
        check(lib().cq_gemm_mfma_dev(self._h, c_void_p(y.data_ptr()), c_void_p(x.data_ptr()), rows, _stream()))

    def gemm_path(self, rows):
        """The kernel gemm_dev runs for `rows` activations."""
        return lib().cq_gemm_path(self._h, rows).decode()

    def row_dev(self, dst, r):
        check(lib().cq_row_dev(self._h, c_void_p(dst.data_ptr()), r, _stream()))

    def row_gather_dev(self, dst, rows_i32, scale=1.0):
        check(lib().cq_row_gather_dev(self._h, c_void_p(dst.data_ptr()), c_void_p(rows_i32.data_ptr()),
                                      int(rows_i32.numel()), float(scale), _stream()))


def New(p: Packed) -> Matrix:
    """cq.New (matrix.go:46-55)."""
    return Matrix._new(p, False)


def NewGather(p: Packed) -> Matrix:
    """cq.NewGather (matrix.go:60-96)."""
    return Matrix._new(p, True)


def GEMMs(ms, dsts, x, rows):
    """cq.GEMMs (kernel.go:134-158) on host arrays."""
    if len(ms) != len(dsts):
        raise CQPanic(f"cq: GEMMs of {len(ms)} matrices into {len(dsts)} outputs")
    n = len(ms)
    x = _f32(x)
    dsts = [_f32(d) for d in dsts]
    hs = (c_void_p * max(n, 1))(*[m.handle for m in ms])
    ds = (POINTER(c_float) * max(n, 1))(*[_fptr(d) for d in dsts])
    ls = (c_size_t * max(n, 1))(*[d.size for d in dsts])
    check(lib().cq_gemms(n, hs, ds, ls, _fptr(x), x.size, rows))


def gemms_dev(ms, ys, x, rows):
    """cq.GEMMs on device tensors."""
    n = len(ms)
    if n != len(ys):
        raise CQPanic(f"cq: GEMMs of {n} matrices into {len(ys)} outputs")
    hs = (c_void_p * max(n, 1))(*[m.handle for m in ms])
    ds = (c_void_p * max(n, 1))(*[c_void_p(y.data_ptr()) for y in ys])
    check(lib().cq_gemms_dev(n, hs, ds, c_void_p(x.data_ptr()), rows, _stream()))


def gemms_fused_dev(ms, ys, x, rows, norm_gain=None, resid=None, act=0):
    """gemms_dev with the input rows ZCRMSNorm'ed by norm_gain first, and
    the output y = resid + product (one matrix) or y = silu(product) (act 1)."""
    n = len(ms)
    if n != len(ys):
        raise CQPanic(f"cq: GEMMs of {n} matrices into {len(ys)} outputs")
    hs = (c_void_p * max(n, 1))(*[m.handle for m in ms])
    ds = (c_void_p * max(n, 1))(*[c_void_p(y.data_ptr()) for y in ys])
    ptr = lambda t: c_void_p(t.data_ptr()) if t is not None else None
    check(lib().cq_gemms_fused_dev(n, hs, ds, c_void_p(x.data_ptr()), rows, ptr(norm_gain), ptr(resid), act,
                                   _stream()))


def gemms_gated_dev(ms, ys, x, gate, rows, resid=None):
    """gemms_dev of x * sigmoid(gate) (Attention.output's gate before
    outProj.Apply, attention.go:242-260; gate is only read), and y = resid +
    product when resid is given (one matrix). One launch (cq_gemms_gated_dev)."""
    n = len(ms)
    if n != len(ys):
        raise CQPanic(f"cq: GEMMs of {n} matrices into {len(ys)} outputs")
    hs = (c_void_p * max(n, 1))(*[m.handle for m in ms])
    ds = (c_void_p * max(n, 1))(*[c_void_p(y.data_ptr()) for y in ys])
    ptr = lambda t: c_void_p(t.data_ptr()) if t is not None else None
    check(lib().cq_gemms_gated_dev(n, hs, ds, c_void_p(x.data_ptr()), ptr(gate), rows, ptr(resid), _stream()))


def gemms_append_dev(ms, ys, x, rows, caches, q_stride, s_stride, pos, cap, norm_gain=None):
    """gemms_fused_dev (norm_gain only) whose product k is also appended to
    an int8 row cache when caches[k] = (codes, scales, rope) is not None:
    row pos[b] of stream b's cache, each 64-wide head quantized as
    Int8Rows.Append, after RoPE at pos[b] when rope = (cos, sin) is given.
    One lut-kernel launch (cq_gemms_append_dev)."""
    n = len(ms)
    if not (n == len(ys) == len(caches)):
        raise CQPanic(f"cq: GEMMs of {n} matrices into {len(ys)} outputs and {len(caches)} caches")
    ptr = lambda t: c_void_p(t.data_ptr()) if t is not None else None
    arr = lambda vals: (c_void_p * max(n, 1))(*vals)
    hs = arr([m.handle for m in ms])
    ds = arr([ptr(y) for y in ys])
    kq = arr([ptr(c[0]) if c is not None else None for c in caches])
    ks = arr([ptr(c[1]) if c is not None else None for c in caches])
    rope = [c[2] if c is not None and c[2] is not None else None for c in caches]
    cs = arr([ptr(r[0]) if r is not None else None for r in rope])
    sn = arr([ptr(r[1]) if r is not None else None for r in rope])
    check(lib().cq_gemms_append_dev(n, hs, ds, c_void_p(x.data_ptr()), rows, ptr(norm_gain), kq, ks, q_stride,
                                    s_stride, ptr(pos), cap, cs, sn, _stream()))


def tables_bytes(ms, rows):
    """Bytes of the tables of the product over ms at `rows` activations that
    gemm_tables_dev can build in the previous product's launch, 0 when that
    product takes no table buffer (cq_tables_bytes)."""
    n = len(ms)
    hs = (c_void_p * max(n, 1))(*[m.handle for m in ms])
    return int(lib().cq_tables_bytes(n, hs, rows))


def gemm_tables_dev(m, y, x, rows, next_ms, tables, gate=None, resid=None, next_gain=None):
    """y = [resid +] m . (x [* sigmoid(gate)]), as gemms_gated_dev, and where
    its launch runs a workgroup per activation over all of m's rows, the
    tables of the next product over next_ms of ZCRMSNorm(y; next_gain) into
    the uint8 device tensor `tables` (tables_bytes(next_ms, rows) bytes; None:
    none asked). Returns True when the tables were built, else the next
    product runs unchained (cq_gemm_tables_dev)."""
    n = len(next_ms)
    hs = (c_void_p * max(n, 1))(*[q.handle for q in next_ms])
    ptr = lambda t: c_void_p(t.data_ptr()) if t is not None else None
    nbytes = tables.numel() * tables.element_size() if tables is not None else 0
    built = ctypes.c_int(0)
    check(lib().cq_gemm_tables_dev(m.handle, ptr(y), ptr(x), ptr(gate), rows, ptr(resid), n, hs, ptr(next_gain),
                                   ptr(tables), nbytes, ctypes.byref(built), _stream()))
    return bool(built.value)


def gemms_tables_dev(ms, ys, rows, tables, resid=None, act=0, caches=None, q_stride=0, s_stride=0, pos=None, cap=0):
    """The product over ms of the activations whose tables gemm_tables_dev
    built into `tables`, with gemms_fused_dev's residual add or SiLU and
    gemms_append_dev's appends (caches as there; None: none)
    (cq_gemms_tables_dev)."""
    n = len(ms)
    caches = caches if caches is not None else [None] * n
    if not (n == len(ys) == len(caches)):
        raise CQPanic(f"cq: GEMMs of {n} matrices into {len(ys)} outputs and {len(caches)} caches")
    ptr = lambda t: c_void_p(t.data_ptr()) if t is not None else None
    arr = lambda vals: (c_void_p * max(n, 1))(*vals)
    hs = arr([m.handle for m in ms])
    ds = arr([ptr(y) for y in ys])
    kq = arr([ptr(c[0]) if c is not None else None for c in caches])
    ks = arr([ptr(c[1]) if c is not None else None for c in caches])
    rope = [c[2] if c is not None and c[2] is not None else None for c in caches]
    cs = arr([ptr(r[0]) if r is not None else None for r in rope])
    sn = arr([ptr(r[1]) if r is not None else None for r in rope])
    nbytes = tables.numel() * tables.element_size()
    check(lib().cq_gemms_tables_dev(n, hs, ds, rows, ptr(resid), act, kq, ks, q_stride, s_stride, ptr(pos), cap, cs,
                                    sn, ptr(tables), nbytes, _stream()))


class Batch:
    """A plan of independent products on device tensors (cq_batch_*): job k
    is ms[k].GEMM of rows[k] activations xs[k] into ys[k]. run() queues one
    lut-kernel launch per kernel geometry on torch's current stream."""

    def __init__(self, ms, ys, xs, rows=None):
        n = len(ms)
        if not (len(ys) == len(xs) == n):
            raise CQPanic(f"cq: batch of {n} matrices, {len(ys)} outputs, {len(xs)} inputs")
        rows = [1] * n if rows is None else list(rows)
        self._keep = (list(ms), list(ys), list(xs))
        hs = (c_void_p * max(n, 1))(*[m.handle for m in ms])
        yp = (c_void_p * max(n, 1))(*[c_void_p(y.data_ptr()) for y in ys])
        xp = (c_void_p * max(n, 1))(*[c_void_p(x.data_ptr()) for x in xs])
        rp = (ctypes.c_int * max(n, 1))(*rows)
        h = c_void_p()
        check(lib().cq_batch_new(n, hs, yp, xp, rp, ctypes.byref(h)))
        self._h = h

    def run(self):
        check(lib().cq_batch_run(self._h, _stream()))

    def launches(self):
        return lib().cq_batch_launches(self._h)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value and lib is not None:  # module globals are gone at interpreter exit
            lib().cq_batch_free(h)
            self._h = None
