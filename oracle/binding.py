"""ctypes binding of the CPU oracle (liboracle.so, oracle.h).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.
"""

import ctypes
import os
from ctypes import POINTER, Structure, c_char_p, c_float, c_int, c_int8, c_int32, c_size_t, c_uint8, c_uint16, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

GATHER, NIBBLE, NIBBLE4, LUT = 0, 1, 2, 3


class _Packed(Structure):
    _fields_ = [("out", c_int), ("in_", c_int), ("group", c_int), ("bits", c_int), ("width", c_int),
                ("codebook", POINTER(c_float)), ("index", POINTER(c_uint8)), ("norms", POINTER(c_uint8)),
                ("index_len", c_size_t), ("norms_len", c_size_t), ("codebook_len", c_size_t)]


class DecModel(Structure):
    """orc_dec_model (oracle.h)."""
    _fields_ = [("vocab", c_int), ("dim", c_int), ("heads", c_int), ("head_dim", c_int), ("ffn", c_int),
                ("layers", c_int), ("frames", c_int), ("max_pos", c_int), ("taps", c_int), ("qk_norm", c_int),
                ("post_norm", c_int), ("cross_norm", c_int), ("lanes", c_int), ("scale", c_float),
                ("emb", c_void_p), ("mats", POINTER(c_void_p)), ("gains", POINTER(c_float)),
                ("rope_cos", POINTER(c_float)), ("rope_sin", POINTER(c_float)), ("qk_gains", POINTER(c_float)),
                ("post_gains", POINTER(c_float)), ("res_scale", POINTER(c_float)), ("taps_w", POINTER(c_float)),
                ("mhc_affine", POINTER(c_float))]


class DecMemory(Structure):
    """orc_dec_memory (oracle.h)."""
    _fields_ = [("kq", POINTER(c_void_p)), ("ks", POINTER(c_void_p)), ("vq", POINTER(c_void_p)),
                ("vs", POINTER(c_void_p))]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built ({LIB_PATH}): make -C oracle")
        lb = ctypes.CDLL(LIB_PATH)
        sig = {
            "orc_f16_to_f32": (c_float, [c_uint16]),
            "orc_f16_to_f32_n": (None, [POINTER(c_float), POINTER(c_uint16), c_size_t]),
            "orc_unpack_lsb": (None, [POINTER(c_uint8), POINTER(c_uint8), c_int, c_int]),
            "orc_fwht": (None, [POINTER(c_float), c_int]),
            "orc_cq_dequant": (c_int, [POINTER(c_float), POINTER(_Packed)]),
            "orc_new": (c_void_p, [POINTER(_Packed), c_char_p, c_size_t]),
            "orc_free": (None, [c_void_p]),
            "orc_rows": (c_void_p, [c_void_p, c_int, c_int]),
            "orc_out": (c_int, [c_void_p]),
            "orc_in": (c_int, [c_void_p]),
            "orc_gemm": (c_int, [c_void_p, c_int, POINTER(c_float), POINTER(c_float), c_int]),
            "orc_gemms": (c_int, [POINTER(c_void_p), c_int, c_int, POINTER(POINTER(c_float)), POINTER(c_float), c_int]),
            "orc_row": (c_int, [c_void_p, POINTER(c_float), c_int]),
            "orc_lut_tables2": (c_float, [POINTER(c_uint8), POINTER(c_float), c_int, POINTER(c_float), c_float]),
            "orc_lut_tables4": (c_float, [POINTER(c_uint8), POINTER(c_float), c_int, POINTER(c_float), c_float]),
            "orc_lut_lookup": (None, [POINTER(c_float), POINTER(c_uint8), POINTER(c_uint8), POINTER(c_float),
                                      POINTER(c_float), c_int, c_int, c_int]),
            "orc_lut_step": (c_float, [c_int]),
            "orc_have_avx2": (c_int, []),
            "orc_fwht_avx2": (None, [POINTER(c_float), c_int]),
            "orc_lut_tables2_avx2": (c_float, [POINTER(c_uint8), POINTER(c_float), c_int, POINTER(c_float), c_float]),
            "orc_lut_tables4_avx2": (c_float, [POINTER(c_uint8), POINTER(c_float), c_int, POINTER(c_float), c_float]),
            "orc_lut_lookup_avx2": (None, [POINTER(c_float), POINTER(c_uint8), POINTER(c_uint8), POINTER(c_float),
                                           POINTER(c_float), c_int, c_int, c_int]),
            "orc_set_cpu": (c_int, [c_int, c_int]),
            "orc_dots_i8_avx2": (None, [POINTER(c_int32), c_int, POINTER(c_int8), c_int, POINTER(c_int8), c_int]),
            "orc_axpys_i8_avx2": (None, [POINTER(c_float), c_int, POINTER(c_float), c_int, POINTER(c_int8), c_int]),
            "orc_exp_sub_sum_avx2": (c_float, [POINTER(c_float), c_int, c_float]),
            "orc_quantize_row": (c_float, [POINTER(c_int8), POINTER(c_float), c_int]),
            "orc_quantize_rows": (None, [POINTER(c_int8), POINTER(c_float), POINTER(c_float), c_int, c_int, c_int]),
            "orc_fake_quant": (None, [POINTER(c_float), POINTER(c_float), ctypes.c_long, c_int, c_int]),
            "orc_dots_i8": (None, [POINTER(c_int32), c_int, POINTER(c_int8), c_int, POINTER(c_int8), c_int]),
            "orc_axpys_i8": (None, [POINTER(c_float), c_int, POINTER(c_float), c_int, POINTER(c_int8), c_int]),
            "orc_dots_f32_i8": (None, [POINTER(c_float), c_int, POINTER(c_float), c_int, POINTER(c_int8), c_int]),
            "orc_exp_sub_sum": (c_float, [POINTER(c_float), c_int, c_float, c_int]),
            "orc_softmax": (None, [POINTER(c_float), c_int, c_int]),
            "orc_exp_lane": (c_float, [c_float]),
            "orc_zc_rmsnorm": (None, [POINTER(c_float), POINTER(c_float), POINTER(c_float), c_int, c_int]),
            "orc_rope": (None, [POINTER(c_float), c_int, c_int, c_int, POINTER(c_float), POINTER(c_float),
                                POINTER(c_int32)]),
            "orc_argmax": (None, [POINTER(c_int32), POINTER(c_float), c_int, c_int]),
            "orc_silu": (None, [POINTER(c_float), ctypes.c_long]),
            "orc_exp64": (ctypes.c_double, [ctypes.c_double]),
            "orc_gate_sigmoid": (c_float, [c_float]),
            "orc_sigmoid_gate": (None, [POINTER(c_float), POINTER(c_float), ctypes.c_long]),
            "orc_rms_unit": (None, [POINTER(c_float), POINTER(c_float), c_int, c_int]),
            "orc_sinkhorn": (None, [POINTER(c_float), c_int, c_int]),
            "orc_mhc_heads": (None, [POINTER(c_float)] * 8 + [c_int, c_int, c_int, c_void_p]),
            "orc_mhc_mix": (None, [POINTER(c_float)] * 6 + [c_int, c_int, c_int]),
            "orc_attend_int8_spans": (c_int, [POINTER(c_float), POINTER(c_float), c_int, c_int, POINTER(c_int8),
                                              POINTER(c_float), c_int, c_int, POINTER(c_int8), POINTER(c_float), c_int,
                                              c_int, c_int, POINTER(c_int32), c_float, c_int, c_int, POINTER(c_float)]),
        }
        dm, dmem = POINTER(DecModel), POINTER(DecMemory)
        sig.update({
            "orc_dec_new": (c_void_p, [dm, dmem]),
            "orc_dec_fork": (c_void_p, [c_void_p]),
            "orc_dec_free": (None, [c_void_p]),
            "orc_dec_len": (c_int, [c_void_p]),
            "orc_dec_step": (c_int, [c_void_p, c_int, POINTER(c_float)]),
            "orc_dec_greedy": (c_int, [c_void_p, c_int, c_int, c_int, POINTER(c_int32), POINTER(c_float),
                                       POINTER(c_int)]),
            "orc_dec_streams": (c_int, [dm, dmem, c_int, POINTER(c_int32), c_int, c_int, POINTER(c_int32),
                                        POINTER(c_int32)]),
        })
        for name, (res, args) in sig.items():
            f = getattr(lb, name)
            f.restype = res
            f.argtypes = args
        _lib = lb
    return _lib


def fp(a):
    return a.ctypes.data_as(POINTER(c_float))


def u8p(a):
    return a.ctypes.data_as(POINTER(c_uint8))


def i8p(a):
    return a.ctypes.data_as(POINTER(c_int8))


def i32p(a):
    return a.ctypes.data_as(POINTER(c_int32))


def _packed(p):
    cb = np.ascontiguousarray(p.Codebook, dtype=np.float32)
    idx = np.ascontiguousarray(p.Index, dtype=np.uint8)
    nrm = np.ascontiguousarray(p.Norms, dtype=np.uint8)
    s = _Packed(p.Out, p.In, p.Group, p.Bits, p.Width, fp(cb), u8p(idx), u8p(nrm), idx.size, nrm.size, cb.size)
    return s, (cb, idx, nrm)


class OracleError(Exception):
    pass


class OMatrix:
    """The oracle's cq.Matrix (New) and Rows views."""

    def __init__(self, h, keep):
        self.h = c_void_p(h)
        self._keep = keep

    @staticmethod
    def new(p):
        s, keep = _packed(p)
        err = ctypes.create_string_buffer(256)
        h = lib().orc_new(ctypes.byref(s), err, 256)
        if not h:
            raise OracleError(err.value.decode())
        return OMatrix(h, keep)

    def __del__(self):
        if getattr(self, "h", None) is not None and self.h.value:
            lib().orc_free(self.h)
            self.h = None

    def rows(self, lo, hi):
        h = lib().orc_rows(self.h, lo, hi)
        if not h:
            raise OracleError(f"cq: Rows({lo}, {hi})")
        return OMatrix(h, self)

    def out(self):
        return lib().orc_out(self.h)

    def inp(self):
        return lib().orc_in(self.h)

    def gemm(self, x, rows, kernel=LUT):
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros(rows * self.out(), dtype=np.float32)
        rc = lib().orc_gemm(self.h, kernel, fp(y), fp(x), rows)
        if rc:
            raise OracleError(f"orc_gemm: {rc}")
        return y

    def row(self, r):
        y = np.zeros(self.inp(), dtype=np.float32)
        if lib().orc_row(self.h, fp(y), r):
            raise OracleError(f"Row({r})")
        return y


def gemms(ms, x, rows, kernel=LUT):
    x = np.ascontiguousarray(x, dtype=np.float32)
    ys = [np.zeros(rows * m.out(), dtype=np.float32) for m in ms]
    hs = (c_void_p * len(ms))(*[m.h for m in ms])
    ds = (POINTER(c_float) * len(ms))(*[fp(y) for y in ys])
    rc = lib().orc_gemms(hs, len(ms), kernel, ds, fp(x), rows)
    if rc:
        raise OracleError(f"orc_gemms: {rc}")
    return ys


def dequant(p):
    s, keep = _packed(p)
    w = np.zeros(p.Out * p.In, dtype=np.float32)
    if lib().orc_cq_dequant(fp(w), ctypes.byref(s)):
        raise OracleError("dequant")
    return w.reshape(p.Out, p.In)


def fwht(x, avx2=False):
    x = np.array(x, dtype=np.float32)
    (lib().orc_fwht_avx2 if avx2 else lib().orc_fwht)(fp(x), x.size)
    return x


def have_avx2():
    return bool(lib().orc_have_avx2())


def set_cpu(avx2=False, threads=1):
    """How lut products run from here on: the generic routines or their AVX2
    forms (the reference's amd64 path), on one thread or split over threads
    as gemmLUT splits them. Process-wide."""
    if lib().orc_set_cpu(int(avx2), int(threads)):
        raise OracleError("this CPU has no AVX2")


def lut_tables(x, cb, cb_max, width, avx2=False):
    """lutTables2/4 (generic or AVX2) of one rotated group x: (tables, M)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    cb = np.ascontiguousarray(cb, dtype=np.float32)
    n_tab = x.size // 2 if width == 2 else x.size
    tab = np.zeros(32 * n_tab, dtype=np.uint8)
    name = f"orc_lut_tables{width}" + ("_avx2" if avx2 else "")
    m = getattr(lib(), name)(u8p(tab), fp(x), x.size, fp(cb), c_float(cb_max))
    return tab, np.float32(m)


def lut_lookup(idx, tab, norm, steps, blocks, groups, gb, avx2=False):
    """lutLookup (generic or AVX2) of 32-row blocks: y [blocks * 32]."""
    y = np.zeros(blocks * 32, dtype=np.float32)
    idx = np.ascontiguousarray(idx, dtype=np.uint8)
    tab = np.ascontiguousarray(tab, dtype=np.uint8)
    norm = np.ascontiguousarray(norm, dtype=np.float32)
    steps = np.ascontiguousarray(steps, dtype=np.float32)
    f = lib().orc_lut_lookup_avx2 if avx2 else lib().orc_lut_lookup
    f(fp(y), u8p(idx), u8p(tab), fp(norm), fp(steps), blocks, groups, gb)
    return y


def quantize_row(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.zeros(x.size, dtype=np.int8)
    s = lib().orc_quantize_row(i8p(q), fp(x), x.size)
    return q, np.float32(s)


def quantize_rows(x, cols, width):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows = x.size // cols
    q = np.zeros(x.size, dtype=np.int8)
    s = np.zeros(rows * (cols // width), dtype=np.float32)
    lib().orc_quantize_rows(i8p(q), fp(s), fp(x), rows, cols, width)
    return q, s


def fake_quant(x, cols, width):
    """fakeQuant (int8.go:62-75) of rows of cols values in chunks of width."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    dst = np.zeros_like(x)
    lib().orc_fake_quant(fp(dst), fp(x), x.size // cols, cols, width)
    return dst


def exp_sub_sum(s, m, variant):
    s = np.array(s, dtype=np.float32)
    total = lib().orc_exp_sub_sum(fp(s), s.size, np.float32(m), variant)
    return s, np.float32(total)


def dots_i8(q, k, n, stride, avx2=False):
    """dotsI8 (int8kernel.go:346-357, or its AVX2 form): n int32 dots of q
    with the rows of k, stride bytes apart."""
    q = np.ascontiguousarray(q, dtype=np.int8)
    k = np.ascontiguousarray(k, dtype=np.int8)
    dst = np.zeros(n, dtype=np.int32)
    (lib().orc_dots_i8_avx2 if avx2 else lib().orc_dots_i8)(i32p(dst), n, i8p(q), q.size, i8p(k), stride)
    return dst


def axpys_i8(out, w, v, stride, avx2=False):
    """axpysI8 (int8kernel.go:360-368, or its AVX2 form): out += w[j] * v row j."""
    out = np.array(out, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.int8)
    (lib().orc_axpys_i8_avx2 if avx2 else lib().orc_axpys_i8)(fp(out), out.size, fp(w), w.size, i8p(v), stride)
    return out


def exp_sub_sum_avx2(s, m):
    """expSubSumAVX2 on a multiple-of-8 length (exp_amd64.s:68-124)."""
    s = np.array(s, dtype=np.float32)
    total = lib().orc_exp_sub_sum_avx2(fp(s), s.size, np.float32(m))
    return s, np.float32(total)


def softmax(s, variant):
    s = np.array(s, dtype=np.float32)
    lib().orc_softmax(fp(s), s.size, variant)
    return s


def attend_int8_spans(q, t, heads, kq, ks, k_cols, qk, vq, vs, v_cols, vd, nk, spans, scale, quant_q, variant=1,
                      want_probs=False):
    q = np.ascontiguousarray(q, dtype=np.float32)
    kq = np.ascontiguousarray(kq, dtype=np.int8)
    vq = np.ascontiguousarray(vq, dtype=np.int8)
    ks = np.ascontiguousarray(ks, dtype=np.float32)
    vs = np.ascontiguousarray(vs, dtype=np.float32)
    spans = np.ascontiguousarray(spans, dtype=np.int32)
    out = np.zeros(t * heads * vd, dtype=np.float32)
    probs = np.zeros(t * heads * nk, dtype=np.float32) if want_probs else None
    rc = lib().orc_attend_int8_spans(fp(out), fp(q), t, heads, i8p(kq), fp(ks), k_cols, qk, i8p(vq), fp(vs), v_cols,
                                     vd, nk, i32p(spans), np.float32(scale), 1 if quant_q else 0, variant,
                                     fp(probs) if probs is not None else None)
    if rc:
        raise OracleError(f"attend: {rc}")
    return (out, probs) if want_probs else out


def zc_rmsnorm(x, gain, dim):
    x = np.ascontiguousarray(x, dtype=np.float32)
    gain = np.ascontiguousarray(gain, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_zc_rmsnorm(fp(out), fp(x), fp(gain), x.size // dim, dim)
    return out


def rope(x, heads, head_dim, cos_t, sin_t, pos):
    x = np.array(x, dtype=np.float32)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    lib().orc_rope(fp(x), pos.size, heads, head_dim, fp(np.ascontiguousarray(cos_t, np.float32)),
                   fp(np.ascontiguousarray(sin_t, np.float32)), i32p(pos))
    return x


def argmax(v, rows, n):
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.zeros(rows, np.int32)
    lib().orc_argmax(i32p(out), fp(v), rows, n)
    return out


def silu(x):
    x = np.array(x, dtype=np.float32)
    lib().orc_silu(fp(x), x.size)
    return x


def exp64(x):
    """fdlibm's float64 exp of each value of x."""
    x = np.asarray(x, np.float64).ravel()
    return np.array([lib().orc_exp64(float(v)) for v in x], np.float64)


def gate_sigmoid(x):
    """float32(1 / (1 + exp(-float64(x)))) of each value of x."""
    x = np.asarray(x, np.float32).ravel()
    return np.array([lib().orc_gate_sigmoid(float(v)) for v in x], np.float32)


def sigmoid_gate(out, gate):
    """Attention.output's gate: returns (out * sigmoid(gate), sigmoid(gate))."""
    out = np.array(out, dtype=np.float32)
    gate = np.array(gate, dtype=np.float32)
    assert out.size == gate.size
    lib().orc_sigmoid_gate(fp(out), fp(gate), out.size)
    return out, gate


def rms_unit(x, rows, dim):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(rows * dim, np.float32)
    lib().orc_rms_unit(fp(out), fp(x), rows, dim)
    return out


def sinkhorn(k, n, iters=20):
    k = np.array(k, dtype=np.float32)
    lib().orc_sinkhorn(fp(k), n, iters)
    return k


def mhc_heads(pre_l, post_l, res_l, stream, rows, n, dim, affine=None):
    """(h_pre, h_post, h_res, u) of MHC.forward from the φ logits."""
    c = lambda a: np.ascontiguousarray(a, np.float32)
    pre_l, post_l, res_l, stream = c(pre_l), c(post_l), c(res_l), c(stream)
    hp, hq = np.zeros(rows * n, np.float32), np.zeros(rows * n, np.float32)
    hr, u = np.zeros(rows * n * n, np.float32), np.zeros(rows * dim, np.float32)
    aff = c(affine) if affine is not None else None
    lib().orc_mhc_heads(fp(hp), fp(hq), fp(hr), fp(u), fp(pre_l), fp(post_l), fp(res_l), fp(stream), rows, n, dim,
                        aff.ctypes.data if aff is not None else None)
    return hp, hq, hr, u


def mhc_mix(stream, h_res, h_post, block_out, u, rows, n, dim):
    c = lambda a: np.ascontiguousarray(a, np.float32)
    out = np.zeros(rows * n * dim, np.float32)
    lib().orc_mhc_mix(fp(out), fp(c(stream)), fp(c(h_res)), fp(c(h_post)), fp(c(block_out)), fp(c(u)), rows, n, dim)
    return out
