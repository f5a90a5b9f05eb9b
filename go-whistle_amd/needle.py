"""go-whistle's int8 KV numerics (internal/needle/int8.go) and its packed
Linear (internal/needle/linear.go) over libcqhip.

QuantizeRows / Int8Rows.Append (int8.go:116-141) on host arrays or device
tensors, AttendInt8Spans (int8.go:208-272) on device tensors for one or
many independent streams, fakeQuant (int8.go:57-75), and Linear with
WithInt8Input, Apply and ApplyShared on device tensors.
"""

import ctypes
from ctypes import POINTER, c_float, c_int8, c_void_p

import numpy as np

from ._lib import CQPanic, check, lib


def QuantizeRows(x, cols, width):
    """Codes and scales of x, rows of cols values, per chunk of width (host)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if width <= 0 or cols % width != 0:
        raise CQPanic(f"needle: int8 rows of {cols} in chunks of {width}")
    if x.size % cols != 0:
        raise CQPanic(f"needle: {x.size} values are not rows of {cols}")
    rows = x.size // cols
    q = np.zeros(x.size, dtype=np.int8)
    s = np.zeros(rows * (cols // width), dtype=np.float32)
    check(lib().kv_quantize_rows(q.ctypes.data_as(POINTER(c_int8)), s.ctypes.data_as(POINTER(c_float)),
                                 x.ctypes.data_as(POINTER(c_float)), rows, cols, width))
    return q, s


def QuantizeRow(x):
    """QuantizeRow (int8.go:36-55): codes and the scale of one chunk."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    q, s = QuantizeRows(x, x.size, x.size) if x.size else (np.zeros(0, np.int8), np.ones(1, np.float32))
    return q, float(s[0])


def _stream():
    import torch

    return c_void_p(torch.cuda.current_stream().cuda_stream)


def quantize_rows_dev(q, s, x, rows, cols, width):
    """Device form: q int8 [rows*cols], s float32 [rows*cols/width], x float32."""
    check(lib().kv_quantize_rows_dev(c_void_p(q.data_ptr()), c_void_p(s.data_ptr()), c_void_p(x.data_ptr()),
                                     rows, cols, width, _stream()))


def attend_int8_dev(out, q, t, heads, kq, ks, k_cols, qk, vq, vs, v_cols, vd, spans, nk_max, scale, quant_q,
                    batch=1, out_stride=0, q_stride=0, kv_stride=0, s_stride=0, rope=None):
    """AttendInt8Spans on device tensors for `batch` streams (see cqhip.h).
    rope = (cos, sin, qpos): the query heads are first rotated by RoPE at
    row qpos[b*t + i] of the tables."""
    args = [c_void_p(out.data_ptr()), out_stride, c_void_p(q.data_ptr()), q_stride, t, heads,
            c_void_p(kq.data_ptr()), c_void_p(ks.data_ptr()), k_cols, qk, c_void_p(vq.data_ptr()),
            c_void_p(vs.data_ptr()), v_cols, vd, kv_stride, s_stride, c_void_p(spans.data_ptr()), nk_max, float(scale),
            1 if quant_q else 0, batch]
    if rope is None:
        check(lib().kv_attend_int8_dev(*args, _stream()))
    else:
        cos, sin, qpos = rope
        check(lib().kv_attend_int8_rope_dev(*args, c_void_p(cos.data_ptr()), c_void_p(sin.data_ptr()),
                                            c_void_p(qpos.data_ptr()), _stream()))


def append_dev(q, s, x, batch, cols, width, q_stride, s_stride, pos, cap, rope=None):
    """Int8Rows.Append of one row per stream at pos[b] (see cqhip.h); rope =
    (cos, sin): each chunk is first rotated by RoPE at row pos[b]."""
    args = [c_void_p(q.data_ptr()), c_void_p(s.data_ptr()), c_void_p(x.data_ptr()), batch, cols, width, q_stride,
            s_stride, c_void_p(pos.data_ptr()), cap]
    if rope is None:
        check(lib().kv_append_dev(*args, _stream()))
    else:
        cos, sin = rope
        check(lib().kv_append_rope_dev(*args, c_void_p(cos.data_ptr()), c_void_p(sin.data_ptr()), _stream()))


def fake_quant_dev(dst, x, rows, cols, width):
    """fakeQuant (int8.go:57-75) on device tensors: rows of cols values, each
    chunk of width through QuantizeRow and back; dst may be x."""
    check(lib().nd_fake_quant_dev(c_void_p(dst.data_ptr()), c_void_p(x.data_ptr()), rows, cols, width, _stream()))


def sigmoid_gate_dev(out, gate, n):
    """Attention.output's gate (attention.go:245-249) on device tensors:
    gate = sigmoid(gate), out *= gate over n values."""
    check(lib().nd_sigmoid_gate_dev(c_void_p(out.data_ptr()), c_void_p(gate.data_ptr()), n, _stream()))


def rms_unit_dev(dst, x, rows, dim):
    """RMSUnit (norm.go:68-81) on device rows."""
    check(lib().nd_rms_unit_dev(c_void_p(dst.data_ptr()), c_void_p(x.data_ptr()), rows, dim, _stream()))


def mhc_heads_dev(h_pre, h_post, h_res, u, pre_logits, post_logits, res_logits, stream, rows, lanes, dim,
                  affine=None):
    """MHC.forward's heads and block input from the φ logits (mhc.go:204-263)."""
    p = lambda t: c_void_p(t.data_ptr()) if t is not None else None
    check(lib().nd_mhc_heads_dev(p(h_pre), p(h_post), p(h_res), p(u), p(pre_logits), p(post_logits), p(res_logits),
                                 p(stream), rows, lanes, dim, p(affine), _stream()))


def mhc_heads_stacked_dev(h_pre, h_post, h_res, u, logits, stream, rows, lanes, dim, affine=None):
    """mhc_heads_dev with the logits of each row side by side, rows x (2 lanes
    + lanes^2): pre, post, res (one product of the stacked φ matrices)."""
    p = lambda t: c_void_p(t.data_ptr()) if t is not None else None
    check(lib().nd_mhc_heads_stacked_dev(p(h_pre), p(h_post), p(h_res), p(u), p(logits), p(stream), rows, lanes, dim,
                                         p(affine), _stream()))


def mhc_mix_dev(out, stream, h_res, h_post, block_out, u, rows, lanes, dim):
    """MHC.forward's output stream (mhc.go:229-299)."""
    p = lambda t: c_void_p(t.data_ptr())
    check(lib().nd_mhc_mix_dev(p(out), p(stream), p(h_res), p(h_post), p(block_out), p(u), rows, lanes, dim,
                               _stream()))


class HadamardMLP:
    """HadamardMLP (internal/needle/hadamard.go:12-24, 172-310), Whistle's
    Monarch FFN, with its weights on the device: w holds d1, d2, b2, d3, d4,
    w1a..w3b (square factors), cond_v (dim x rank), cond_u (rank x n) and the
    permutations p1, p2 (hada_p1/p2). forward_dev(out, x, rows) runs
    nd_hadamard_mlp_dev on device tensors of rows x dim."""

    def __init__(self, w, device="cuda"):
        import torch

        f32 = lambda a: torch.as_tensor(np.ascontiguousarray(a, np.float32), device=device)
        self.na, self.nb = int(np.shape(w["w1a"])[0]), int(np.shape(w["w1b"])[0])
        self.dim, self.rank = int(np.shape(w["cond_v"])[0]), int(np.shape(w["cond_v"])[1])
        self._vecs = [f32(w[k]) for k in ("d1", "d2", "b2", "d3", "d4")]
        self._facs = [f32(w[f"w{s}{h}"]) for s in (1, 2, 3) for h in ("a", "b")]
        self._cv, self._cu = f32(w["cond_v"]), f32(w["cond_u"])
        self._p = [torch.as_tensor(np.ascontiguousarray(w[k], np.int32), device=device) for k in ("p1", "p2")]
        n = self.na * self.nb
        for k in ("p1", "p2"):
            if sorted(np.asarray(w[k]).tolist()) != list(range(n)):
                raise CQPanic(f"needle: {k} is not a permutation of {n}")

    def forward_dev(self, out, x, rows):
        vp = (c_void_p * 5)(*[t.data_ptr() for t in self._vecs])
        fp_ = (c_void_p * 6)(*[t.data_ptr() for t in self._facs])
        check(lib().nd_hadamard_mlp_dev(c_void_p(out.data_ptr()), c_void_p(x.data_ptr()), rows, self.dim, self.na,
                                        self.nb, self.rank, vp, fp_, c_void_p(self._cv.data_ptr()),
                                        c_void_p(self._cu.data_ptr()), c_void_p(self._p[0].data_ptr()),
                                        c_void_p(self._p[1].data_ptr()), _stream()))


class Linear:
    """needle.Linear over a packed matrix (internal/needle/linear.go:11-145),
    on device tensors: x rows × In -> dst rows × Out. With WithInt8Input the
    input rows are first quantised per row (quantInput, int8.go:81-88)."""

    def __init__(self, m, act8=False):
        self.q, self.act8 = m, bool(act8)
        self.In, self.Out = m.In(), m.Out()

    def WithInt8Input(self, on):
        return Linear(self.q, on)

    def Int8Input(self):
        return self.act8

    def _quant_input(self, x, rows):
        import torch

        xq = torch.empty(rows * self.In, dtype=torch.float32, device=x.device)
        fake_quant_dev(xq, x, rows, self.In, self.In)
        return xq

    def Apply(self, dst, x, rows):
        """linear.go:82-95."""
        from . import cq

        if self.act8:
            x = self._quant_input(x, rows)
        cq.gemms_dev([self.q], [dst], x, rows)


def ApplyShared(dsts, x, rows, *ls):
    """ApplyShared (linear.go:97-145): each dsts[k] = ls[k].Apply's result bit
    for bit; the linears that quantise their input share one quantised copy
    of x, and the packed ones of each kind run through one cq.GEMMs."""
    from . import cq

    if len(dsts) != len(ls):
        raise CQPanic(f"needle: ApplyShared of {len(ls)} linears into {len(dsts)} outputs")
    if not ls:
        return
    xq = next((l._quant_input(x, rows) for l in ls if l.act8), None)
    for quant in (False, True):
        sel = [k for k, l in enumerate(ls) if l.act8 == quant]
        if sel:
            cq.gemms_dev([ls[k].q for k in sel], [dsts[k] for k in sel], xq if quant else x, rows)
