"""The synthetic decoder's greedy decode on the CPU oracle.

RefDecoder holds the model as the C restatement's orc_dec_model
(decode_oracle.c): every token's step, and the greedy loop, run in C
(embedding Row x scale, the layers with ZCRMSNorm, lut GEMMs, the taps,
the q/k norms, RoPE, int8 append and AttendInt8 with the int8 query and
amd64's exponent, the sigmoid output gates, the post norms and residual
factors, the cross-attention over the stream's memory, SiLU FFN, the mHC
lanes; the tied head and first-index argmax), the same operations in the
same order as go-whistle_amd/decoder.py's device step. The cross memory
is built here from the encoder states with the oracle's GEMMs and
QuantizeRows (cross.project, cross.go:181-204).

compose_step restates one step in Python from the oracle's single
operations, a second, independently written form of the same layer that
tests hold the C loop to.

TEST INFRASTRUCTURE ONLY: the checker for the device decoder and the
cpu_baseline of bench.py's decode leg.
"""

import ctypes
import math
from ctypes import POINTER, c_float, c_int, c_int32, c_void_p

import numpy as np

from . import binding as orc

MAT_ORDER = ("wq", "wk", "wv", "wg", "wo", "wcq", "wcg", "wco", "wck", "wcv", "w1", "w2", "phi_pre", "phi_post",
             "phi_res")


def _f(a):
    a = np.ascontiguousarray(a, np.float32)
    return a, a.ctypes.data_as(POINTER(c_float))


class RefDecoder:
    def __init__(self, model):
        self.model, self.cfg = model, model.cfg
        c = self.cfg
        self.emb = orc.OMatrix.new(model.emb)
        self.mats = [{n: orc.OMatrix.new(p[n]) for n in p} for p in model.layers]
        mats = (c_void_p * (c.layers * len(MAT_ORDER)))()
        for l, w in enumerate(self.mats):
            for i, n in enumerate(MAT_ORDER):
                if n in w:
                    mats[l * len(MAT_ORDER) + i] = w[n].h.value
        self._keep = [mats]
        arrs = {}
        for name, a in (("gains", model.gains), ("rope_cos", model.rope_cos), ("rope_sin", model.rope_sin),
                        ("qk_gains", model.qk_gains), ("post_gains", model.post_gains),
                        ("res_scale", model.res_scale), ("taps_w", model.taps_w),
                        ("mhc_affine", model.mhc_affine)):
            a, p = _f(a)
            self._keep.append(a)
            arrs[name] = p
        self._m = orc.DecModel(c.vocab, c.dim, c.heads, c.head_dim, c.ffn, c.layers, c.frames, c.max_pos, c.taps,
                               int(c.qk_norm), int(c.post_norm), int(c.cross_norm), c.lanes, float(model.scale),
                               self.emb.h.value, mats, **arrs)
        self.mem = None

    def memory(self, enc):
        """The stream's int8 cross memory from its encoder states enc, float32
        [frames*dim] (cross.project, cross.go:181-204): per layer K, V =
        GEMMs(Wck, Wcv) over the frames (needle.ApplyShared), the per-head k
        norm with cross_norm, QuantizeRows per head."""
        self.mem = self.build_memory(enc)

    def build_memory(self, enc):
        c, m = self.cfg, self.model
        layers = []
        for l, w in enumerate(self.mats):
            k, v = orc.gemms([w["wck"], w["wcv"]], enc, c.frames)
            if c.cross_norm:
                k = orc.zc_rmsnorm(k, m.qk_gains[l, 3], c.head_dim)
            kq, ks = orc.quantize_rows(k, c.dim, c.head_dim)
            vq, vs = orc.quantize_rows(v, c.dim, c.head_dim)
            layers.append((kq, ks, vq, vs))
        return _Memory(layers)

    def state(self, mem=None):
        mem = mem or self.mem
        return RefState(self, mem, orc.lib().orc_dec_new(ctypes.byref(self._m), ctypes.byref(mem.s)))

    def decode(self, first, n, want_logits=False, eos=None):
        """Greedy tokens after first, at most n (MaxTokens); with eos, the
        loop stops at EOS, which it leaves out, and self.stopped says so
        (GreedyMemory, greedy.go:50-66)."""
        st = self.state()
        toks, logits, self.stopped = st.greedy(first, n, want_logits, eos)
        return (toks, logits) if want_logits else toks

    def decode_streams(self, mems, firsts, n, threads):
        """len(mems) streams decoded from fresh states, n tokens each, on
        `threads` threads (one stream per thread at a time); [streams, n]."""
        s = len(mems)
        arr = (orc.DecMemory * s)(*[m.s for m in mems])
        first = np.ascontiguousarray(firsts, np.int32)
        toks = np.zeros((s, n), np.int32)
        counts = np.zeros(s, np.int32)
        orc.lib().orc_dec_streams(ctypes.byref(self._m), arr, s, orc.i32p(first), n, threads, orc.i32p(toks),
                                  orc.i32p(counts))
        return toks, counts


class _Memory:
    def __init__(self, layers):
        self.layers = layers
        L = len(layers)
        ptr = lambda a: a.ctypes.data
        self._arrs = [(c_void_p * L)(*[ptr(t[i]) for t in layers]) for i in range(4)]
        self.s = orc.DecMemory(*self._arrs)


class RefState:
    """One stream's state (NewState / State.Fork, decoder.go:212-240)."""

    def __init__(self, dec, mem, h):
        self.dec, self.mem, self.h = dec, mem, c_void_p(h)

    def __del__(self):
        if getattr(self, "h", None) is not None and self.h.value:
            orc.lib().orc_dec_free(self.h)
            self.h = None

    def fork(self):
        return RefState(self.dec, self.mem, orc.lib().orc_dec_fork(self.h))

    def __len__(self):
        return orc.lib().orc_dec_len(self.h)

    def step(self, token):
        """Decoder.Extend of one token: (argmax, logits)."""
        lg = np.zeros(self.dec.cfg.vocab, np.float32)
        tok = orc.lib().orc_dec_step(self.h, int(token), orc.fp(lg))
        if tok < 0:
            raise orc.OracleError(f"decoder step of token {token} at {len(self)}")
        return tok, lg

    def greedy(self, first, n, want_logits=False, eos=None):
        c = self.dec.cfg
        toks = np.zeros(max(n, 1), np.int32)
        lg = np.zeros((max(n, 1), c.vocab), np.float32) if want_logits else None
        stopped = c_int(0)
        got = orc.lib().orc_dec_greedy(self.h, int(first), n, -1 if eos is None else int(eos), orc.i32p(toks),
                                       orc.fp(lg) if lg is not None else None, ctypes.byref(stopped))
        if got < 0:
            raise orc.OracleError("decoder greedy loop")
        logits = list(lg[:got]) if want_logits else None
        return [int(t) for t in toks[:got]], logits, bool(stopped.value)


def compose_step(ref, mem, hist, caches, tok, pos):
    """One token's step composed in Python from the oracle's single
    operations (the layer of decoder.go:446-505 with block.go:147-215, the
    cross branch cross.go:209-264, the taps of cache.go:143-154, the mHC of
    mhc.go:182-299): (logits, argmax). hist[l] holds, per q/k/v, the raw
    rows of the last taps - 1 positions (oldest first) and caches[l] the
    self K/V codes and scales; both are updated."""
    c, m = ref.cfg, ref.model
    D, H, hd = c.dim, c.heads, c.head_dim
    hk = D // hd
    scale = np.float32(math.sqrt(hd))
    sp = np.array([[0, 0, 0, pos + 1]], np.int32)

    def block(l, h):
        w = ref.mats[l]
        n = orc.zc_rmsnorm(h, m.gains[3 * l], D)
        q, k, v, g = orc.gemms([w["wq"], w["wk"], w["wv"], w["wg"]], n, 1)
        if c.taps:
            out = []
            for z, raw in enumerate((q, k, v)):
                rows = hist[l][z] + [raw]
                i = len(rows) - 1
                acc = np.zeros(D, np.float32)
                for j in range(c.taps):
                    if i - j < 0:
                        break
                    acc = (acc + (m.taps_w[l, z, j] * rows[i - j]).astype(np.float32)).astype(np.float32)
                hist[l][z] = rows[-(c.taps - 1):] if c.taps > 1 else []
                out.append(acc)
            q, k, v = out
        if c.qk_norm:
            q = orc.zc_rmsnorm(q, m.qk_gains[l, 0], hd)
            k = orc.zc_rmsnorm(k, m.qk_gains[l, 1], hd)
        q = orc.rope(q, H, hd, m.rope_cos, m.rope_sin, [pos])
        k = orc.rope(k, hk, hd, m.rope_cos, m.rope_sin, [pos])
        kc, ksc, vc, vsc = caches[l]
        kc[pos * D:(pos + 1) * D], ksc[pos * hk:(pos + 1) * hk] = orc.quantize_rows(k, D, hd)
        vc[pos * D:(pos + 1) * D], vsc[pos * hk:(pos + 1) * hk] = orc.quantize_rows(v, D, hd)
        nk = pos + 1
        a = orc.attend_int8_spans(q, 1, H, kc[:nk * D], ksc[:nk * hk], D, hd, vc[:nk * D], vsc[:nk * hk], D, hd, nk,
                                  sp, scale, True, 1)
        a, _ = orc.sigmoid_gate(a, g)
        o = w["wo"].gemm(a, 1)
        if c.post_norm:
            o = orc.zc_rmsnorm(o, m.post_gains[l, 0], D)
            h = (h + (m.res_scale[l, 0] * o).astype(np.float32)).astype(np.float32)
        else:
            h = (h + o).astype(np.float32)
        n = orc.zc_rmsnorm(h, m.gains[3 * l + 1], D)
        qc, gc = orc.gemms([w["wcq"], w["wcg"]], n, 1)
        if c.cross_norm:
            qc = orc.zc_rmsnorm(qc, m.qk_gains[l, 2], hd)
        mk, mks, mv, mvs = mem.layers[l]
        a = orc.attend_int8_spans(qc, 1, H, mk, mks, D, hd, mv, mvs, D, hd, c.frames,
                                  np.array([[0, 0, 0, c.frames]], np.int32), scale, True, 1)
        a, _ = orc.sigmoid_gate(a, gc)
        y = w["wco"].gemm(a, 1)
        if c.cross_norm:
            y = orc.zc_rmsnorm(y, m.post_gains[l, 1], D)
            y = (m.res_scale[l, 1] * y).astype(np.float32)
        h = (h + y).astype(np.float32)
        n = orc.zc_rmsnorm(h, m.gains[3 * l + 2], D)
        u = orc.silu(w["w1"].gemm(n, 1))
        return (w["w2"].gemm(u, 1) + h).astype(np.float32)

    x = (ref.emb.row(tok) * m.scale).astype(np.float32)
    if c.lanes:
        nl = c.lanes
        stream = np.tile(x, nl).astype(np.float32)
        for l in range(c.layers):
            w = ref.mats[l]
            nx = orc.rms_unit(stream, 1, nl * D)
            nxq = orc.fake_quant(nx, nl * D, nl * D)
            pl, ql, rl = orc.gemms([w["phi_pre"], w["phi_post"], w["phi_res"]], nxq, 1)
            hp, hq, hr, u = orc.mhc_heads(pl, ql, rl, stream, 1, nl, D, m.mhc_affine[l])
            out = block(l, u)
            stream = orc.mhc_mix(stream, hr, hq, out, u, 1, nl, D)
        acc = np.zeros(D, np.float32)
        for k in range(nl):
            acc = (acc + stream[k * D:(k + 1) * D]).astype(np.float32)
        x = (acc / np.float32(nl)).astype(np.float32)
    else:
        for l in range(c.layers):
            x = block(l, x)
    h = orc.zc_rmsnorm(x, m.gains[3 * c.layers], D)
    logits = ref.emb.gemm(h, 1)
    return logits, int(orc.argmax(logits, 1, c.vocab)[0])
