"""The synthetic decoder's greedy decode restated on the CPU oracle, one
stream at a time: the same operations in the same order as
go-whistle_amd/decoder.py's device step (embedding Row x sqrt(d),
ZCRMSNorm, lut GEMMs, RoPE, int8 append and AttendInt8 with the int8 query
and amd64's exponent, the sigmoid output gates, SiLU, tied head,
first-index argmax), over a cross
memory projected from the encoder states and quantised per head.

TEST INFRASTRUCTURE ONLY: the checker for the device decoder and the
cpu_baseline of bench.py's decode leg.
"""

import math

import numpy as np

from . import binding as orc


class RefDecoder:
    def __init__(self, model):
        self.model, self.cfg = model, model.cfg
        self.emb = orc.OMatrix.new(model.emb)
        self.mats = [{n: orc.OMatrix.new(p[n]) for n in p} for p in model.layers]

    def memory(self, enc):
        """The stream's int8 cross memory from its encoder states enc, float32
        [frames*dim] (cross.project, cross.go:181-204): per layer K, V =
        GEMMs(Wck, Wcv) over the frames (needle.ApplyShared), QuantizeRows
        per head."""
        c = self.cfg
        self.mem = []
        for w in self.mats:
            k, v = orc.gemms([w["wck"], w["wcv"]], enc, c.frames)
            kq, ks = orc.quantize_rows(k, c.dim, c.head_dim)
            vq, vs = orc.quantize_rows(v, c.dim, c.head_dim)
            self.mem.append((kq, ks, vq, vs))

    def decode(self, first, n, want_logits=False, eos=None):
        """Greedy tokens after first, at most n (MaxTokens); with eos, the
        loop stops at EOS, which it leaves out, and self.stopped says so
        (GreedyMemory, greedy.go:50-66)."""
        c, m = self.cfg, self.model
        self.stopped = False
        hk = c.dim // c.head_dim
        scale = np.float32(math.sqrt(c.head_dim))
        caches = [[np.zeros(c.max_pos * c.dim, np.int8), np.zeros(c.max_pos * hk, np.float32),
                   np.zeros(c.max_pos * c.dim, np.int8), np.zeros(c.max_pos * hk, np.float32)]
                  for _ in range(c.layers)]
        tok, out, logits_all = int(first), [], []
        for pos in range(n):
            x = (self.emb.row(tok) * m.scale).astype(np.float32)
            for l in range(c.layers):
                w = self.mats[l]
                h = orc.zc_rmsnorm(x, m.gains[3 * l], c.dim)
                q, k, v, g = orc.gemms([w["wq"], w["wk"], w["wv"], w["wg"]], h, 1)
                q = orc.rope(q, c.heads, c.head_dim, m.rope_cos, m.rope_sin, [pos])
                k = orc.rope(k, c.heads, c.head_dim, m.rope_cos, m.rope_sin, [pos])
                kc, ksc, vc, vsc = caches[l]
                kq, ks = orc.quantize_rows(k, c.dim, c.head_dim)
                vq, vs = orc.quantize_rows(v, c.dim, c.head_dim)
                kc[pos * c.dim:(pos + 1) * c.dim], ksc[pos * hk:(pos + 1) * hk] = kq, ks
                vc[pos * c.dim:(pos + 1) * c.dim], vsc[pos * hk:(pos + 1) * hk] = vq, vs
                n_keys = pos + 1
                a = orc.attend_int8_spans(q, 1, c.heads, kc[:n_keys * c.dim], ksc[:n_keys * hk], c.dim, c.head_dim,
                                          vc[:n_keys * c.dim], vsc[:n_keys * hk], c.dim, c.head_dim, n_keys,
                                          np.array([[0, 0, 0, n_keys]], np.int32), scale, True, 1)
                a, _ = orc.sigmoid_gate(a, g)  # Attention.output (attention.go:242-260)
                x = (x + w["wo"].gemm(a, 1)).astype(np.float32)
                h = orc.zc_rmsnorm(x, m.gains[3 * l + 1], c.dim)
                qc, gc = orc.gemms([w["wcq"], w["wcg"]], h, 1)
                mk, mks, mv, mvs = self.mem[l]
                a = orc.attend_int8_spans(qc, 1, c.heads, mk, mks, c.dim, c.head_dim, mv, mvs, c.dim, c.head_dim,
                                          c.frames, np.array([[0, 0, 0, c.frames]], np.int32), scale, True, 1)
                a, _ = orc.sigmoid_gate(a, gc)  # cross.go:231-252
                x = (x + w["wco"].gemm(a, 1)).astype(np.float32)
                h = orc.zc_rmsnorm(x, m.gains[3 * l + 2], c.dim)
                u = orc.silu(w["w1"].gemm(h, 1))
                x = (x + w["w2"].gemm(u, 1)).astype(np.float32)
            h = orc.zc_rmsnorm(x, m.gains[3 * c.layers], c.dim)
            logits = self.emb.gemm(h, 1)
            tok = int(orc.argmax(logits, 1, c.vocab)[0])
            if eos is not None and tok == eos:
                self.stopped = True
                break
            out.append(tok)
            if want_logits:
                logits_all.append(logits)
        return (out, logits_all) if want_logits else out
