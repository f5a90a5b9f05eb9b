"""A synthetic Whistle-shaped decoder on the device, for greedy decoding.

The configuration is the one the benchmark names: 8 layers, d_model 512,
8 heads of 64, FFN 2048, vocabulary 16384, cross-attention over 1500
frames, an int8 self- and cross-KV cache, CQ-packed linears (4-bit
attention, 2-bit FFN) and a 4-bit embedding tied to the head. Whistle's
real decoder (internal/decoder) has mHC, engram and a float Monarch MLP;
this one keeps the CQ, int8 and float pieces of its decode step that the
quantized path serves:

  x = E.Row(token) * scale                          decoder.go:269-275
  per layer:
    h = ZCRMSNorm(x); q, k, v, g = GEMMs(Wq, Wk, Wv, Wg; h)  norm.go, attention.go:265-271
    RoPE(q), RoPE(k) at the position                 rope.go:69-81
    append int8 k, v; a = AttendInt8(q, 0..pos)      int8.go:125-141, 208-272
    x += Wo (a * sigmoid(g))                         attention.go:242-260
    h = ZCRMSNorm(x); q, g = GEMMs(Wcq, Wcg; h)      cross.go:209-252
    a = AttendInt8(q, memory); x += Wco (a * sigmoid(g))
    h = ZCRMSNorm(x); x += W2 SiLU(W1 h)
  logits = E ZCRMSNorm(x); token = argmax           decoder.go:507-523, greedy.go:181-191

with the int8 query (Int8.Act) and amd64's softmax exponent. Every step is
bit for bit the same arithmetic as the C restatement in oracle/, so the
greedy tokens match exactly. The cross memory of each stream is built once
from its own 1500 x 512 encoder states drawn N(0, 1), as cross.project
does it (cross.go:181-204, without q/k norms or cross RoPE):

  per layer: K, V = GEMMs(Wck, Wcv; enc) over the frames  needle.ApplyShared
             int8 K, V = QuantizeRows per head             int8.go:116-141
             (stored head-major: [head][frame][64] per stream)

on the device (the batched products take the MFMA form); that build is
not part of the decode step.

All state lives on the device; step() queues one token's launches on
torch's current stream and can be captured in a HIP graph.
"""

from dataclasses import dataclass, field
import math

import numpy as np

from . import cq, needle, synth
from ._lib import check, lib


@dataclass
class DecoderConfig:
    vocab: int = 16384
    dim: int = 512
    heads: int = 8
    head_dim: int = 64
    ffn: int = 2048
    layers: int = 8
    frames: int = 1500
    max_pos: int = 256
    attn_bits: int = 4
    ffn_bits: int = 2
    group: int = 128
    theta: float = 1e5
    # The reference decode step's features (each off by default):
    taps: int = 0             # causal taps on the raw q/k/v (Whistle: 3; cache.go:143-154)
    qk_norm: bool = False     # per-head q/k ZCRMSNorm before RoPE (attention.go:298-330)
    post_norm: bool = False   # the attention's post norm, h += float32(gate * a) (block.go:183-188)
    cross_norm: bool = False  # cross q/k norms, post norm, residual factor (cross.go:181-264)
    lanes: int = 0            # mHC lanes around each layer (Whistle: 4; mhc.go:182-299)

    @staticmethod
    def whistle(**kw):
        """Every feature of Whistle's decode step on: 3 taps, the q/k norms,
        both post norms and residual factors, 4 mHC lanes."""
        return DecoderConfig(taps=3, qk_norm=True, post_norm=True, cross_norm=True, lanes=4, **kw)

    @property
    def features(self):
        return bool(self.taps or self.qk_norm or self.post_norm or self.cross_norm or self.lanes)


LAYER_MATS = ("wq", "wk", "wv", "wg", "wo", "wcq", "wcg", "wco", "wck", "wcv", "w1", "w2")
PHI_MATS = ("phi_pre", "phi_post", "phi_res")


@dataclass
class Model:
    cfg: DecoderConfig
    emb: cq.Packed
    layers: list  # per layer: dict name -> Packed
    gains: np.ndarray  # [layers*3 + 1, dim]: attn, cross, ffn per layer, then final
    rope_cos: np.ndarray
    rope_sin: np.ndarray
    scale: np.float32 = field(default=np.float32(0))
    # the decode step's features (present whatever the configuration enables)
    qk_gains: np.ndarray = None    # [layers, 4, head_dim]: self q, self k, cross q, cross k (ZCRMSNorm gains)
    post_gains: np.ndarray = None  # [layers, 2, dim]: the self and cross post norms
    res_scale: np.ndarray = None   # [layers, 2]: sigmoid(attn_gate), sigmoid(cross_gate) as loaded
    taps_w: np.ndarray = None      # [layers, 3, taps, dim]: q, k, v taps
    mhc_affine: np.ndarray = None  # [layers, 3 + 4 lanes + lanes^2]: a_pre, a_post, a_res, b_pre, pre_off,
    #                                b_post, post_off, b_res


def _share(p, cb):
    p.Codebook = cb
    return p


def stack_rows(ps):
    """The matrices ps (one input width, group and codebook) stacked row-wise
    into one: its product is theirs, row for row and bit for bit, with one
    table build per activation instead of one per matrix."""
    p0 = ps[0]
    for p in ps[1:]:
        if (p.In, p.Group, p.Bits, p.Width) != (p0.In, p0.Group, p0.Bits, p0.Width) or \
                not np.array_equal(np.asarray(p.Codebook), np.asarray(p0.Codebook)):
            raise ValueError("stacked matrices share their input width, group, width and codebook")
    return cq.Packed(Out=sum(p.Out for p in ps), In=p0.In, Group=p0.Group, Bits=p0.Bits, Width=p0.Width,
                     Codebook=p0.Codebook, Index=np.concatenate([np.asarray(p.Index, np.uint8) for p in ps]),
                     Norms=np.concatenate([np.asarray(p.Norms, np.uint8) for p in ps]))


def rope_tables(head_dim, n, theta):
    """NewRope (internal/needle/rope.go:17-44): float32 frequencies, float64
    cos/sin of float32 angles, rounded to float32."""
    half = head_dim // 2
    freqs = np.zeros(half, np.float32)
    for i in range(half):
        e = np.float32(2 * i) / np.float32(head_dim)
        freqs[i] = np.float32(1) / np.float32(math.pow(theta, float(e)))
    cos = np.zeros((n, half), np.float32)
    sin = np.zeros((n, half), np.float32)
    for t in range(n):
        ang = (np.float32(t) * freqs).astype(np.float64)
        cos[t] = np.cos(ang).astype(np.float32)
        sin[t] = np.sin(ang).astype(np.float32)
    return cos, sin


def make_model(seed, cfg=DecoderConfig()):
    """Seeded weights: one zero-mean codebook per index width (as a .cact file holds),
    uniform indices, FP16 norms 2^-3..2^1 (the embedding's 0.5..0.56, so
    that no row outscores the others for every input), gains 1 + N(0, 0.1)."""
    g = synth.rng(seed)

    def symmetric(n):  # N(0, 0.05) magnitudes mirrored: a zero-mean codebook, as Lloyd-Max levels are
        m = np.abs(g.standard_normal(n // 2) * 0.05).astype(np.float32)
        return np.sort(np.concatenate([-m, m])).astype(np.float32)

    cb4, cb2 = symmetric(16), symmetric(4)

    def packed(out, inp, bits, exps=(12, 16), mants=1024):
        p = synth.random_packed(g, out, inp, cfg.group, bits, sigma=0.05)
        groups = (inp + cfg.group - 1) // cfg.group
        exp = g.integers(exps[0], exps[1], size=out * groups).astype(np.uint16)
        man = g.integers(0, mants, size=out * groups).astype(np.uint16)
        p.Norms = ((exp << 10) | man).astype("<u2").view(np.uint8)
        return _share(p, cb4 if bits == 4 else cb2)

    d, f = cfg.dim, cfg.ffn
    emb = packed(cfg.vocab, d, cfg.attn_bits, exps=(14, 15), mants=128)  # rows of about equal norm
    layers = []
    for _ in range(cfg.layers):
        layers.append({"wq": packed(d, d, cfg.attn_bits), "wk": packed(d, d, cfg.attn_bits),
                       "wv": packed(d, d, cfg.attn_bits), "wo": packed(d, d, cfg.attn_bits),
                       "wcq": packed(d, d, cfg.attn_bits), "wco": packed(d, d, cfg.attn_bits),
                       "wck": packed(d, d, cfg.attn_bits), "wcv": packed(d, d, cfg.attn_bits),
                       "w1": packed(f, d, cfg.ffn_bits), "w2": packed(d, f, cfg.ffn_bits),
                       "wg": packed(d, d, cfg.attn_bits), "wcg": packed(d, d, cfg.attn_bits)})
    scales = (g.standard_normal((cfg.layers * 3 + 1, d)) * 0.1).astype(np.float32)
    gains = (np.float32(1) + scales).astype(np.float32)  # NewZCRMSNorm (norm.go:22-30)
    cos, sin = rope_tables(cfg.head_dim, cfg.max_pos, cfg.theta)
    # The unscaled input (Whistle's InputScale off, decoder.go:322-326): with
    # sqrt(d), a random tied embedding makes every token its own argmax.
    model = Model(cfg=cfg, emb=emb, layers=layers, gains=gains, rope_cos=cos, rope_sin=sin, scale=np.float32(1))
    _feature_weights(model, seed, cb4)
    return model


def lane_offsets(n, layer):
    """laneOffsets (internal/needle/mhc.go:122-135): the layer's own lane
    gets pre +4 and post 0, the others -4 and -4."""
    pre, post = np.full(n, -4, np.float32), np.full(n, -4, np.float32)
    pre[layer % n], post[layer % n] = 4, 0
    return pre, post


def _feature_weights(model, seed, cb4):
    """The weights of the decode step's features, from their own seeded
    stream (the base model's draws stay as they are): ZCRMSNorm gains 1 +
    N(0, 0.1), residual factors in (0.2, 0.8), taps 1 + N(0, 0.1) at the
    current position and N(0, 0.3) before it, and per layer the three mHC
    phi products (CQ4 of lanes x lanes*dim, lanes x lanes*dim, lanes^2 x
    lanes*dim on the attention codebook) with affine maps a = 0.5 + U(0, 0.5),
    b ~ N(0, 0.5) and the lane offsets."""
    cfg = model.cfg
    g = synth.rng(seed * 7919 + 17)
    L, D, hd = cfg.layers, cfg.dim, cfg.head_dim
    nt, n = max(cfg.taps, 1), max(cfg.lanes, 1)
    model.qk_gains = (1 + g.standard_normal((L, 4, hd)) * 0.1).astype(np.float32)
    model.post_gains = (1 + g.standard_normal((L, 2, D)) * 0.1).astype(np.float32)
    model.res_scale = g.uniform(0.2, 0.8, (L, 2)).astype(np.float32)
    tw = (g.standard_normal((L, 3, nt, D)) * 0.3).astype(np.float32)
    tw[:, :, 0] = (1 + g.standard_normal((L, 3, D)) * 0.1).astype(np.float32)
    model.taps_w = tw
    aff = np.zeros((L, 3 + 4 * n + n * n), np.float32)
    for l in range(L):
        pre, post = lane_offsets(n, l)
        aff[l, :3] = 0.5 + g.uniform(0, 0.5, 3)
        aff[l, 3:3 + n] = g.standard_normal(n) * 0.5
        aff[l, 3 + n:3 + 2 * n] = pre
        aff[l, 3 + 2 * n:3 + 3 * n] = g.standard_normal(n) * 0.5
        aff[l, 3 + 3 * n:3 + 4 * n] = post
        aff[l, 3 + 4 * n:] = g.standard_normal(n * n) * 0.5
    model.mhc_affine = aff
    if cfg.lanes:
        for l in range(L):
            for name, out in zip(PHI_MATS, (n, n, n * n)):
                p = synth.random_packed(g, out, n * D, cfg.group, 4, sigma=0.05)
                groups = (n * D + cfg.group - 1) // cfg.group
                exp = g.integers(12, 16, size=out * groups).astype(np.uint16)
                man = g.integers(0, 1024, size=out * groups).astype(np.uint16)
                p.Norms = ((exp << 10) | man).astype("<u2").view(np.uint8)
                model.layers[l][name] = _share(p, cb4)


def encoder_states(seed, cfg, stream):
    """One stream's encoder output, N(0, 1), [frames, dim]."""
    g = synth.rng(seed * 1000003 + stream)
    return g.standard_normal(cfg.frames * cfg.dim).astype(np.float32)


def fork_page_tables(pt, parents, pos, page_rows, pool_pages):
    """The page tables after stream b takes stream parents[b]'s state at
    position pos[b] (KVCache.Fork, internal/needle/cache.go:62-67: the rows
    so far are shared until one side appends). pt is [streams, pages per
    stream] of pool pages. Every stream starts from its parent's table; the
    pages from the one its next append writes on (pos // page_rows) onward
    must be its own, so each of them that another entry still references is
    replaced by a free pool page, and the partly filled one (pos not on a
    page boundary) is copied first. Returns (tables, [(from, to)] page
    copies). With one page row per stream's position there are at most
    len(parents) copies, whatever the positions; the pool needs no more
    pages than streams x pages per stream."""
    pt = np.asarray(pt, np.int32)[np.asarray(parents, np.int64)].copy()
    streams, per = pt.shape
    pos = np.asarray(pos, np.int64)
    lp0 = np.minimum(pos // page_rows, per)
    # References a stream must own from now on, in stream-then-page order.
    # Taken one at a time in that order, a page's reference is replaced
    # while another entry still references it: all of a page's must-own
    # references but the last, and that one too unless every reference to
    # the page is one of them. Free pages go out smallest first.
    must = np.arange(per)[None, :] >= lp0[:, None]
    total = np.bincount(pt.ravel(), minlength=pool_pages)
    b_idx, lp_idx = np.nonzero(must)
    mp = pt[b_idx, lp_idx].astype(np.int64)
    mcount = np.bincount(mp, minlength=pool_pages)
    order = np.argsort(mp, kind="stable")
    ranks = np.empty(mp.size, np.int64)
    ranks[order] = np.arange(mp.size) - np.searchsorted(mp[order], mp[order], side="left")
    repl = ~((total[mp] == mcount[mp]) & (ranks == mcount[mp] - 1))
    free = np.flatnonzero(total == 0)
    if repl.sum() > free.size:
        raise ValueError(f"decoder: a fork needs {int(repl.sum())} free pages, the pool has {free.size}")
    newp = mp.copy()
    newp[repl] = free[:int(repl.sum())]
    pt[b_idx, lp_idx] = newp
    partial = repl & (lp_idx == lp0[b_idx]) & (pos[b_idx] % page_rows != 0)
    copies = list(zip(mp[partial].tolist(), newp[partial].tolist()))
    return pt, copies


def _ptr(t):
    from ctypes import c_void_p

    return c_void_p(t.data_ptr())


class Decoder:
    """The model on the device for `batch` streams decoding in lockstep.
    fused: the norms, residual adds, output gates, SiLU, RoPE and the K/V
    appends ride in the products and the attention (8 launches per layer
    instead of 21, the same bits)."""

    PAGE_ROWS = 16  # rows per page of the paged self caches

    def __init__(self, model, batch, device="cuda", fused=True, paged=None):
        import torch

        self.model, self.cfg, self.batch, self.fused = model, model.cfg, batch, fused
        c, B = model.cfg, batch
        # The paged step: the decode-step features and self caches read
        # through per-stream page tables, so that a fork shares the rows so
        # far (the default whenever a feature is on).
        self.paged = c.features if paged is None else bool(paged)
        if self.paged and (c.head_dim != 64 or c.max_pos % self.PAGE_ROWS != 0):
            raise ValueError("the paged step runs heads of 64 and max_pos a multiple of 16")
        self.emb = cq.New(model.emb)
        self.mats = [{n: cq.New(p[n]) for n in p} for p in model.layers]
        if c.lanes:  # the three phi products as one: their logits side by side per activation
            for mm, p in zip(self.mats, model.layers):
                mm["phi"] = cq.New(stack_rows([p[n] for n in PHI_MATS]))
        f32, i8, i32 = torch.float32, torch.int8, torch.int32
        z = lambda *shape, dt=f32: torch.zeros(*shape, dtype=dt, device=device)
        self.gains = torch.from_numpy(model.gains).to(device)
        self.cos = torch.from_numpy(model.rope_cos).to(device)
        self.sin = torch.from_numpy(model.rope_sin).to(device)
        self.tok = z(B, dt=i32)
        self.pos = z(B, dt=i32)
        # Greedy's stop (greedy.go:50-66): with a stop token set, done[b]
        # becomes 1 at stream b's EOS and its token and position stay put.
        self.done = z(B, dt=i32)
        self.eos = None
        self.spans_self = z(B, 4, dt=i32)
        self.spans_self[:, 3] = 1  # keys 0..pos after the first step's append
        self.steps = 0  # steps run since reset (a stream that stopped at EOS is behind it)
        hk = c.dim // c.head_dim
        # The cross memory is head-major, [stream][head][frame][code]: every
        # (stream, head) a contiguous block, read as batch * heads one-head
        # streams (faster than the key-major rows Int8Rows uses for the self
        # cache; profiles/attend_ring_kernel_decode_b256_pmc.txt).
        self.spans_cross = z(B * hk, 4, dt=i32)
        self.spans_cross[:, 3] = c.frames
        # After a fork, stream b reads the cross memory built for stream
        # mem_of[b] (State.Fork shares it, decoder.go:223-240): the
        # attention takes the (stream, head) -> memory-block index.
        # After a fork the attention reads the index from one buffer, updated
        # in place, so a step graph captured after a fork stays valid across
        # later forks.
        self.mem_of = np.arange(B)
        self.mem_index = None
        self._mem_index_buf = z(B * hk, dt=i32)
        self.x, self.h = z(B, c.dim), z(B, c.dim)
        self.q, self.k, self.v, self.g = z(B, c.dim), z(B, c.dim), z(B, c.dim), z(B, c.dim)
        self.att, self.o = z(B, c.dim), z(B, c.dim)
        self.u = z(B, c.ffn)
        self.logits = z(B, c.vocab)
        # Chained products (cq.gemm_tables_dev): the launch of wo, cross-wo
        # and FFN-down also builds the next product's tables where that
        # product takes the table form, into one buffer the size of the
        # largest (each producer rewrites it after its consumer has read it,
        # in stream order).
        self.chain = fused and not self.paged
        nb = 0
        if self.chain:
            sets = [[self.emb]] + [[mm["wcq"], mm["wcg"]] for mm in self.mats] + [[mm["w1"]] for mm in self.mats]
            if c.head_dim == 64:
                sets += [[mm["wq"], mm["wk"], mm["wv"], mm["wg"]] for mm in self.mats]
            nb = max(cq.tables_bytes(st, B) for st in sets)
        self.tables = z(max(nb, 1), dt=torch.uint8)
        self.n_chained = 0  # products of the last step run on tables their producer built
        hk = c.dim // c.head_dim
        # Every layer's self K and V caches are slices of one array (codes and
        # scales), [2 * layers][stream][position][...], K of layer l at 2l and
        # V at 2l + 1: the paged fork copies all their pages in one launch.
        self._self_q = z(2 * c.layers, B, c.max_pos, c.dim, dt=i8)
        self._self_s = z(2 * c.layers, B, c.max_pos, hk)
        self.self_k = [self._self_q[2 * l] for l in range(c.layers)]
        self.self_ks = [self._self_s[2 * l] for l in range(c.layers)]
        self.self_v = [self._self_q[2 * l + 1] for l in range(c.layers)]
        self.self_vs = [self._self_s[2 * l + 1] for l in range(c.layers)]
        self.cross_k = [z(B, hk, c.frames, c.head_dim, dt=i8) for _ in range(c.layers)]
        self.cross_ks = [z(B, hk, c.frames) for _ in range(c.layers)]
        self.cross_v = [z(B, hk, c.frames, c.head_dim, dt=i8) for _ in range(c.layers)]
        self.cross_vs = [z(B, hk, c.frames) for _ in range(c.layers)]
        if self.paged:
            self._init_paged(torch, z)

    def _init_paged(self, torch, z):
        """The paged step's state: the page tables (identity: stream b's
        logical page j is pool page b * pages_per_stream + j, the same layout
        as the unpaged caches), the tap histories, the feature weights and
        the mHC buffers."""
        c, B, m = self.cfg, self.batch, self.model
        f32 = torch.float32
        dev = self.x.device
        self.page_stride = c.max_pos // self.PAGE_ROWS
        self.pool_pages = B * self.page_stride
        self.pt = np.arange(self.pool_pages, dtype=np.int32).reshape(B, self.page_stride)
        self.pages = torch.from_numpy(self.pt.copy()).to(dev)
        # the tap history: a ring of taps slots per stream, [batch][taps][3][dim]
        # (all layers' in one array: a fork gathers them in one launch)
        self._hist_all = z(c.layers, B, c.taps, 3, c.dim) if c.taps > 1 else None
        self.hist = [self._hist_all[l] for l in range(c.layers)] if c.taps > 1 else None
        dv = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)
        self.qk_gains, self.post_gains = dv(m.qk_gains), dv(m.post_gains)
        self.taps_w, self.mhc_affine = dv(m.taps_w), dv(m.mhc_affine)
        self.res_scale = np.asarray(m.res_scale, np.float32)
        self.o = z(B, c.dim)
        if c.lanes:
            n = c.lanes
            self.lane_s = [z(B, n * c.dim), z(B, n * c.dim)]
            self.nxq = z(B, n * c.dim)
            self.phil = z(B, 2 * n + n * n)  # pre, post, res logits of each activation
            self.hp, self.hq, self.hr = z(B, n), z(B, n), z(B, n * n)
            self.u_mhc, self.blk = z(B, c.dim), z(B, c.dim)

    def set_memory(self, seed, generator="numpy"):
        """Builds each stream's int8 cross memory from its encoder states
        (cross.project, cross.go:181-204): per layer K, V = GEMMs(Wck, Wcv)
        over the frames, then QuantizeRows per head, bit for bit. generator
        "numpy" draws the states with encoder_states; "device" draws them on
        the GPU (torch's seeded Philox) for large batches."""
        import torch

        c = self.cfg
        enc = torch.empty(c.frames * c.dim, dtype=torch.float32, device=self.x.device)
        tmp_k = torch.empty_like(enc)
        tmp_v = torch.empty_like(enc)
        gen = torch.Generator(device=self.x.device)
        for b in range(self.batch):
            if generator == "numpy":
                enc.copy_(torch.from_numpy(encoder_states(seed, c, b)))
            else:
                gen.manual_seed(seed * 1000003 + b)
                torch.randn(enc.shape, generator=gen, out=enc, device=enc.device)
            for layer in range(c.layers):
                m = self.mats[layer]
                cq.gemms_dev([m["wck"], m["wcv"]], [tmp_k, tmp_v], enc, c.frames)
                hk = c.dim // c.head_dim
                if c.cross_norm:  # the memory keys' per-head norm (cross.go:186-188)
                    check(lib().nd_zcrmsnorm_dev(_ptr(tmp_k), _ptr(tmp_k), _ptr(self.qk_gains[layer, 3]),
                                                 c.frames * hk, c.head_dim, cq._stream()))
                for tmp, dq, ds in ((tmp_k, self.cross_k[layer][b], self.cross_ks[layer][b]),
                                    (tmp_v, self.cross_v[layer][b], self.cross_vs[layer][b])):
                    # head-major rows of one head each: QuantizeRow per 64-wide chunk, as on the key-major rows
                    hm = tmp.view(c.frames, hk, c.head_dim).transpose(0, 1).contiguous()
                    needle.quantize_rows_dev(dq, ds, hm, hk * c.frames, c.head_dim, c.head_dim)
        self.mem_of = np.arange(self.batch)
        self.mem_index = None
        self._mem_index_buf.copy_(torch.arange(self._mem_index_buf.numel(), dtype=torch.int32))  # graphs that read it
        torch.cuda.synchronize()

    def encoder_states_device(self, seed, stream):
        """The encoder states set_memory(generator="device") drew for one
        stream, copied to the host."""
        import torch

        c = self.cfg
        gen = torch.Generator(device=self.x.device)
        gen.manual_seed(seed * 1000003 + stream)
        return torch.randn(c.frames * c.dim, generator=gen, device=self.x.device).cpu().numpy()

    def reset(self, tokens):
        import torch

        self.tok.copy_(torch.as_tensor(np.asarray(tokens, np.int32), device=self.tok.device))
        self.pos.zero_()
        self.done.zero_()
        self._sync_spans()
        self.steps = 0
        if self.paged:
            self.pt = np.arange(self.pool_pages, dtype=np.int32).reshape(self.batch, self.page_stride)
            self.pages.copy_(torch.from_numpy(self.pt.copy()))

    def _sync_spans(self):
        """The self-attention key bound of the next step, pos + 1 (the step
        itself keeps it, in its argmax launch)."""
        import torch

        torch.add(self.pos, 1, out=self.spans_self[:, 3])

    def _reserve(self, n):
        """Checks that n more steps fit the caches and RoPE tables: the
        reference's cache slicing and table lookup panic past them."""
        from ._lib import CQPanic

        if n < 0 or self.steps + n > self.cfg.max_pos:
            raise CQPanic(f"decoder: {n} more tokens after {self.steps} exceed max_pos {self.cfg.max_pos}")

    def _attend(self, layer, cross, s, rope=None):
        c, B = self.cfg, self.batch
        hk = c.dim // c.head_dim
        if cross:  # head-major memory: batch * heads streams of one head
            n, d = c.frames, c.head_dim
            args = [_ptr(self.att), 0, _ptr(self.q), 0, 1, 1, _ptr(self.cross_k[layer]), _ptr(self.cross_ks[layer]), d,
                    d, _ptr(self.cross_v[layer]), _ptr(self.cross_vs[layer]), d, d, n * d, n, _ptr(self.spans_cross),
                    n, float(np.float32(math.sqrt(c.head_dim))), 1, B * hk]
            if self.mem_index is None:
                check(lib().kv_attend_int8_dev(*args, s))
            else:  # forked streams share their parents' memories
                check(lib().kv_attend_int8_shared_dev(*args, _ptr(self.mem_index), B * hk, s))
            return
        else:
            kq, ks, vq, vs, spans, n = (self.self_k[layer], self.self_ks[layer], self.self_v[layer],
                                        self.self_vs[layer], self.spans_self, c.max_pos)
        args = [_ptr(self.att), 0, _ptr(self.q), 0, 1, c.heads, _ptr(kq), _ptr(ks), c.dim, c.head_dim, _ptr(vq),
                _ptr(vs), c.dim, c.head_dim, n * c.dim, n * hk, _ptr(spans), n,
                float(np.float32(math.sqrt(c.head_dim))), 1, B]
        if rope is None:
            check(lib().kv_attend_int8_dev(*args, s))
        else:
            check(lib().kv_attend_int8_rope_dev(*args, *[_ptr(t) for t in rope], s))

    def step(self):
        """One greedy token for every stream: reads tok and pos, writes the
        next token to tok and advances pos (and the key bound pos + 1)."""
        self._reserve(1)
        if self.paged:
            self._step_paged()
        elif self.fused:
            self._step_fused()
        else:
            self._step_plain()
        self.steps += 1

    def _advance(self, s):
        """argmax of the logits into tok, pos += 1 and the next step's key
        bound, in one launch."""
        c = self.cfg
        if self.eos is None:
            check(lib().nd_argmax_advance_dev(_ptr(self.tok), _ptr(self.logits), self.batch, c.vocab, _ptr(self.pos),
                                              _ptr(self.spans_self[:, 3]), 4, s))
        else:
            check(lib().nd_argmax_advance_eos_dev(_ptr(self.tok), _ptr(self.logits), self.batch, c.vocab,
                                                  _ptr(self.pos), _ptr(self.spans_self[:, 3]), 4, _ptr(self.done),
                                                  int(self.eos), s))

    def _produce(self, m, y, x, nxt, gain, gate=None, resid=None):
        """y = [resid +] m . (x [* sigmoid(gate)]); returns the tables of the
        next product over nxt (of ZCRMSNorm(y; gain)) when the launch built
        them, else None (the next product then runs unchained)."""
        B = self.batch
        nb = cq.tables_bytes(nxt, B) if self.chain and nxt else 0
        if nb:
            t = self.tables[:nb]
            return t if cq.gemm_tables_dev(m, y, x, B, nxt, t, gate=gate, resid=resid, next_gain=gain) else None
        if gate is not None:
            cq.gemms_gated_dev([m], [y], x, gate, B, resid=resid)
        else:
            cq.gemms_fused_dev([m], [y], x, B, resid=resid)
        return None

    def _step_fused(self):
        c, B = self.cfg, self.batch
        s = cq._stream()
        D, hk = c.dim, c.dim // c.head_dim
        self.emb.row_gather_dev(self.x, self.tok, float(self.model.scale))
        rope = (self.cos, self.sin)
        qkvg = lambda m: [m["wq"], m["wk"], m["wv"], m["wg"]]
        tab = None  # the next product's tables, built by the previous product's launch
        self.n_chained = 0
        for l in range(c.layers):
            m = self.mats[l]
            if c.head_dim == 64:  # heads are the lut kernel's 64-row blocks: the appends ride on the product
                caches = [None, (self.self_k[l], self.self_ks[l], rope), (self.self_v[l], self.self_vs[l], None),
                          None]
                if tab is not None:
                    self.n_chained += 1
                    cq.gemms_tables_dev(qkvg(m), [self.q, self.k, self.v, self.g], B, tab, caches=caches,
                                        q_stride=c.max_pos * D, s_stride=c.max_pos * hk, pos=self.pos, cap=c.max_pos)
                else:
                    cq.gemms_append_dev(qkvg(m), [self.q, self.k, self.v, self.g], self.x, B, caches, c.max_pos * D,
                                        c.max_pos * hk, self.pos, c.max_pos, norm_gain=self.gains[3 * l])
            else:
                cq.gemms_fused_dev(qkvg(m), [self.q, self.k, self.v, self.g], self.x, B, norm_gain=self.gains[3 * l])
                needle.append_dev(self.self_k[l], self.self_ks[l], self.k, B, D, c.head_dim, c.max_pos * D,
                                  c.max_pos * hk, self.pos, c.max_pos, rope=rope)
                needle.append_dev(self.self_v[l], self.self_vs[l], self.v, B, D, c.head_dim, c.max_pos * D,
                                  c.max_pos * hk, self.pos, c.max_pos)
            self._attend(l, False, s, rope=(self.cos, self.sin, self.pos))
            cross = [m["wcq"], m["wcg"]]
            tab = self._produce(m["wo"], self.x, self.att, cross, self.gains[3 * l + 1], gate=self.g, resid=self.x)
            if tab is not None:
                self.n_chained += 1
                cq.gemms_tables_dev(cross, [self.q, self.g], B, tab)
            else:
                cq.gemms_fused_dev(cross, [self.q, self.g], self.x, B, norm_gain=self.gains[3 * l + 1])
            self._attend(l, True, s)
            tab = self._produce(m["wco"], self.x, self.att, [m["w1"]], self.gains[3 * l + 2], gate=self.g,
                                resid=self.x)
            if tab is not None:
                self.n_chained += 1
                cq.gemms_tables_dev([m["w1"]], [self.u], B, tab, act=1)
            else:
                cq.gemms_fused_dev([m["w1"]], [self.u], self.x, B, norm_gain=self.gains[3 * l + 2], act=1)
            if l + 1 < c.layers:
                nxt = qkvg(self.mats[l + 1]) if c.head_dim == 64 else None
            else:
                nxt = [self.emb]
            tab = self._produce(m["w2"], self.x, self.u, nxt, self.gains[3 * l + 3], resid=self.x)
        if tab is not None:
            self.n_chained += 1
            cq.gemms_tables_dev([self.emb], [self.logits], B, tab)
        else:
            cq.gemms_fused_dev([self.emb], [self.logits], self.x, B, norm_gain=self.gains[3 * c.layers])
        self._advance(s)

    def _step_plain(self):
        c, B, L = self.cfg, self.batch, lib()
        s = cq._stream()
        D, hk = c.dim, c.dim // c.head_dim
        self.emb.row_gather_dev(self.x, self.tok, float(self.model.scale))
        for l in range(c.layers):
            m = self.mats[l]
            check(L.nd_zcrmsnorm_dev(_ptr(self.h), _ptr(self.x), _ptr(self.gains[3 * l]), B, D, s))
            cq.gemms_dev([m["wq"], m["wk"], m["wv"], m["wg"]], [self.q, self.k, self.v, self.g], self.h, B)
            for t in (self.q, self.k):
                check(L.nd_rope_dev(_ptr(t), B, c.heads, c.head_dim, _ptr(self.cos), _ptr(self.sin), c.max_pos,
                                    _ptr(self.pos), 1, s))
            for src, cq_, cs_ in ((self.k, self.self_k[l], self.self_ks[l]), (self.v, self.self_v[l], self.self_vs[l])):
                check(L.kv_append_dev(_ptr(cq_), _ptr(cs_), _ptr(src), B, D, c.head_dim, c.max_pos * D,
                                      c.max_pos * hk, _ptr(self.pos), c.max_pos, s))
            self._attend(l, False, s)
            check(L.nd_sigmoid_gate_dev(_ptr(self.att), _ptr(self.g), B * D, s))
            m["wo"].gemm_dev(self.o, self.att, B)
            check(L.nd_add_dev(_ptr(self.x), _ptr(self.o), B * D, s))
            check(L.nd_zcrmsnorm_dev(_ptr(self.h), _ptr(self.x), _ptr(self.gains[3 * l + 1]), B, D, s))
            cq.gemms_dev([m["wcq"], m["wcg"]], [self.q, self.g], self.h, B)
            self._attend(l, True, s)
            check(L.nd_sigmoid_gate_dev(_ptr(self.att), _ptr(self.g), B * D, s))
            m["wco"].gemm_dev(self.o, self.att, B)
            check(L.nd_add_dev(_ptr(self.x), _ptr(self.o), B * D, s))
            check(L.nd_zcrmsnorm_dev(_ptr(self.h), _ptr(self.x), _ptr(self.gains[3 * l + 2]), B, D, s))
            m["w1"].gemm_dev(self.u, self.h, B)
            check(L.nd_silu_dev(_ptr(self.u), B * c.ffn, s))
            m["w2"].gemm_dev(self.o, self.u, B)
            check(L.nd_add_dev(_ptr(self.x), _ptr(self.o), B * D, s))
        check(L.nd_zcrmsnorm_dev(_ptr(self.h), _ptr(self.x), _ptr(self.gains[3 * c.layers]), B, D, s))
        self.emb.gemm_dev(self.logits, self.h, B)
        self._advance(s)

    def _step_paged(self):
        """One token with the reference step's features (each per the
        configuration): the layer of decoder.go:446-505 (Block.run with the
        cross branch after the attention, block.go:147-215) inside the mHC
        lanes (mhc.go:182-299), the self caches read and written through the
        page tables."""
        c, B, L = self.cfg, self.batch, lib()
        s = cq._stream()
        D, H, hd = c.dim, c.heads, c.head_dim
        n = c.lanes
        P = _ptr
        rope = (self.cos, self.sin)
        self.emb.row_gather_dev(self.x, self.tok, float(self.model.scale))
        cur = None
        if n:
            check(L.nd_expand_lanes_dev(P(self.lane_s[0]), P(self.x), B, n, D, s))
            cur, nxt = self.lane_s
        for l in range(c.layers):
            m = self.mats[l]
            h_in = self.x  # the block's input h; with lanes u, which stays unchanged for the mix
            if n:  # the mHC heads and the block input u (mhc.go:196-219)
                check(L.nd_rms_unit_quant_dev(P(self.nxq), P(cur), B, n * D, s))
                m["phi"].gemm_dev(self.phil, self.nxq, B)
                check(L.nd_mhc_heads_stacked_dev(P(self.hp), P(self.hq), P(self.hr), P(self.u_mhc), P(self.phil),
                                                 P(cur), B, n, D, P(self.mhc_affine[l]), s))
                h_in = self.u_mhc
            cq.gemms_fused_dev([m["wq"], m["wk"], m["wv"], m["wg"]], [self.q, self.k, self.v, self.g], h_in, B,
                               norm_gain=self.gains[3 * l])
            qg = P(self.qk_gains[l, 0]) if c.qk_norm else None
            kg = P(self.qk_gains[l, 1]) if c.qk_norm else None
            hist = P(self.hist[l]) if self.hist is not None else None
            check(L.nd_qkv_prep_dev(P(self.q), P(self.k), P(self.v), B, D, hist, P(self.taps_w[l]), c.taps, qg, kg,
                                    P(self.cos), P(self.sin), c.max_pos, P(self.pos), c.max_pos, P(self.self_k[l]),
                                    P(self.self_ks[l]), P(self.self_v[l]), P(self.self_vs[l]), P(self.pages),
                                    self.page_stride, self.PAGE_ROWS, self.pool_pages, s))
            check(L.kv_attend_int8_paged_dev(P(self.att), 0, P(self.q), 0, 1, H, P(self.self_k[l]), P(self.self_ks[l]),
                                             D, hd, P(self.self_v[l]), P(self.self_vs[l]), D, hd, P(self.spans_self),
                                             c.max_pos, float(np.float32(math.sqrt(hd))), 1, B, P(self.cos),
                                             P(self.sin), P(self.pos), P(self.pages), self.page_stride,
                                             self.PAGE_ROWS, self.pool_pages, s))
            if c.post_norm:  # block.go:183-188: x = h + float32(gate * postNorm(o))
                cq.gemms_gated_dev([m["wo"]], [self.o], self.att, self.g, B)
                check(L.nd_norm_scaled_add_dev(P(self.x), P(h_in), P(self.o), P(self.post_gains[l, 0]),
                                               float(self.res_scale[l, 0]), B, D, s))
            else:
                cq.gemms_gated_dev([m["wo"]], [self.x], self.att, self.g, B, resid=h_in)
            cq.gemms_fused_dev([m["wcq"], m["wcg"]], [self.q, self.g], self.x, B, norm_gain=self.gains[3 * l + 1])
            if c.cross_norm:  # cross.go:217-219
                check(L.nd_zcrmsnorm_dev(P(self.q), P(self.q), P(self.qk_gains[l, 2]), B * H, hd, s))
            self._attend(l, True, s)
            if c.cross_norm:  # cross.go:255-263 and the hook's add
                cq.gemms_gated_dev([m["wco"]], [self.o], self.att, self.g, B)
                check(L.nd_norm_scaled_add_dev(P(self.x), None, P(self.o), P(self.post_gains[l, 1]),
                                               float(self.res_scale[l, 1]), B, D, s))
            else:
                cq.gemms_gated_dev([m["wco"]], [self.x], self.att, self.g, B, resid=self.x)
            cq.gemms_fused_dev([m["w1"]], [self.u], self.x, B, norm_gain=self.gains[3 * l + 2], act=1)
            if n:  # the block's output, then y = out - u and the lane mix (mhc.go:221-234)
                cq.gemms_fused_dev([m["w2"]], [self.blk], self.u, B, resid=self.x)
                check(L.nd_mhc_mix_dev(P(nxt), P(cur), P(self.hr), P(self.hq), P(self.blk), P(self.u_mhc), B, n, D,
                                       s))
                cur, nxt = nxt, cur
            else:
                cq.gemms_fused_dev([m["w2"]], [self.x], self.u, B, resid=self.x)
        if n:
            check(L.nd_collapse_lanes_dev(P(self.x), P(cur), B, n, D, s))
        cq.gemms_fused_dev([self.emb], [self.logits], self.x, B, norm_gain=self.gains[3 * c.layers])
        self._advance(s)

    def _fork_paged(self, parents, pos):
        """The paged fork: stream b takes its parent's page table, so the
        full pages so far are shared, never copied; every page from the one
        the next append writes on must be the stream's own, so a shared one
        is replaced by a free page (the partly filled one copied first, at
        most a page of rows per stream and layer, whatever the position).
        Then the tap histories follow the parents."""
        import torch

        c, B, R = self.cfg, self.batch, self.PAGE_ROWS
        pt, copies = fork_page_tables(self.pt, parents, pos, R, self.pool_pages)
        self.pt = pt
        dev = self.x.device
        self.pages.copy_(torch.from_numpy(pt))
        s = cq._stream()
        if copies:
            # every layer's K and V pool at once: pool k of the 2 * layers
            # is pages [k * pool_pages, (k + 1) * pool_pages) of one array
            npool = 2 * c.layers
            base = np.arange(npool, dtype=np.int64)[:, None] * self.pool_pages
            cp = np.array(copies, np.int64).T
            src, dst = (cp[0][None, :] + base).ravel(), (cp[1][None, :] + base).ravel()
            cpd = torch.as_tensor(np.stack([src, dst]).astype(np.int32), device=dev)
            check(lib().kv_page_copy_dev(_ptr(self._self_q), _ptr(self._self_s), _ptr(cpd[0]), _ptr(cpd[1]), src.size,
                                         R, c.dim, c.head_dim, npool * self.pool_pages, s))
        if self.hist is not None:
            # row l * B + b of every layer's history takes row l * B + parents[b]
            L = c.layers
            idx = (np.arange(L, dtype=np.int64)[:, None] * B + np.asarray(parents, np.int64)[None, :]).ravel()
            par = torch.as_tensor(idx.astype(np.int32), device=dev)
            width = self.hist[0][0].numel()
            if getattr(self, "_hist_tmp", None) is None:
                self._hist_tmp = torch.empty_like(self._hist_all)
            check(lib().nd_gather_rows_dev(_ptr(self._hist_tmp), _ptr(self._hist_all), _ptr(par), L * B, width, s))
            check(lib().nd_gather_rows_dev(_ptr(self._hist_all), _ptr(self._hist_tmp), None, L * B, width, s))
        self.fork_copies = len(copies)

    def fork(self, parents):
        """KVCache.Fork / State.Fork for every stream at once (cache.go:
        62-67, decoder.go:223-240), as a beam search reorders its
        hypotheses: stream b continues from stream parents[b]'s state (its
        token, position, self-attention rows so far and cross memory), after
        which every stream extends on its own. The cross memory is shared,
        never copied: stream b reads its parent's through the attention's
        memory index. The self rows so far are copied (kv_reorder_dev), not
        shared until written, so a fork's cost grows with the decoded
        positions only, not with the frames."""
        import torch

        from ._lib import CQPanic

        c, B = self.cfg, self.batch
        if len(parents) != B or any(not 0 <= int(p) < B for p in parents):
            raise CQPanic(f"decoder: fork of {B} streams from parents {list(parents)}")
        dev = self.tok.device
        parents = np.asarray(parents, np.int64)
        par = torch.as_tensor(parents.astype(np.int32), device=dev)
        self_len = self.pos.index_select(0, par.long()).to(torch.int32)
        hk = c.dim // c.head_dim
        if self.paged:
            self._fork_paged(parents, self_len.cpu().numpy())
        else:
            if getattr(self, "_fork_tmp", None) is None:
                self._fork_tmp = (torch.empty(B * c.max_pos * c.dim, dtype=torch.int8, device=dev),
                                  torch.empty(B * c.max_pos * hk, dtype=torch.float32, device=dev))
            tq, ts = self._fork_tmp
            s = cq._stream()
            for l in range(c.layers):
                for q, sc in ((self.self_k[l], self.self_ks[l]), (self.self_v[l], self.self_vs[l])):
                    check(lib().kv_reorder_dev(_ptr(q), _ptr(sc), _ptr(tq), _ptr(ts), _ptr(par), _ptr(self_len), B,
                                               c.max_pos, c.dim, c.head_dim, s))
        self.mem_of = self.mem_of[parents]
        blocks = (self.mem_of[:, None] * hk + np.arange(hk)[None, :]).astype(np.int32).reshape(-1)
        self._mem_index_buf.copy_(torch.from_numpy(blocks))
        self.mem_index = self._mem_index_buf
        self.tok.copy_(self.tok.index_select(0, par.long()))
        self.pos.copy_(self.pos.index_select(0, par.long()))
        self.done.copy_(self.done.index_select(0, par.long()))
        self._sync_spans()

    def resume(self, n, graph=True, eos=None, check_every=16):
        """Greedy-decodes n more tokens from the current state; [batch, n].

        With eos (a token id), each stream stops at its own EOS, as
        GreedyMemory stops (greedy.go:50-66): the row holds the stream's
        tokens, then -1 from its EOS on (the reference's Result.Tokens
        leaves EOS out); stopped[b] is True for a stream that stopped at
        EOS, False for one that reached n tokens (MaxTokens). Every
        check_every steps the host looks at the streams' done flags and
        ends early once all have stopped."""
        import torch

        from ._lib import CQPanic

        self._reserve(n)
        if eos is not None and not 0 <= int(eos) < self.cfg.vocab:
            raise CQPanic(f"decoder: stop token {eos} outside a vocabulary of {self.cfg.vocab}")
        self.eos = None if eos is None else int(eos)
        out = torch.zeros(self.batch, n, dtype=torch.int32, device=self.tok.device)
        try:
            done = 0
            g = self.capture() if graph and n > 0 else None
            while done < n:
                if g is None:
                    self.step()
                else:
                    g.replay()
                    self.steps += 1
                out[:, done] = self.tok
                done += 1
                if self.eos is not None and done % check_every == 0 and done < n and bool(self.done.all()):
                    out[:, done:] = self.eos
                    break
        finally:
            eos, self.eos = self.eos, None
        if eos is not None:
            hit = out == eos
            after = torch.cumsum(hit.to(torch.int32), dim=1) > 0
            out[after] = -1
            self.stopped = hit.any(dim=1).cpu().numpy()
        return out

    def decode(self, first_tokens, n, graph=True, eos=None):
        """Greedy-decodes n tokens after first_tokens; returns [batch, n]
        (with eos: each stream up to its EOS, then -1, as resume says).
        n past max_pos raises CQPanic before anything runs."""
        from ._lib import CQPanic

        if not 0 <= n <= self.cfg.max_pos:
            raise CQPanic(f"decoder: {n} tokens exceed max_pos {self.cfg.max_pos}")
        self.reset(first_tokens)
        return self.resume(n, graph, eos)

    def capture(self):
        """A HIP graph of one step (the state it reads is on the device).
        Replaying it does not advance the host's step count: resume() does."""
        import torch

        pos0, tok0, done0, steps0 = self.pos.clone(), self.tok.clone(), self.done.clone(), self.steps
        self.step()  # kernel attributes are set outside the capture
        torch.cuda.synchronize()
        self.pos.copy_(pos0)
        self.tok.copy_(tok0)
        self.done.copy_(done0)
        self._sync_spans()
        self.steps = steps0
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        self.steps = steps0
        return g  # capturing runs nothing: the state is as before
