"""The decode step with the reference step's features on the device (the
paged step of go-whistle_amd/decoder.py) against the oracle decoder
(oracle/decode_oracle.c): the causal taps (internal/needle/cache.go:
143-154), the per-head q/k norms before RoPE (attention.go:298-330), the
attention's post norm and residual factor (block.go:183-188), the cross
q/k norms, post norm and residual factor (internal/decoder/cross.go:
181-264) and the mHC lanes (internal/needle/mhc.go:182-299), each alone
and all together, greedy tokens identical and the last logits bit for
bit; the paged self caches with forks that share the rows so far
(KVCache.Fork, cache.go:62-67; State.Fork, decoder.go:218-240), at any
position, repeatedly, against the oracle's forked states; and the kernels
of the step against the oracle one by one."""

import math

import numpy as np
import pytest

from go_whistle_amd import decoder as dec
from go_whistle_amd._lib import check, lib
from oracle import binding as orc
from oracle import decoder_ref

pytestmark = pytest.mark.gpu

SMALL = dict(vocab=4096, layers=2, frames=100, max_pos=64)


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _p(t):
    from ctypes import c_void_p

    return c_void_p(t.data_ptr()) if t is not None else None


def _s():
    from go_whistle_amd import cq

    return cq._stream()


def _check(cfg, seed, batch, first, n, streams, generator="numpy", paged=None):
    model = dec.make_model(seed, cfg)
    d = dec.Decoder(model, batch, paged=paged)
    d.set_memory(seed, generator)
    toks = d.decode(first, n).cpu().numpy()
    logits = d.logits.cpu().numpy()
    ref = decoder_ref.RefDecoder(model)
    for b in streams:
        enc = dec.encoder_states(seed, cfg, b) if generator == "numpy" else d.encoder_states_device(seed, b)
        ref.memory(enc)
        want, wl = ref.decode(first[b], n, want_logits=True)
        assert list(toks[b]) == want, (b, list(toks[b]), want)
        assert same(logits[b], wl[-1]), b
    return toks


FEATURES = {
    "taps": dict(taps=3),
    "qk_norm": dict(qk_norm=True),
    "post_norm": dict(post_norm=True),
    "cross_norm": dict(cross_norm=True),
    "lanes": dict(lanes=4),
    "all": dict(taps=3, qk_norm=True, post_norm=True, cross_norm=True, lanes=4),
}


@pytest.mark.parametrize("name", list(FEATURES))
def test_feature_step_bit_exact(name):
    cfg = dec.DecoderConfig(**SMALL, **FEATURES[name])
    print("feature step", name, flush=True)
    _check(cfg, 5, 3, [1, 2, 3], 24, [0, 1, 2])


def test_paged_step_without_features_equals_fused():
    # the paged step with every feature off is the synthetic decoder: its
    # tokens equal the fused step's (and the oracle's)
    cfg = dec.DecoderConfig(**SMALL)
    got = _check(cfg, 5, 3, [1, 2, 3], 24, [0, 1, 2], paged=True)
    model = dec.make_model(5, cfg)
    d = dec.Decoder(model, 3)
    d.set_memory(5)
    assert np.array_equal(d.decode([1, 2, 3], 24).cpu().numpy(), got)


def test_whistle_step_batch1_200_tokens():
    cfg = dec.DecoderConfig.whistle()
    print("whistle step, batch 1, 200 tokens", flush=True)
    toks = _check(cfg, 7, 1, [1], 200, [0])
    assert len(set(toks[0].tolist())) > 3


def test_whistle_step_batch256_streams():
    cfg = dec.DecoderConfig.whistle()
    print("whistle step, batch 256, 100 tokens", flush=True)
    _check(cfg, 9, 256, list(range(256)), 100, [0, 131, 255], generator="device")


def _fork_case(cfg, batch, rounds, seed=21):
    """Decode n tokens, fork to random parents, repeat; every stream against
    the oracle's states forked the same way."""
    model = dec.make_model(seed, cfg)
    d = dec.Decoder(model, batch)
    d.set_memory(seed)
    ref = decoder_ref.RefDecoder(model)
    mems = [ref.build_memory(dec.encoder_states(seed, cfg, b)) for b in range(batch)]
    first = list(range(3, 3 + batch))
    states = [ref.state(mems[b]) for b in range(batch)]
    g = np.random.default_rng(seed)
    last = list(first)
    d.reset(first)
    copies = []
    for r, (n, parents) in enumerate(rounds):
        got = d.resume(n).cpu().numpy()
        for b in range(batch):
            want, _, _ = states[b].greedy(last[b], n)
            assert list(got[b]) == want, (r, b, list(got[b]), want)
            last[b] = want[-1]
        if parents is None:
            continue
        parents = list(parents) if parents != "random" else list(g.integers(0, batch, size=batch))
        d.fork(parents)
        copies.append(d.fork_copies)
        states = [states[p].fork() for p in parents]
        last = [last[p] for p in parents]
    return copies


def test_fork_shares_pages_at_any_position():
    # forks mid-page (position 21), on a page boundary (32) and late (53):
    # every stream continues as its oracle fork, and a fork copies at most
    # one page per stream and layer pair whatever the position
    cfg = dec.DecoderConfig(**SMALL, **FEATURES["all"])
    copies = _fork_case(cfg, 4, [(21, [2, 0, 2, 3]), (11, [1, 1, 0, 3]), (21, [3, 3, 3, 3]), (6, None)])
    assert copies[0] <= 4 and copies[1] == 0 and copies[2] <= 4
    assert copies[0] > 0 and copies[2] > 0


def test_fork_beam_rounds():
    # beam-like: a fork after every few tokens, random parents, 8 rounds
    cfg = dec.DecoderConfig(**SMALL, taps=3, lanes=4, qk_norm=True)
    rounds = [(3, "random")] * 8 + [(5, None)]
    copies = _fork_case(cfg, 5, rounds, seed=33)
    assert max(copies) <= 5


def test_capture_at_a_later_position_keeps_the_taps():
    # a step graph captured at position 19 (its capture run steps once):
    # the tap history the replayed step reads is the one before it
    cfg = dec.DecoderConfig(**SMALL, taps=3)
    model = dec.make_model(5, cfg)
    d = dec.Decoder(model, 2)
    d.set_memory(5)
    d.reset([1, 2])
    a = d.resume(19, graph=False).cpu().numpy()
    b = d.resume(10).cpu().numpy()
    ref = decoder_ref.RefDecoder(model)
    for s in range(2):
        ref.memory(dec.encoder_states(5, cfg, s))
        want = ref.decode(s + 1, 29)
        assert list(a[s]) + list(b[s]) == want, s


def test_graph_captured_after_a_fork_replays_after_another():
    # a step graph captured after one fork and replayed after a second: the
    # graph reads the page tables, the cross-memory index and the tap
    # histories in place, so every stream still continues as its oracle fork
    cfg = dec.DecoderConfig(**SMALL, **FEATURES["all"])
    model = dec.make_model(23, cfg)
    batch = 4
    d = dec.Decoder(model, batch)
    d.set_memory(23)
    ref = decoder_ref.RefDecoder(model)
    states = [ref.state(ref.build_memory(dec.encoder_states(23, cfg, b))) for b in range(batch)]
    first = [3, 4, 5, 6]
    d.reset(first)
    got = d.resume(7).cpu().numpy()
    last = []
    for b in range(batch):
        want, _, _ = states[b].greedy(first[b], 7)
        assert list(got[b]) == want, b
        last.append(want[-1])
    for k, parents in enumerate(([1, 1, 3, 0], [2, 0, 0, 3])):
        d.fork(parents)
        states = [states[p].fork() for p in parents]
        last = [last[p] for p in parents]
        if k == 0:
            g = d.capture()
    toks = []
    for _ in range(6):
        g.replay()
        d.steps += 1
        toks.append(d.tok.cpu().numpy().copy())
    got = np.stack(toks, 1)
    for b in range(batch):
        want, _, _ = states[b].greedy(last[b], 6)
        assert list(got[b]) == want, (b, list(got[b]), want)


def test_fork_plain_config_paged():
    # the synthetic decoder (no features) on the paged step forks by pages too
    cfg = dec.DecoderConfig(**SMALL)
    model = dec.make_model(5, cfg)
    d = dec.Decoder(model, 3, paged=True)
    d.set_memory(5)
    d.decode([1, 2, 3], 10)
    d.fork([2, 2, 1])
    assert d.fork_copies <= 3
    got = d.resume(8).cpu().numpy()
    ref = decoder_ref.RefDecoder(model)
    states = []
    for b in range(3):
        ref.memory(dec.encoder_states(5, cfg, b))
        st = ref.state()
        toks, _, _ = st.greedy(b + 1, 10)
        states.append((st, toks[-1]))
    for b, p in enumerate([2, 2, 1]):
        f = states[p][0].fork()
        want, _, _ = f.greedy(states[p][1], 8)
        assert list(got[b]) == want, b


# ---- the step's kernels, one by one, against the oracle -------------------


def test_qkv_prep_kernel():
    # taps over the history, the q/k head norms, RoPE of k and the paged
    # int8 appends at each stream's position, against the oracle's pieces
    import torch

    g = np.random.default_rng(4)
    B, D, taps, R, per = 5, 512, 3, 16, 4
    pool = B * per
    hk = D // 64
    pos = np.array([0, 1, 2, 17, 63], np.int32)
    q, k, v = (g.standard_normal((B, D)).astype(np.float32) * 3 for _ in range(3))
    hist = g.standard_normal((B, taps, 3, D)).astype(np.float32)
    w = g.standard_normal((3, taps, D)).astype(np.float32)
    qg, kg = (1 + g.standard_normal(64) * 0.1).astype(np.float32), (1 + g.standard_normal(64) * 0.1).astype(np.float32)
    cos, sin = dec.rope_tables(64, 64, 1e5)
    pt = g.permutation(pool).astype(np.int32).reshape(B, per)
    kq, vq = torch.zeros(pool * R, D, dtype=torch.int8, device="cuda"), torch.zeros(pool * R, D, dtype=torch.int8,
                                                                                   device="cuda")
    ks, vs = torch.zeros(pool * R, hk, device="cuda"), torch.zeros(pool * R, hk, device="cuda")
    # every device operand held in a name for the call (a temporary's memory
    # goes back to torch's cache at once and the next tensor takes it)
    qd, hd, kd, vd, wd, qgd, kgd, cd, sd, posd, ptd = (_t(a) for a in (q, hist, k, v, w, qg, kg, cos, sin, pos, pt))
    check(lib().nd_qkv_prep_dev(_p(qd), _p(kd), _p(vd), B, D, _p(hd), _p(wd), taps, _p(qgd), _p(kgd), _p(cd), _p(sd),
                                64, _p(posd), 64, _p(kq), _p(ks), _p(vq), _p(vs), _p(ptd), per, R, pool, _s()))
    torch.cuda.synchronize()
    gq, gh = qd.cpu().numpy(), hd.cpu().numpy()
    kqn, ksn, vqn, vsn = kq.cpu().numpy(), ks.cpu().numpy(), vq.cpu().numpy(), vs.cpu().numpy()
    for b in range(B):
        p = int(pos[b])
        out = []
        for z, raw in enumerate((q[b], k[b], v[b])):
            acc = np.zeros(D, np.float32)
            for j in range(taps):
                if j > p:
                    break
                src = raw if j == 0 else hist[b, (p - j) % taps, z]
                acc = (acc + (w[z, j] * src).astype(np.float32)).astype(np.float32)
            out.append(acc)
            assert same(gh[b, p % taps, z], raw)
            for j in range(1, taps):  # the slots the step reads are untouched
                assert same(gh[b, (p - j) % taps, z], hist[b, (p - j) % taps, z])
        tq = orc.zc_rmsnorm(out[0], qg, 64)
        tk = orc.rope(orc.zc_rmsnorm(out[1], kg, 64), hk, 64, cos, sin, [p])
        assert same(gq[b], tq), b
        row = pt[b, p // R] * R + p % R
        for got_q, got_s, val in ((kqn, ksn, tk), (vqn, vsn, out[2])):
            wq, ws = orc.quantize_rows(val, D, 64)
            assert np.array_equal(got_q[row], wq) and same(got_s[row], ws), b


def test_norm_scaled_add_and_lanes():
    import torch

    g = np.random.default_rng(5)
    rows, D, n = 7, 512, 4
    h, y = g.standard_normal((rows, D)).astype(np.float32), (g.standard_normal((rows, D)) * 5).astype(np.float32)
    gain = (1 + g.standard_normal(D) * 0.1).astype(np.float32)
    hd, yd, gd, h2 = _t(h), _t(y), _t(gain), _t(h)
    check(lib().nd_norm_scaled_add_dev(_p(hd), None, _p(yd), _p(gd), 0.37, rows, D, _s()))
    r = g.standard_normal((rows, D)).astype(np.float32)
    rd, od = _t(r), torch.zeros(rows, D, device="cuda")
    check(lib().nd_norm_scaled_add_dev(_p(od), _p(rd), _p(yd), _p(gd), 0.37, rows, D, _s()))
    torch.cuda.synchronize()
    ny = orc.zc_rmsnorm(y.ravel(), gain, D).reshape(rows, D)
    want = (h + (np.float32(0.37) * ny).astype(np.float32)).astype(np.float32)
    assert same(hd.cpu().numpy(), want)
    assert same(od.cpu().numpy(), (r + (np.float32(0.37) * ny).astype(np.float32)).astype(np.float32))
    # RMSUnit and its fused fakeQuant over rows of 2048 (and 512), with a zero
    # row and rows holding NaN / Inf, against the oracle
    for dim in (2048, 512):
        xs = (g.standard_normal((6, dim)) * 3).astype(np.float32)
        xs[1] = 0
        xs[2, 7], xs[3, 100], xs[4, 5] = np.nan, np.inf, -np.inf
        xsd, u1, u2 = _t(xs), torch.zeros(6, dim, device="cuda"), torch.zeros(6, dim, device="cuda")
        check(lib().nd_rms_unit_dev(_p(u1), _p(xsd), 6, dim, _s()))
        check(lib().nd_rms_unit_quant_dev(_p(u2), _p(xsd), 6, dim, _s()))
        torch.cuda.synchronize()
        wu = orc.rms_unit(xs.ravel(), 6, dim)
        wq = orc.fake_quant(wu, dim, dim)
        for got, want in ((u1, wu), (u2, wq)):
            a, b = got.cpu().numpy().ravel(), want.ravel()
            nb = np.isnan(b)
            assert np.array_equal(np.isnan(a), nb) and np.array_equal(a[~nb].view(np.uint32), b[~nb].view(np.uint32))
    st = torch.zeros(rows, n * D, device="cuda")
    check(lib().nd_expand_lanes_dev(_p(st), _p(h2), rows, n, D, _s()))
    s2 = g.standard_normal((rows, n * D)).astype(np.float32)
    xd, s2d = torch.zeros(rows, D, device="cuda"), _t(s2)
    check(lib().nd_collapse_lanes_dev(_p(xd), _p(s2d), rows, n, D, _s()))
    torch.cuda.synchronize()
    assert same(st.cpu().numpy(), np.tile(h, n))
    acc = np.zeros((rows, D), np.float32)
    for k in range(n):
        acc = (acc + s2[:, k * D:(k + 1) * D]).astype(np.float32)
    assert same(xd.cpu().numpy(), (acc / np.float32(n)).astype(np.float32))


def test_paged_attention_equals_contiguous():
    # the four attention kernels through a shuffled page table equal the
    # same keys laid out contiguously: the resident chain kernel (1 and 3
    # streams), the ring (72 streams), the one-wavefront chain (48-code
    # keys), the streamed kernel (128-code values) and the general kernel
    # (widths 20/40)
    import torch

    g = np.random.default_rng(6)
    R, per = 16, 8
    for B, H, qk, vd in ((1, 8, 64, 64), (3, 8, 64, 64), (72, 8, 64, 64), (72, 8, 48, 64), (3, 4, 64, 128),
                         (3, 4, 20, 40)):
        print("paged attention", B, H, qk, vd, flush=True)
        cap = R * per
        pool = B * per
        kc, vc = H * qk, H * vd
        kq = g.integers(-128, 128, size=(pool * R, kc), dtype=np.int8)
        vq = g.integers(-128, 128, size=(pool * R, vc), dtype=np.int8)
        ks, vs = g.uniform(0.01, 0.1, (pool * R, H)).astype(np.float32), g.uniform(0.01, 0.1, (pool * R, H)).astype(
            np.float32)
        pt = g.permutation(pool).astype(np.int32).reshape(B, per)
        n = g.integers(1, cap + 1, size=B)
        spans = np.zeros((B, 4), np.int32)
        spans[:, 3] = n
        q = g.standard_normal((B, H * qk)).astype(np.float32)
        out = torch.zeros(B, H * vd, device="cuda")
        qd, kqd, ksd, vqd, vsd, spd, ptd = (_t(a) for a in (q, kq, ks, vq, vs, spans, pt))
        check(lib().kv_attend_int8_paged_dev(_p(out), 0, _p(qd), 0, 1, H, _p(kqd), _p(ksd), kc, qk, _p(vqd), _p(vsd), vc,
                                             vd, _p(spd), cap, float(np.float32(math.sqrt(qk))), 1, B, None, None,
                                             None, _p(ptd), per, R, pool, _s()))
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        for b in range(B):  # the oracle over the stream's rows gathered through its table
            rows = (pt[b][:, None] * R + np.arange(R)[None, :]).reshape(-1)[:n[b]]
            want = orc.attend_int8_spans(q[b], 1, H, kq[rows].reshape(-1), ks[rows].reshape(-1), kc, qk,
                                         vq[rows].reshape(-1), vs[rows].reshape(-1), vc, vd, int(n[b]),
                                         np.array([[0, 0, 0, n[b]]], np.int32), np.float32(math.sqrt(qk)), True, 1)
            assert same(got[b], want), (B, qk, vd, b)
