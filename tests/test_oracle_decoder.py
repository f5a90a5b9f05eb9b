"""The oracle decoder's C token loop (decode_oracle.c) against compose_step,
a second restatement of the same layer written in Python over the
oracle's single operations (each pinned on its own in test_oracle_*.py):
logits bit for bit and tokens identical, with every feature of the
reference step off, all on, and in part (taps, mHC lanes with q/k norms);
a fork continues exactly as its parent; the threaded many-stream loop
equals one stream at a time."""

import numpy as np
import pytest

from go_whistle_amd import decoder as dec
from oracle import decoder_ref as dr

SMALL = dict(layers=2, vocab=2048, frames=64, max_pos=16)
CFGS = {
    "plain": dec.DecoderConfig(**SMALL),
    "whistle": dec.DecoderConfig.whistle(**SMALL),
    "taps": dec.DecoderConfig(taps=3, **SMALL),
    "lanes_qk": dec.DecoderConfig(lanes=4, qk_norm=True, **dict(SMALL, layers=3)),
    "norms": dec.DecoderConfig(post_norm=True, cross_norm=True, **SMALL),
}


def _composed(ref, first, n):
    c = ref.cfg
    hk = c.dim // c.head_dim
    hist = [[[], [], []] for _ in range(c.layers)]
    caches = [[np.zeros(c.max_pos * c.dim, np.int8), np.zeros(c.max_pos * hk, np.float32),
               np.zeros(c.max_pos * c.dim, np.int8), np.zeros(c.max_pos * hk, np.float32)] for _ in range(c.layers)]
    tok, toks, lgs = first, [], []
    for pos in range(n):
        lg, tok = dr.compose_step(ref, ref.mem, hist, caches, tok, pos)
        toks.append(tok)
        lgs.append(lg)
    return toks, lgs


@pytest.mark.parametrize("name", list(CFGS))
def test_c_loop_equals_composition(name):
    cfg = CFGS[name]
    model = dec.make_model(7, cfg)
    ref = dr.RefDecoder(model)
    ref.memory(dec.encoder_states(7, cfg, 0))
    toks, lgs = ref.decode(5, 10, want_logits=True)
    wt, wl = _composed(ref, 5, 10)
    assert toks == wt
    for a, b in zip(lgs, wl):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_features_change_the_step():
    # each feature on its own changes the logits (so each is exercised)
    base = dict(SMALL)
    logits = {}
    for name, cfg in [("plain", dec.DecoderConfig(**base)), ("taps", dec.DecoderConfig(taps=3, **base)),
                      ("qk", dec.DecoderConfig(qk_norm=True, **base)), ("post", dec.DecoderConfig(post_norm=True, **base)),
                      ("cross", dec.DecoderConfig(cross_norm=True, **base)), ("lanes", dec.DecoderConfig(lanes=4, **base))]:
        ref = dr.RefDecoder(dec.make_model(7, cfg))
        ref.memory(dec.encoder_states(7, cfg, 0))
        st = ref.state()
        st.step(5)
        logits[name] = st.step(9)[1]  # position 1: the taps reach back
    for name in logits:
        if name != "plain":
            assert not np.array_equal(logits[name], logits["plain"]), name


def test_taps_identity():
    # taps [1, 0, 0] are the identity: the step equals the one without taps
    cfg = dec.DecoderConfig(taps=3, **SMALL)
    model = dec.make_model(7, cfg)
    model.taps_w[:] = 0
    model.taps_w[:, :, 0] = 1
    plain = dec.make_model(7, dec.DecoderConfig(**SMALL))
    a, b = dr.RefDecoder(model), dr.RefDecoder(plain)
    a.memory(dec.encoder_states(7, cfg, 0))
    b.memory(dec.encoder_states(7, cfg, 0))
    ta, la = a.decode(3, 8, want_logits=True)
    tb, lb = b.decode(3, 8, want_logits=True)
    assert ta == tb and all(np.array_equal(x, y) for x, y in zip(la, lb))


def test_fork_continues_as_parent():
    cfg = CFGS["whistle"]
    ref = dr.RefDecoder(dec.make_model(11, cfg))
    ref.memory(dec.encoder_states(11, cfg, 0))
    whole = ref.decode(4, 12)
    st = ref.state()
    head, _, _ = st.greedy(4, 5)
    f = st.fork()
    assert head == whole[:5] and len(f) == len(st) == 5
    ta, _, _ = st.greedy(head[-1], 7)
    tb, _, _ = f.greedy(head[-1], 7)
    assert ta == tb == whole[5:]


def test_streams_loop_equals_single():
    cfg = CFGS["whistle"]
    ref = dr.RefDecoder(dec.make_model(13, cfg))
    mems = [ref.build_memory(dec.encoder_states(13, cfg, b)) for b in range(3)]
    toks, counts = ref.decode_streams(mems, [1, 2, 3], 6, 3)
    assert list(counts) == [6, 6, 6]
    for b in range(3):
        ref.mem = mems[b]
        assert list(toks[b]) == ref.decode(b + 1, 6)
