"""GPU parity of the decode step with the CPU oracle, through the C ABI:
the float blocks (ZCRMSNorm, RoPE, argmax, SiLU, the residual add, the int8
append) bit for bit, and greedy decoding of the synthetic decoder with
identical tokens and bit-identical logits, at batch 1 (the full model, 200
tokens) and for streams of a batched run."""

import numpy as np
import pytest

from go_whistle_amd import decoder as dec
from go_whistle_amd import needle, synth
from go_whistle_amd._lib import check, lib
from oracle import binding as orc
from oracle import decoder_ref

pytestmark = pytest.mark.gpu


def _t(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _p(t):
    from ctypes import c_void_p

    return c_void_p(t.data_ptr())


def _s():
    import torch
    from ctypes import c_void_p

    return c_void_p(torch.cuda.current_stream().cuda_stream)


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_step_blocks_bit_exact():
    import torch

    g = synth.rng(11)
    rows, dim = 7, 512
    x = (g.standard_normal(rows * dim) * 2).astype(np.float32)
    gain = (1 + g.standard_normal(dim) * 0.1).astype(np.float32)
    xd, yd, gd = _t(x), torch.zeros(rows * dim, device="cuda"), _t(gain)
    check(lib().nd_zcrmsnorm_dev(_p(yd), _p(xd), _p(gd), rows, dim, _s()))
    cos, sin = dec.rope_tables(64, 300, 1e5)
    pos = np.array([0, 1, 5, 63, 100, 200, 299], np.int32)
    rd, cd, sd, pd = _t(x.copy()), _t(cos), _t(sin), _t(pos)  # held: a freed temporary's block is reused
    check(lib().nd_rope_dev(_p(rd), rows, 8, 64, _p(cd), _p(sd), 300, _p(pd), 1, _s()))
    v = g.standard_normal((5, 16384)).astype(np.float32)
    v[1, 3], v[1, 16000] = 40, 40
    v[2] = 1.5
    v[3, 16383] = 30
    am, vd = torch.zeros(5, dtype=torch.int32, device="cuda"), _t(v)
    check(lib().nd_argmax_dev(_p(am), _p(vd), 5, 16384, _s()))
    u = np.concatenate([np.linspace(-40, 40, 4001), (g.standard_normal(3000) * 5)]).astype(np.float32)
    ud = _t(u)
    check(lib().nd_silu_dev(_p(ud), u.size, _s()))
    a, b = g.standard_normal(1000).astype(np.float32), g.standard_normal(1000).astype(np.float32)
    ad, bd = _t(a), _t(b)
    check(lib().nd_add_dev(_p(ad), _p(bd), 1000, _s()))
    torch.cuda.synchronize()
    assert same(yd.cpu().numpy(), orc.zc_rmsnorm(x, gain, dim))
    assert same(rd.cpu().numpy(), orc.rope(x, 8, 64, cos, sin, pos))
    assert list(am.cpu().numpy()) == list(orc.argmax(v, 5, 16384))
    assert list(am.cpu().numpy())[1:4] == [3, 0, 16383]
    assert same(ud.cpu().numpy(), orc.silu(u))
    assert same(ad.cpu().numpy(), (a + b).astype(np.float32))


def test_append_at_positions():
    import torch

    g = synth.rng(12)
    B, cap, cols, width = 3, 10, 512, 64
    x = g.standard_normal(B * cols).astype(np.float32)
    q = torch.zeros(B, cap, cols, dtype=torch.int8, device="cuda")
    s = torch.zeros(B, cap, cols // width, device="cuda")
    pos = np.array([0, 4, 9], np.int32)
    xd, pd = _t(x), _t(pos)
    check(lib().kv_append_dev(_p(q), _p(s), _p(xd), B, cols, width, cap * cols, cap * cols // width, _p(pd), cap,
                              _s()))
    torch.cuda.synchronize()
    qh, sh = q.cpu().numpy(), s.cpu().numpy()
    for b in range(B):
        wq, ws = orc.quantize_rows(x[b * cols:(b + 1) * cols], cols, width)
        assert np.array_equal(qh[b, pos[b]], wq) and same(sh[b, pos[b]], ws)
        others = [p for p in range(cap) if p != pos[b]]
        assert not qh[b, others].any()


@pytest.mark.parametrize("n", [16384, 1001, 5, 4100])
def test_argmax_edges(n):
    # greedy.go's argmax on the device against the oracle: ties (first
    # index), NaN anywhere (never a winner; at index 0 the answer is 0), -0
    # against +0, -inf rows; n = 1001 and 5 take the scalar path, 4100 a
    # partial last round of 16-byte loads
    import torch

    g = synth.rng(n)
    rows = 8
    v = g.standard_normal((rows, n)).astype(np.float32)
    nan = np.float32("nan")
    v[0, n // 2] = v[0, n - 1] = 60  # tie: first wins
    v[1, 0] = nan  # answer 0
    v[2, 1 % n] = nan  # a thread's first value NaN, the true maximum after it
    v[2, n - 1] = 70
    v[3, :] = 0.0
    v[3, 0] = -0.0  # +0 does not beat -0
    v[4, :] = -np.inf
    v[5, ::3] = nan
    v[6, :] = nan
    v[7, n - 1] = 80
    am, vd = torch.zeros(rows, dtype=torch.int32, device="cuda"), _t(v)
    check(lib().nd_argmax_dev(_p(am), _p(vd), rows, n, _s()))
    torch.cuda.synchronize()
    assert list(am.cpu().numpy()) == list(orc.argmax(v, rows, n))


@pytest.mark.parametrize("graph", [True, False])
def test_fork_continues_as_parent(graph):
    import torch

    # KVCache.Fork (cache.go:62-67) for a beam reorder: after 8 tokens, stream
    # b takes stream parents[b]'s state and must go on exactly as that stream
    # does without the fork (its self rows, cross memory, token, position)
    cfg = dec.DecoderConfig(vocab=4096, layers=2, frames=100, max_pos=64)
    model = dec.make_model(9, cfg)
    first, parents = [1, 2, 3, 4], [2, 2, 0, 3]
    whole = dec.Decoder(model, 4)
    whole.set_memory(9)
    full = whole.decode(first, 16, graph=graph).cpu().numpy()
    d = dec.Decoder(model, 4)
    d.set_memory(9)
    head = d.decode(first, 8, graph=graph).cpu().numpy()
    assert np.array_equal(head, full[:, :8])
    cross = [t.clone() for t in d.cross_k + d.cross_vs]
    d.fork(parents)
    # the memories are shared through the index, not copied (State.Fork,
    # decoder.go:223-240): the arrays are as they were
    assert all(torch.equal(a, b) for a, b in zip(cross, d.cross_k + d.cross_vs))
    assert list(d.mem_of) == parents
    tail = d.resume(8, graph=graph).cpu().numpy()
    for b, p in enumerate(parents):
        assert list(tail[b]) == list(full[p, 8:]), (b, p)
    # a second fork composes: stream b now reads the memory of parents[p2[b]]
    d.fork([1, 1, 3, 0])
    assert list(d.mem_of) == [parents[1], parents[1], parents[3], parents[0]]
    with pytest.raises(Exception):
        d.fork([0, 1, 2])


def test_reorder_rows():
    # kv_reorder_dev against numpy: stream b <- rows [0, len[b]) of stream
    # parent[b], the rest untouched, for code rows of 16-byte multiples and
    # of odd widths (the byte path)
    import torch

    g = synth.rng(44)
    for cols, width in ((512, 64), (40, 8)):
        B, cap = 5, 7
        q = g.integers(-128, 128, size=(B, cap, cols), dtype=np.int8)
        s = g.random((B, cap, cols // width)).astype(np.float32)
        parent = np.array([3, 3, 0, 4, 1], np.int32)
        ln = np.array([0, 7, 3, 9, 1], np.int32)  # 9 > cap: clamped
        qd, sd = _t(q), _t(s)
        tq, ts = torch.empty_like(qd), torch.empty_like(sd)
        pd, ld = _t(parent), _t(ln)  # held: a freed temporary's block is reused
        check(lib().kv_reorder_dev(_p(qd), _p(sd), _p(tq), _p(ts), _p(pd), _p(ld), B, cap, cols, width, _s()))
        torch.cuda.synchronize()
        wq, ws = q.copy(), s.copy()
        for b in range(B):
            n = min(int(ln[b]), cap)
            wq[b, :n], ws[b, :n] = q[parent[b], :n], s[parent[b], :n]
        assert np.array_equal(qd.cpu().numpy(), wq) and same(sd.cpu().numpy(), ws)


def _run(cfg, seed, batch, first, n, check_streams, generator="numpy"):
    model = dec.make_model(seed, cfg)
    d = dec.Decoder(model, batch)
    d.set_memory(seed, generator)
    toks = d.decode(first, n).cpu().numpy()
    logits = d.logits.cpu().numpy()
    ref = decoder_ref.RefDecoder(model)
    for b in check_streams:
        enc = dec.encoder_states(seed, cfg, b) if generator == "numpy" else d.encoder_states_device(seed, b)
        ref.memory(enc)
        want, wl = ref.decode(first[b], n, want_logits=True)
        assert list(toks[b]) == want, (b, list(toks[b]), want)
        assert same(logits[b], wl[-1]), b
    return toks


def test_small_decoder_batch_bit_exact():
    cfg = dec.DecoderConfig(vocab=4096, layers=2, frames=100, max_pos=64)
    toks = _run(cfg, 5, 3, [1, 2, 3], 24, [0, 1, 2])
    assert len(set(toks[0].tolist())) > 1


def _eos_case(n_batch, first, n, eos_from, check_every=16, shared=False):
    """Decodes without a stop token, picks EOS as a token stream eos_from[0]
    emits at step eos_from[1], decodes again with it: each stream must give
    its oracle's GreedyMemory tokens, stopping at its own first EOS. shared:
    every stream reads stream 0's cross memory (a fork from stream 0)."""
    cfg = dec.DecoderConfig(vocab=4096, layers=2, frames=100, max_pos=64)
    model = dec.make_model(5, cfg)
    d = dec.Decoder(model, n_batch)
    d.set_memory(5)
    if shared:
        d.fork([0] * n_batch)
    plain = d.decode(first, n).cpu().numpy()
    eos = int(plain[eos_from[0], eos_from[1]])
    d.reset(first)
    got = d.resume(n, eos=eos, check_every=check_every).cpu().numpy()
    pos = d.pos.cpu().numpy()
    ref = decoder_ref.RefDecoder(model)
    enc = {}
    for b in range(n_batch):
        m = 0 if shared else b
        ref.memory(enc.setdefault(m, dec.encoder_states(5, cfg, m)))
        want = ref.decode(first[b], n, eos=eos)
        row = list(got[b])
        k = row.index(-1) if -1 in row else n
        assert row[:k] == want and all(t == -1 for t in row[k:]), (b, row, want)
        assert bool(d.stopped[b]) == ref.stopped, b
        # a stopped stream's position froze after the step that gave EOS
        assert pos[b] == (len(want) + 1 if ref.stopped else n), (b, pos[b])
        # tokens before the stop are the plain run's
        assert list(plain[b][:k]) == want, b
    return d, eos


def test_eos_stops_each_stream():
    d, eos = _eos_case(4, [1, 2, 3, 4], 40, (1, 12))
    assert d.stopped[1]


def test_eos_ends_the_batch_once_every_stream_stopped():
    # two streams with the same first token and memory decode alike: both
    # stop at the same step, and the host ends the run at its next check
    d, eos = _eos_case(2, [7, 7], 40, (0, 2), check_every=4, shared=True)
    assert all(d.stopped)
    assert d.steps <= 8


def test_full_decoder_batch1_200_tokens():
    cfg = dec.DecoderConfig()
    print("full decoder, batch 1, 200 tokens", flush=True)
    toks = _run(cfg, 7, 1, [1], 200, [0])
    assert len(set(toks[0].tolist())) > 5


def test_full_decoder_batch256_streams():
    # config 5 at batch 256: the whole 200-token run, five streams checked
    # (each against its own C restatement), among them the last
    cfg = dec.DecoderConfig()
    print("full decoder, batch 256, 200 tokens", flush=True)
    _run(cfg, 9, 256, list(range(256)), 200, [0, 77, 131, 200, 255], generator="device")


def test_argmax_advances_positions():
    # nd_argmax_advance_dev: the argmax of nd_argmax_dev, pos += 1 and the
    # key bound pos + 1 in the spans' fourth column, nothing else touched
    import torch

    g = synth.rng(3)
    rows, n = 6, 16384
    v = g.standard_normal((rows, n)).astype(np.float32)
    pos = np.array([0, 5, 9, 200, 1, 7], np.int32)
    spans = g.integers(0, 9, size=(rows, 4)).astype(np.int32)
    am, vd, pd, sd = torch.zeros(rows, dtype=torch.int32, device="cuda"), _t(v), _t(pos), _t(spans)
    check(lib().nd_argmax_advance_dev(_p(am), _p(vd), rows, n, _p(pd), _p(sd[:, 3]), 4, _s()))
    torch.cuda.synchronize()
    assert list(am.cpu().numpy()) == list(orc.argmax(v, rows, n))
    assert list(pd.cpu().numpy()) == list(pos + 1)
    want = spans.copy()
    want[:, 3] = pos + 2
    assert np.array_equal(sd.cpu().numpy(), want)
