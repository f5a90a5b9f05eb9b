"""CPU baselines of bench.py's legs beyond the GEMV sweep, on the oracle's
restatement of the reference's CPU path (AVX2 forms where the host has
them): the batched GEMM, int8 attention at batch 1 and 256, the decode at
batch 1 and 256, and the reference's own benchmark shapes.

Batch-256 legs run streams concurrently, one stream per worker process, as
the reference runs one goroutine per hypothesis (internal/search/
beam.go:508-521); each worker's products and attention are single-threaded.
Workers are spawned (a fresh interpreter that never touches the GPU).

TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline legs import it; the
product package never does.
"""

import concurrent.futures as cf
import importlib.util
import math
import multiprocessing as mp
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _package():
    """The go_whistle_amd package for its seeded generators (numpy only: no
    library call, no device)."""
    if "go_whistle_amd" in sys.modules:
        return sys.modules["go_whistle_amd"]
    pkg_dir = os.path.join(ROOT, "go-whistle_amd")
    spec = importlib.util.spec_from_file_location("go_whistle_amd", os.path.join(pkg_dir, "__init__.py"),
                                                  submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["go_whistle_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def _orc():
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    from oracle import binding as orc

    return orc


def _pool(workers):
    return cf.ProcessPoolExecutor(max_workers=workers, mp_context=mp.get_context("spawn"))


# ---------------------------------------------------------------- attention

def attention_inputs(kind, n, seed, heads=8, head_dim=64):
    """One stream of config 4: Q ~N(0,1); K, V ~N(0,1) quantised per row and
    head (QuantizeRows, int8.go:36-55) into key-major rows of heads*head_dim
    codes. kind 'self' attends keys 0..n-1 of an n-key cache, 'cross' a
    memory of n frames (the same call, as cross.attend makes it)."""
    orc = _orc()
    g = np.random.Generator(np.random.PCG64(seed))
    cols = heads * head_dim
    q = g.standard_normal(cols).astype(np.float32)
    k = g.standard_normal(n * cols).astype(np.float32)
    v = g.standard_normal(n * cols).astype(np.float32)
    kq, ks = orc.quantize_rows(k, cols, head_dim)
    vq, vs = orc.quantize_rows(v, cols, head_dim)
    spans = np.array([[0, n, 0, 0]] if kind == "self" else [[0, 0, 0, n]], np.int32)
    return q, kq, ks, vq, vs, spans


def _attend(orc, inp, n, heads=8, head_dim=64):
    q, kq, ks, vq, vs, spans = inp
    cols = heads * head_dim
    return orc.attend_int8_spans(q, 1, heads, kq, ks, cols, head_dim, vq, vs, cols, head_dim, n, spans,
                                 np.float32(math.sqrt(head_dim)), True, 1)


def attention_calls(kind, n, seconds, seed):
    """Calls of one stream's int8 attention (8 heads) in about `seconds`, on
    one thread: (calls, elapsed)."""
    orc = _orc()
    orc.set_cpu(orc.have_avx2(), 1)
    inp = attention_inputs(kind, n, seed)
    _attend(orc, inp, n)
    done, t0 = 0, time.perf_counter()
    while True:
        _attend(orc, inp, n)
        done += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            return done, el


def attention_baseline(cases, seconds, workers):
    """For each (kind, n): batch 1, one stream on one thread; batch 256,
    `workers` streams at once in worker processes. Rates in stream-steps/s
    (one query row of every head against the stream's keys)."""
    orc = _orc()
    out = {}
    for kind, n in cases:
        c, el = attention_calls(kind, n, seconds, 5)
        out[f"b1_{kind}{n}"] = {"stream_steps_per_s": round(c / el, 1), "us_per_step": round(el / c * 1e6, 2),
                                "threads": 1, "calls": c, "seconds": round(el, 2)}
    with _pool(workers) as ex:
        for kind, n in cases:
            t0 = time.perf_counter()
            futs = [ex.submit(attention_calls, kind, n, seconds, 100 + w) for w in range(workers)]
            res = [f.result() for f in futs]
            wall = time.perf_counter() - t0
            calls = sum(r[0] for r in res)
            rate = sum(r[0] / r[1] for r in res)
            out[f"b256_{kind}{n}"] = {"stream_steps_per_s": round(rate, 1), "processes": workers,
                                      "calls": calls, "seconds": round(wall, 2)}
    return {"unit": "stream-steps/s", "cores": workers, "kind": "port", "avx2": bool(orc.have_avx2()),
            "cases": out,
            "sample": f"oracle AttendInt8Spans (int8 query, amd64 exp; {'AVX2' if orc.have_avx2() else 'generic'} "
                      f"dots/axpys), 8 heads x 64, K/V ~N(0,1) quantised per row; batch 1 on one thread, batch 256 "
                      f"as {workers} concurrent single-threaded streams, about {seconds:.1f} s per case"}


# ---------------------------------------------------------------- GEMM

def gemm_baseline(shapes, threads, seconds):
    """The oracle's lut GEMM (gemmLUT's split over `threads`) on each
    (bits, out, in, rows): rows per second, timed on at most min(rows, cap)
    activations within about `seconds` per shape (time is linear in rows)."""
    orc = _orc()
    gw = _package()
    orc.set_cpu(orc.have_avx2(), threads)
    g = gw.synth.rng(31)
    out = {}
    try:
        for bits, o, i, rows in shapes:
            m = orc.OMatrix.new(gw.synth.random_packed(g, o, i, 128, bits, sigma=0.05))
            r = min(rows, 375)
            x = gw.synth.activations(g, r, i)
            m.gemm(x[:i], 1)
            done, t0 = 0, time.perf_counter()
            while True:
                m.gemm(x, r)
                done += r
                el = time.perf_counter() - t0
                if el >= seconds:
                    break
            rps = done / el
            out[f"cq{bits}_{o}x{i}_M{rows}"] = {"rows_per_s": round(rps, 1), "us_per_call": round(rows / rps * 1e6, 1),
                                                "dense_TFLOPs": round(2.0 * o * i * rps / 1e12, 4),
                                                "timed_rows": done, "seconds": round(el, 2)}
    finally:
        orc.set_cpu(False, 1)
    return out


# ---------------------------------------------------------------- decode

def decode_baseline(tokens, threads, workers, cfg=None):
    """The oracle decoder's greedy decode, the token loop in C (one call per
    timed run: orc_dec_greedy / orc_dec_streams), on the 200-token
    workload from position 0. Batch 1: one stream, the lut products split
    over `threads`. Batch 256: `workers` streams decoded at once on as many
    threads, one stream per thread, single-threaded products (as beams run
    one goroutine each; the rate per stream is the same for all 256). Each
    stream's cross memory is built before the timed region (once per clip).
    cfg: the decoder configuration (default: the benchmark's)."""
    orc = _orc()
    gw = _package()
    from go_whistle_amd import decoder as dec
    from oracle import decoder_ref

    cfg = cfg or dec.DecoderConfig()
    model = dec.make_model(7, cfg)
    ref = decoder_ref.RefDecoder(model)
    avx2 = orc.have_avx2()
    kind = "AVX2" if avx2 else "generic"
    try:
        orc.set_cpu(avx2, threads)
        ref.memory(dec.encoder_states(7, cfg, 0))
        t0 = time.perf_counter()
        got = ref.decode(1, tokens)
        el1 = time.perf_counter() - t0
        mems = [ref.build_memory(dec.encoder_states(7, cfg, b)) for b in range(workers)]
        orc.set_cpu(avx2, 1)
        t0 = time.perf_counter()
        toks, counts = ref.decode_streams(mems, list(range(1, workers + 1)), tokens, workers)
        wall = time.perf_counter() - t0
    finally:
        orc.set_cpu(False, 1)
    n256 = int(counts.sum())
    return {
        "batch1": {"value": round(len(got) / el1, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
                   "sample": f"{len(got)} greedy tokens of one stream from position 0 (the 200-token workload), the "
                             f"oracle decoder's C token loop ({kind} lut products split over {threads} threads, int8 "
                             f"attention), {el1:.2f} s"},
        "batch256": {"value": round(n256 / wall, 2), "unit": "tokens/s", "cores": workers, "kind": "port",
                     "sample": f"{workers} streams decoded concurrently on {workers} threads, one stream per thread "
                               f"(as beams run one goroutine each), {tokens} tokens each from position 0, "
                               f"single-threaded {kind} products, the C token loop; {n256} tokens in {wall:.2f} s "
                               f"(cross memories built before)"},
    }


# ---------------------------------------------------------------- reference shapes

def shapes_baseline(shapes, seconds):
    """The reference's BenchmarkGEMM shapes (internal/cq/bench_test.go:23-
    39) on one thread (its -cpu 1): microseconds per call."""
    orc = _orc()
    gw = _package()
    orc.set_cpu(orc.have_avx2(), 1)
    out = {}
    try:
        for name, o, i, bits, rows in shapes:
            g = gw.synth.rng(o * 7919 + i)
            m = orc.OMatrix.new(gw.synth.random_packed(g, o, i, 128, bits, sigma=0.05))
            x = gw.synth.activations(g, rows, i)
            m.gemm(x, rows)
            done, t0 = 0, time.perf_counter()
            while True:
                m.gemm(x, rows)
                done += 1
                el = time.perf_counter() - t0
                if el >= seconds:
                    break
            out[f"{name}_{o}x{i}_cq{bits}_rows{rows}"] = round(el / done * 1e6, 2)
    finally:
        orc.set_cpu(False, 1)
    return out
