"""Benchmark: go-whistle's CQ LUT GEMV at batch 1 on one MI355X.

Workload (the reference's GEMV sweep): 2- and 4-bit CQ matrices of
512x512, 2048x512, 512x2048 and 16384x512 (group 128, 4 or 16 codebook
levels ~N(0, 0.05), uniform random indices, FP16 norms), x ~N(0, 1), one
activation each. A step multiplies every matrix of `copies` distinct device
copies of the sweep once (the copies together exceed twice the 256 MiB
MALL, so the weights stream from HBM). The GEMVs run through a batch
plan of the C ABI (cq_batch_*): one lut-kernel launch per index width, 2
launches per step, each GEMV bit for bit cq_gemm_dev's result. Inputs are
resident in HBM before the timed region.

value = weight bytes (packed index + FP16 norms) of all GEMVs of a step /
step time, in GB/s. The roofline object is the step's dominant launch, the
4-bit one (HIP events on its stream around 4 back-to-back launches, inside
steps). detail holds per-shape
rates and the rate of one launch per GEMV (a captured graph of 8 * copies
launches). The cpu_baseline is the C restatement of the reference's lut
kernel (oracle/) on the host cores, on a bounded sample of the same sweep.

Further legs, each with its own cpu_baseline (the oracle, bounded samples;
batch-256 legs run streams concurrently, one per host process, as the
reference runs one goroutine per hypothesis): batched_gemm (the encoder's
M x 512 / M x 2048 products, M = 375, 1500, 12000), ref_shapes (the
reference's BenchmarkGEMM shapes with its published M5 Pro times),
attention (int8 KV attention at batch 1 and 256, self and cross), aux
(HadamardMLP and the mHC block at 1/375/1500 rows) and decode (the
synthetic decoder's 200-token greedy decode at batch 1 and 256).
"""

import argparse
import importlib.util
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
SHAPES = [(512, 512), (2048, 512), (512, 2048), (16384, 512)]
BITS = (4, 2)
GROUP = 128
ROOF_REPS = 4
PMC_SUMMARY = os.path.join(ROOT, "profiles", "lut_kernel_4bit_sweep_pmc.txt")


def _package():
    if "go_whistle_amd" in sys.modules:
        return sys.modules["go_whistle_amd"]
    pkg_dir = os.path.join(ROOT, "go-whistle_amd")
    spec = importlib.util.spec_from_file_location("go_whistle_amd", os.path.join(pkg_dir, "__init__.py"),
                                                  submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["go_whistle_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def weight_bytes(out, inp, bits):
    groups = (inp + GROUP - 1) // GROUP
    return out * groups * GROUP * bits // 8 + 2 * out * groups


def algorithmic_bytes(out, inp, bits):
    return weight_bytes(out, inp, bits) + 4 * inp + 4 * out + 4 * (1 << bits)


def pmc_traffic():
    """HBM bytes per 4-bit sweep launch from the committed rocprofv3 counter
    summary (FETCH_SIZE and WRITE_SIZE, each scaled by what the counter
    reads for a plain copy of known size), or None without it."""
    try:
        for line in open(PMC_SUMMARY):
            if line.startswith("traffic_bytes_per_launch"):
                return int(line.split("=")[1].split()[0])
    except OSError:
        pass
    return None


PREWARM_MS = 60.0


def prewarm(torch, fn, target_ms=PREWARM_MS):
    """Runs fn back to back for about target_ms of GPU time before a timed
    region, whatever --warmup says: the GPU's clocks settle over the first
    ~10 ms of sustained load, and launches before that run up to ~20%
    slower. Returns the GPU milliseconds it ran (HIP events)."""
    for _ in range(2):
        fn()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    fn()
    e1.record()
    torch.cuda.synchronize()
    once = max(e0.elapsed_time(e1), 1e-3)
    n = max(1, math.ceil(target_ms / once))
    e0.record()
    for _ in range(n):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def cpu_threads():
    """Host cores this process may use, at most 16 (one GPU's share)."""
    return max(1, min(16, len(os.sched_getaffinity(0))))


def cpu_host():
    """The host CPU's model name, its logical CPU count and the CPUs this
    process may use."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"model": model, "nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0))}


def cpu_baseline(gw, packs, seconds):
    """The oracle's lut GEMV over the sweep, bounded in time, three ways: the
    generic restatement on one thread, its AVX2 form (the reference's amd64
    path, lut_amd64.s, bit for bit the generic one) on one thread, and the
    AVX2 form on every host core this process may use, split as the
    reference splits a GEMV (lut.go:102-201). value is the last: the
    reference's own CPU path at its own parallelism."""
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    from oracle import binding as orc

    g = gw.synth.rng(99)
    mats = [(orc.OMatrix.new(p), gw.synth.activations(g, 1, p.In), weight_bytes(p.Out, p.In, p.Bits))
            for p in packs]
    threads = cpu_threads()
    legs = [("generic_1t", False, 1)]
    if orc.have_avx2():
        legs += [("avx2_1t", True, 1), (f"avx2_{threads}t", True, threads)]
    res = {}
    for name, avx2, th in legs:
        orc.set_cpu(avx2, th)
        done, passes, t0 = 0, 0, time.perf_counter()
        while True:
            for m, x, wb in mats:
                m.gemm(x, 1, orc.LUT)
                done += wb
            passes += 1
            el = time.perf_counter() - t0
            if el >= seconds / len(legs):
                break
        res[name] = (done / el / 1e9, passes, el, th)
    orc.set_cpu(False, 1)
    name = legs[-1][0]
    rate, passes, el, th = res[name]
    return {"value": round(rate, 4), "unit": "GB/s", "cores": th, "kind": "port",
            "sample": f"{passes} passes over the 8-matrix sweep (one copy each), oracle lut GEMV, {name} "
                      f"({'AVX2' if 'avx2' in name else 'generic'}, {th} threads, the reference's split), {el:.1f} s",
            "legs": {k: {"GBps": round(v[0], 4), "threads": v[3], "passes": v[1], "seconds": round(v[2], 2)}
                     for k, v in res.items()},
            "host": cpu_host()}


INT8_PEAK_OPS = 5.0e15  # MI355X dense int8 MFMA, ops/s
FP32_PEAK_FLOPS = 157.3e12  # MI355X dense fp32 MFMA, flop/s


def _gemm_times(torch, call, reps, eager_reps=40):
    """(graph-replayed us per call, eager us per call) of `call`, each after
    20 ms of the same work: a graph of `reps` calls replayed 4 times, and
    `eager_reps` calls queued one by one (enough that the first call's host
    latency does not dominate)."""
    call()
    torch.cuda.synchronize()
    prewarm(torch, call, 20)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(eager_reps):
        call()
    e1.record()
    torch.cuda.synchronize()
    eager = e0.elapsed_time(e1) * 1e3 / eager_reps
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            call()
    graph.replay()
    torch.cuda.synchronize()
    prewarm(torch, graph.replay, 20)
    e0.record()
    for _ in range(4):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (4 * reps)
    del graph
    return us, eager


def batched_gemm_leg(gw, torch, reps=5):
    """The encoder's batched CQ GEMMs: X [M x In] ~N(0, 1) times 4/2-bit
    2048x512 and 512x2048 (FFN up/down), M in {375, 1500, 12000}, through
    cq_gemm_dev (which picks the lut kernel or its MFMA form). `us` is the
    GPU time of one call: a graph of `reps` calls replayed after 20 ms of
    replays; `us_eager` times 40 calls queued from Python one after the
    other (the launches' own gaps, and the workspace lease's event between
    calls, are then part of it).
    Flops are the
    dense equivalent 2*M*Out*In; for the MFMA forms, mfma_util is the int8 MFMA
    work it issues (one 32x32x32 product per 64-row block, 64-activation tile,
    position and 32x32 quadrant) over the time, against 5.0 POP/s. dense_f32
    times the same matrix's Dense view (Exact's semantics on fp32 MFMA, the
    whole call: rotation, product and any fold); its mfma_util_fp32 is the
    fp32 MFMA work the padded 128 x 128 tiles issue over that time, against
    157.3 TFLOP/s."""
    g = gw.synth.rng(31)
    out = {}
    for bits in (4, 2):
        for (o, i) in ((2048, 512), (512, 2048)):
            m = gw.cq.New(gw.synth.random_packed(g, o, i, GROUP, bits, sigma=0.05))
            for M in (375, 1500, 12000):
                x = torch.randn(M, i, device="cuda")
                y = torch.empty(M, o, device="cuda")
                us, us_eager = _gemm_times(torch, lambda: m.gemm_dev(y, x, M), reps)
                path = m.gemm_path(M)
                rec = {"path": path, "us": round(us, 2), "us_eager": round(us_eager, 2),
                       "dense_TFLOPs": round(2.0 * M * o * i / us / 1e6, 2)}
                if path in ("lut-mfma", "lut-mfma-split", "lut-mfma-tab"):
                    # one 32x32x32 int8 product per 32 weight rows, 32 activations and table position
                    # (the 512-row form pads activations to its 64-wide tiles, the split and table
                    # forms to 32)
                    positions = (i // GROUP) * (2 * GROUP * bits // 8)
                    tile = 64 if path == "lut-mfma" else 32
                    mfmas = -(-o // 64) * 2 * (-(-M // tile) * tile // 32) * positions
                    ops = mfmas * 2 * 32 * 32 * 32
                    rec["mfma_TOPs"] = round(ops / us / 1e6, 1)
                    rec["mfma_util"] = round(ops / (us * 1e-6) / INT8_PEAK_OPS, 4)
                # The Dense view of the same matrix: Exact's semantics on fp32
                # MFMA (v_mfma_f32_32x32x2_f32 over 128 x 128 tiles, the
                # activations rotated first), within float32 rounding of Exact.
                d = m.Dense()
                dus, dus_eager = _gemm_times(torch, lambda: d.gemm_dev(y, x, M), reps)
                issued = 2.0 * (-(-M // 128) * 128) * (-(-o // 128) * 128) * (-(-i // 64) * 64)
                rec["dense_f32"] = {"path": d.gemm_path(M), "us": round(dus, 2), "us_eager": round(dus_eager, 2),
                                    "dense_TFLOPs": round(2.0 * M * o * i / dus / 1e6, 2),
                                    "mfma_util_fp32": round(issued / (dus * 1e-6) / FP32_PEAK_FLOPS, 4)}
                out[f"cq{bits}_{o}x{i}_M{M}"] = rec
                del x, y
    return out


def batched_gemm_cpu(seconds):
    """The batched GEMM leg's shapes on the oracle's lut GEMM, split over
    the host cores as gemmLUT splits a GEMM (lut.go:88-124)."""
    from oracle import cpu_legs

    threads = cpu_threads()
    shapes = [(bits, o, i, M) for bits in (4, 2) for (o, i) in ((2048, 512), (512, 2048)) for M in (375, 1500, 12000)]
    res = cpu_legs.gemm_baseline(shapes, threads, seconds)
    return {"unit": "rows/s", "cores": threads, "kind": "port", "host": cpu_host(), "configs": res,
            "sample": f"oracle lut GEMM (AVX2 where the host has it) over at most 375 activations of each shape, "
                      f"repeated for about {seconds:.1f} s, split over {threads} threads; time is linear in rows"}


# The reference's own benchmark shapes (internal/cq/bench_test.go:23-39)
# and its published M5 Pro single-core lut times (docs/FINDINGS.md:2675-2686).
REF_SHAPES = [("k_proj", 96, 512, 2, 1, 1.15), ("q_proj", 384, 512, 2, 1, 2.91), ("out_proj", 512, 512, 2, 1, 3.68),
              ("pw1", 1024, 512, 2, 1, 6.84), ("stem.out", 512, 1280, 2, 1, 9.18), ("phi_res", 128, 2048, 4, 1, 8.89),
              ("head", 8199, 512, 4, 1, 97.2), ("q_proj", 384, 512, 2, 5, 14.5), ("head", 8199, 512, 4, 5, 487.0),
              ("q_proj", 384, 512, 2, 375, 1090.0)]


def ref_shapes_leg(gw, torch, with_cpu, cpu_seconds):
    """BenchmarkGEMM's shapes and batches through cq_gemm_dev: microseconds
    per call (a captured graph of 20 calls on the same inputs, so the small
    matrices stay cache-resident, as the reference's repeated b.Loop calls
    do), next to the reference's published M5 Pro times and the oracle on
    one host thread (its -cpu 1)."""
    out = {}
    for name, o, i, bits, rows, m5 in REF_SHAPES:
        g = gw.synth.rng(o * 7919 + i)
        m = gw.cq.New(gw.synth.random_packed(g, o, i, GROUP, bits, sigma=0.05))
        x = torch.from_numpy(gw.synth.activations(g, rows, i)).cuda()
        y = torch.empty(rows, o, device="cuda")
        m.gemm_dev(y, x, rows)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(20):
                m.gemm_dev(y, x, rows)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / 100
        out[f"{name}_{o}x{i}_cq{bits}_rows{rows}"] = {"us": round(us, 2), "path": m.gemm_path(rows),
                                                       "m5pro_lut_1core_us": m5,
                                                       "weight_GBps": round(weight_bytes(o, i, bits) / us / 1e3, 1)}
        del graph, m, x, y
    res = {"shapes": out}
    res.update(ref_benchmarks(gw, torch, with_cpu))
    if with_cpu:
        from oracle import cpu_legs

        cpu = cpu_legs.shapes_baseline([(n, o, i, b, r) for n, o, i, b, r, _ in REF_SHAPES], cpu_seconds)
        for k, v in cpu.items():
            out[k]["cpu_1t_us"] = v
        res["cpu_baseline"] = {"unit": "us per call", "cores": 1, "kind": "port", "host": cpu_host(),
                               "sample": f"oracle lut GEMM on one thread (AVX2 where the host has it), each "
                                         f"shape repeated for about {cpu_seconds:.2f} s"}
    return res


def _graph_us(torch, fn, calls=20, reps=5):
    """Microseconds per call of fn, from a captured graph of `calls` calls
    replayed `reps` times (inputs cache-resident, as repeated b.Loop calls)."""
    fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (calls * reps)


def _cpu_us(fn, seconds):
    fn()
    done, t0 = 0, time.perf_counter()
    while True:
        fn()
        done += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            return el / done * 1e6


# BenchmarkGEMMs (internal/cq/bench_test.go:92-150): matrices reading one
# input, shared tables (GEMMs) against a GEMM per matrix, with the
# published M5 Pro -cpu 1 times (docs/FINDINGS.md:3244-3251), us.
REF_GEMMS = [("qkvg", 512, 2, (384, 96, 96, 384), {1: (6.47, 8.20), 375: (2430.0, 3040.0)}),
             ("phi", 2048, 4, (4, 4, 16), {1: (7.43, 13.2), 375: (2800.0, 4960.0)})]


def ref_benchmarks(gw, torch, with_cpu, cpu_seconds=0.3):
    """The reference's other benchmarks of this path on the device, each
    next to its published M5 Pro time and the oracle on one host thread:
    BenchmarkGEMMs (shared tables vs a GEMM per matrix, at 1 and 375 rows),
    BenchmarkCrossAttendStep (one decode step's int8 cross-attention, 8 heads
    of qk 48 / vd 64 over 375 frames; internal/needle/int8_bench_test.go:
    35-56; published 23.9 us NEON int8, 55.0 us float32) and
    BenchmarkQuantizeRow (one row of 48, 64 and 2048 values, int8_bench_test.go:
    18-33; published 0.83 ns per value), the latter also over 65536 rows in
    one launch."""
    import numpy as np

    from go_whistle_amd import needle

    orc = None
    if with_cpu:
        if ROOT not in sys.path:
            sys.path.insert(0, ROOT)
        from oracle import binding as orc

        orc.set_cpu(orc.have_avx2(), 1)
    res = {}
    try:
        gem = {}
        for name, inp, bits, outs, pub in REF_GEMMS:
            g = gw.synth.rng(38 + inp)
            packs = [gw.synth.random_packed(g, o, inp, GROUP, bits, sigma=0.05) for o in outs]
            for p in packs[1:]:
                p.Codebook = packs[0].Codebook  # one codebook per width, as in .cact
            ms = [gw.cq.New(p) for p in packs]
            for rows in (1, 375):
                x = torch.from_numpy(gw.synth.activations(g, rows, inp)).cuda()
                ys = [torch.empty(rows, o, device="cuda") for o in outs]
                shared = _graph_us(torch, lambda: gw.cq.gemms_dev(ms, ys, x, rows))

                def separate():
                    for m, y in zip(ms, ys):
                        m.gemm_dev(y, x, rows)

                sep = _graph_us(torch, separate)
                e = {"shared_us": round(shared, 2), "separate_us": round(sep, 2),
                     "m5pro_1core_shared_us": pub[rows][0], "m5pro_1core_separate_us": pub[rows][1]}
                if orc is not None:
                    oms = [orc.OMatrix.new(p) for p in packs]
                    xh = gw.synth.activations(g, rows, inp)
                    e["cpu_1t_shared_us"] = round(_cpu_us(lambda: orc.gemms(oms, xh, rows), cpu_seconds), 2)
                gem[f"{name}_rows{rows}"] = e
        res["gemms"] = gem

        H, qk, vd, frames = 8, 48, 64, 375
        g = gw.synth.rng(34)
        kf = g.standard_normal((frames, H * qk)).astype(np.float32)
        vf = g.standard_normal((frames, H * vd)).astype(np.float32)
        q = g.standard_normal(H * qk).astype(np.float32)
        kq, ks = torch.empty(frames * H * qk, dtype=torch.int8, device="cuda"), torch.empty(frames * H, device="cuda")
        vq, vs = torch.empty(frames * H * vd, dtype=torch.int8, device="cuda"), torch.empty(frames * H, device="cuda")
        kd, vdev, qd = torch.from_numpy(kf).cuda(), torch.from_numpy(vf).cuda(), torch.from_numpy(q).cuda()
        needle.quantize_rows_dev(kq, ks, kd, frames, H * qk, qk)
        needle.quantize_rows_dev(vq, vs, vdev, frames, H * vd, vd)
        spans = torch.tensor([[0, 0, 0, frames]], dtype=torch.int32, device="cuda")
        o = torch.empty(H * vd, device="cuda")
        us = _graph_us(torch, lambda: needle.attend_int8_dev(o, qd, 1, H, kq, ks, H * qk, qk, vq, vs, H * vd, vd,
                                                              spans, frames, np.float32(6.928203), True))
        ca = {"us": round(us, 2), "m5pro_1core_int8_neon_us": 23.9, "m5pro_1core_float32_us": 55.0}
        if orc is not None:
            kq8, ks8 = orc.quantize_rows(kf.reshape(-1), H * qk, qk)
            vq8, vs8 = orc.quantize_rows(vf.reshape(-1), H * vd, vd)
            sp = np.array([[0, 0, 0, frames]], np.int32)
            ca["cpu_1t_us"] = round(_cpu_us(lambda: orc.attend_int8_spans(q, 1, H, kq8, ks8, H * qk, qk, vq8, vs8,
                                                                            H * vd, vd, frames, sp,
                                                                            np.float32(6.928203), True, 1),
                                            cpu_seconds), 2)
        res["cross_attend_step_8x48_375"] = ca

        qr = {}
        for n in (48, 64, 2048):
            x = torch.from_numpy(g.standard_normal(n).astype(np.float32)).cuda()
            q8, sc = torch.empty(n, dtype=torch.int8, device="cuda"), torch.empty(1, device="cuda")
            one = _graph_us(torch, lambda: needle.quantize_rows_dev(q8, sc, x, 1, n, n))
            rows = 65536
            xb = torch.from_numpy(g.standard_normal(rows * n).astype(np.float32) if n < 2048 else
                                  g.standard_normal(rows * n // 16).astype(np.float32)).cuda()
            rb = xb.numel() // n
            qb, sb = torch.empty(xb.numel(), dtype=torch.int8, device="cuda"), torch.empty(rb, device="cuda")
            many = _graph_us(torch, lambda: needle.quantize_rows_dev(qb, sb, xb, rb, n, n), calls=10)
            e = {"one_row_us": round(one, 3), "rows_per_launch": rb,
                 "ns_per_value": round(many * 1e3 / (rb * n), 5), "m5pro_1core_ns_per_value": 0.83}
            if orc is not None:
                xh = g.standard_normal(n).astype(np.float32)
                e["cpu_1t_ns_per_value"] = round(_cpu_us(lambda: orc.quantize_row(xh), cpu_seconds) * 1e3 / n, 3)
            qr[str(n)] = e
        res["quantize_row"] = qr
    finally:
        if orc is not None:
            orc.set_cpu(False, 1)
    return res


def aux_leg(gw, torch, with_cpu, cpu_seconds):
    """The device forms of two float blocks next to the CQ linears, timed
    at Whistle's shapes (a captured graph of 20 calls): HadamardMLP.Forward
    (internal/needle/hadamard.go:172-294; 16 x 32 Monarch blocks, rank 8,
    width 512) and an mHC layer's heads, Sinkhorn and lane mix
    (internal/needle/mhc.go:182-299; 4 lanes of 512), at 1, 375 and 1500
    rows. The cpu_baseline is the oracle on one host thread: the C mHC
    routines and the float64 numpy restatement of HadamardMLP."""
    import numpy as np

    from go_whistle_amd import needle

    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    from oracle import binding as orc
    from oracle import hadamard_ref as hr

    def graph_us(call):
        call()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(20):
                call()
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / 100

    def cpu_us(call):
        call()
        n, t0 = 0, time.perf_counter()
        while True:
            call()
            n += 1
            el = time.perf_counter() - t0
            if el >= cpu_seconds:
                return el / n * 1e6

    g = np.random.default_rng(17)
    w = hr.random_weights(g, 16, 32, 8, 512)
    h = needle.HadamardMLP(w)
    n, dim = 4, 512
    out = {}
    for rows in (1, 375, 1500):
        x = (g.standard_normal((rows, 512)) * 1.5).astype(np.float32)
        xd = torch.from_numpy(x).cuda()
        yd = torch.empty(rows, 512, device="cuda")
        rec = {"us": round(graph_us(lambda: h.forward_dev(yd, xd, rows)), 2)}
        if with_cpu:
            rec["cpu_1t_us"] = round(cpu_us(lambda: hr.forward(w, x, rows)), 1)
        out[f"hadamard_mlp_rows{rows}"] = rec

        pre, post = g.standard_normal((rows, n)).astype(np.float32), g.standard_normal((rows, n)).astype(np.float32)
        res = g.standard_normal((rows, n * n)).astype(np.float32)
        stream = g.standard_normal((rows, n, dim)).astype(np.float32)
        block_out = g.standard_normal((rows, dim)).astype(np.float32)
        t = [torch.from_numpy(a.reshape(-1)).cuda() for a in (pre, post, res, stream, block_out)]
        hp, hq = torch.zeros(rows * n, device="cuda"), torch.zeros(rows * n, device="cuda")
        hres, u = torch.zeros(rows * n * n, device="cuda"), torch.zeros(rows * dim, device="cuda")
        mixed = torch.zeros(rows * n * dim, device="cuda")

        def mhc():
            needle.mhc_heads_dev(hp, hq, hres, u, t[0], t[1], t[2], t[3], rows, n, dim, None)
            needle.mhc_mix_dev(mixed, t[3], hres, hq, t[4], u, rows, n, dim)

        rec = {"us": round(graph_us(mhc), 2)}
        if with_cpu:
            def mhc_cpu():
                _, ohq, ohr, ou = orc.mhc_heads(pre, post, res, stream, rows, n, dim)
                orc.mhc_mix(stream, ohr, ohq, block_out, ou, rows, n, dim)

            rec["cpu_1t_us"] = round(cpu_us(mhc_cpu), 1)
        out[f"mhc_heads_mix_rows{rows}"] = rec
    res = {"cases": out}
    if with_cpu:
        res["cpu_baseline"] = {"unit": "us per call", "cores": 1, "kind": "port", "host": cpu_host(),
                               "sample": "oracle on one thread: C mHC heads/Sinkhorn/mix; HadamardMLP as the "
                                         f"float64 numpy restatement; each case repeated for about {cpu_seconds} s"}
    return res


ATTN_CASES = [("self", 64), ("self", 200), ("self", 448), ("cross", 1500)]


def attention_leg(gw, torch, with_cpu, cpu_seconds):
    """Int8 KV attention (AttendInt8Spans) of one query row per stream, 8
    heads x 64, at batch 1 and 256: self over n keys of an n-key cache and
    cross over 1500 frames, K/V ~N(0,1) quantised per row on the device
    (QuantizeRows), Q ~N(0,1), int8 query. Microseconds per call (a captured
    graph of 20 calls), stream-steps/s and the K/V bytes read (codes and
    scales) per second against 8 TB/s. The cross cases are timed in the
    key-major layout ([stream][frame][8 heads x 64]) and, as _head_major,
    in the decoder's ([stream][head][frame][64])."""
    from go_whistle_amd import needle

    H, D = 8, 64
    C = H * D
    out = {}
    for batch in (1, 256):
        for kind, n in ATTN_CASES:
            gen = torch.Generator(device="cuda")
            gen.manual_seed(11 + n)
            kq = torch.empty(batch * n, C, dtype=torch.int8, device="cuda")
            vq = torch.empty_like(kq)
            ks = torch.empty(batch * n, H, device="cuda")
            vs = torch.empty_like(ks)
            for dq, ds in ((kq, ks), (vq, vs)):
                f32 = torch.randn(batch * n, C, generator=gen, device="cuda")
                needle.quantize_rows_dev(dq, ds, f32, batch * n, C, D)
                del f32
            q = torch.randn(batch, C, generator=gen, device="cuda")
            o = torch.zeros(batch, C, device="cuda")
            span = [0, n, 0, 0] if kind == "self" else [0, 0, 0, n]
            spans = torch.tensor([span] * batch, dtype=torch.int32, device="cuda")

            def call():
                needle.attend_int8_dev(o, q, 1, H, kq, ks, C, D, vq, vs, C, D, spans, n, math.sqrt(D), True,
                                       batch=batch, kv_stride=n * C, s_stride=n * H)

            kv = batch * n * (2 * C + 2 * 4 * H)

            def timed(fn, name):
                fn()
                torch.cuda.synchronize()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    for _ in range(20):
                        fn()
                graph.replay()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(5):
                    graph.replay()
                e1.record()
                torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / 100
                out[name] = {"us": round(us, 2), "stream_steps_per_s": round(batch / us * 1e6, 1),
                             "kv_GBps": round(kv / us / 1e3, 1), "hbm_frac": round(kv / us / 1e3 / HBM_PEAK_GBS, 4)}
                del graph

            timed(call, f"b{batch}_{kind}{n}")
            if kind == "cross":
                # The decoder's layout of the cross memory: head-major, [stream][head][frame][64], one
                # AttendInt8Spans stream per (stream, head) (the same bytes, read as batch * 8 streams).
                spans_hm = torch.tensor([span] * (batch * H), dtype=torch.int32, device="cuda")

                def call_hm():
                    needle.attend_int8_dev(o, q, 1, 1, kq, ks, D, D, vq, vs, D, D, spans_hm, n, math.sqrt(D), True,
                                           batch=batch * H, kv_stride=n * D, s_stride=n)

                timed(call_hm, f"b{batch}_{kind}{n}_head_major")
                del spans_hm
            del kq, vq, ks, vs, q, o, spans
        torch.cuda.empty_cache()
    res = {"cases": out}
    if with_cpu:
        from oracle import cpu_legs

        res["cpu_baseline"] = cpu_legs.attention_baseline(ATTN_CASES, cpu_seconds, cpu_threads())
        res["cpu_baseline"]["host"] = cpu_host()
    return res


def _decode_rate(gw, torch, model, batch, tokens):
    """tokens/s and ms per step of one captured step graph replayed per
    token, from position 0."""
    from go_whistle_amd import decoder as dec

    d = dec.Decoder(model, batch)
    d.set_memory(7, "numpy" if batch == 1 else "device")
    first = list(range(1, batch + 1))
    d.reset(first)
    g = d.capture()
    for _ in range(3):
        g.replay()
    d.reset(first)
    d._reserve(tokens)  # the caches and RoPE tables hold max_pos positions
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(tokens):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    return d, g, {"tokens_per_s": round(batch * tokens / ms * 1e3, 1), "ms_per_step": round(ms / tokens, 4)}


def decode_leg(gw, torch, tokens, cpu_seconds, with_cpu, models=("synthetic", "whistle")):
    """Greedy decode of the synthetic 8-layer decoder (d 512, 8 heads, FFN
    2048, vocab 16384, 1500-frame int8 cross memory per stream), 200 tokens
    at batch 1 and 256: one captured step graph replayed per token. Then
    the same decoder with the reference step's features on (3 taps, q/k
    norms, post norms and residual factors, 4 mHC lanes; the paged step),
    and the cost of its fork at two positions (independent of the
    position: full pages are shared)."""
    from go_whistle_amd import decoder as dec

    cfg = dec.DecoderConfig()
    model = dec.make_model(7, cfg)
    res = {"model": "synthetic Whistle-shaped decoder: 8 layers, d 512, 8x64 heads, FFN 2048 (CQ2), attention "
                    "CQ4 (self q/k/v/gate/o, cross q/gate/o: sigmoid output gates), tied CQ4 head 16384x512, int8 "
                    "self/cross KV; cross memory: 1500 random encoder states through CQ4 K/V projections",
           "tokens": tokens}
    for batch in (1, 256) if "synthetic" in models else ():
        d, g, res[f"batch{batch}"] = _decode_rate(gw, torch, model, batch, tokens)
        del d, g
        torch.cuda.empty_cache()
    wcfg = dec.DecoderConfig.whistle()
    if "whistle" not in models:
        if with_cpu:
            if ROOT not in sys.path:
                sys.path.insert(0, ROOT)
            from oracle import cpu_legs

            base = cpu_legs.decode_baseline(tokens, cpu_threads(), cpu_threads())
            res["cpu_baseline"] = dict(base["batch1"], host=cpu_host())
            res["cpu_baseline_batch256"] = dict(base["batch256"], host=cpu_host())
        return res
    wmodel = dec.make_model(7, wcfg)
    wres = {"model": "the same decoder with the reference step's features: causal taps (3) on q/k/v, per-head "
                     "q/k ZCRMSNorm before RoPE, the attention's post norm and residual factor, the cross q/k "
                     "norms, post norm and residual factor, 4 mHC lanes (RMSUnit, CQ4 phi products on int8 "
                     "input, Sinkhorn heads, lane mix) around every layer; paged self caches"}
    for batch in (1, 256):
        d, g, wres[f"batch{batch}"] = _decode_rate(gw, torch, wmodel, batch, tokens)
        if batch == 256:  # fork cost at two positions (random parents, as a beam step reorders)
            rng = __import__("numpy").random.default_rng(3)
            fk = {}
            d.fork(list(rng.integers(0, batch, size=batch)))  # untimed: its first call allocates its buffers
            for at in (40, 200):
                d.reset(list(range(1, batch + 1)))
                for _ in range(at):
                    g.replay()
                d.steps = at
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                d.fork(list(rng.integers(0, batch, size=batch)))
                torch.cuda.synchronize()
                fk[f"pos{at}"] = {"ms": round((time.perf_counter() - t0) * 1e3, 3), "page_copies": d.fork_copies}
            wres["fork_batch256"] = fk
        del d, g
        torch.cuda.empty_cache()
    res["whistle_step"] = wres
    if with_cpu:
        if ROOT not in sys.path:
            sys.path.insert(0, ROOT)
        from oracle import cpu_legs

        if "synthetic" in models:
            base = cpu_legs.decode_baseline(tokens, cpu_threads(), cpu_threads())
            res["cpu_baseline"] = dict(base["batch1"], host=cpu_host())
            res["cpu_baseline_batch256"] = dict(base["batch256"], host=cpu_host())
        wb = cpu_legs.decode_baseline(tokens, cpu_threads(), cpu_threads(), cfg=wcfg)
        wres["cpu_baseline"] = dict(wb["batch1"], host=cpu_host())
        wres["cpu_baseline_batch256"] = dict(wb["batch256"], host=cpu_host())
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # The GPU's clocks settle over the first ~10 ms of sustained load (the
    # sweep's launches run ~15% slower before that), so the default warm-up
    # is ~50 ms of steps.
    ap.add_argument("--warmup", type=int, default=400)
    ap.add_argument("--copies", type=int, default=0, help="device copies of the sweep (0: > 2x MALL)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-tokens", type=int, default=200)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--decode-model", choices=("both", "synthetic", "whistle"), default="both",
                    help="the decode leg's decoders: the synthetic one, the one with the reference step's features")
    ap.add_argument("--no-gemm", action="store_true", help="skip the batched GEMM leg")
    ap.add_argument("--gemm-only", action="store_true", help="run only the batched GEMM leg (prints its JSON)")
    ap.add_argument("--decode-only", action="store_true", help="run only the decode leg (prints its JSON)")
    ap.add_argument("--no-attention", action="store_true", help="skip the int8 attention leg")
    ap.add_argument("--no-aux", action="store_true", help="skip the HadamardMLP / mHC leg")
    ap.add_argument("--aux-only", action="store_true", help="run only the HadamardMLP / mHC leg")
    ap.add_argument("--no-ref-shapes", action="store_true", help="skip the reference's benchmark shapes")
    ap.add_argument("--attention-only", action="store_true", help="run only the attention leg (prints its JSON)")
    ap.add_argument("--roofline-only", action="store_true",
                    help="run only the roofline leg's launches (4 of 4 bits, 1 of 2 bits, per step) after 50 ms of "
                         "512 MiB device copies, then 4 more copies (for rocprofv3 traces and counters)")
    args = ap.parse_args()
    if not 0 <= args.decode_tokens <= 256:
        # the synthetic decoder's caches and RoPE tables hold 256 positions
        print(json.dumps({"error": f"--decode-tokens {args.decode_tokens} outside 0..256 (the decoder's max_pos)"}))
        sys.exit(2)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus above 1 is not supported"}))
        sys.exit(2)

    import numpy as np
    import torch

    gw = _package()
    torch.cuda.set_device(0)
    dev = torch.device("cuda:0")
    if args.gemm_only:
        leg = batched_gemm_leg(gw, torch)
        if not args.no_cpu:
            leg["cpu_baseline"] = batched_gemm_cpu(0.5)
        print(json.dumps({"batched_gemm": leg}))
        return
    if args.aux_only:
        print(json.dumps({"aux": aux_leg(gw, torch, not args.no_cpu, 0.3)}))
        return
    if args.attention_only:
        print(json.dumps({"attention": attention_leg(gw, torch, not args.no_cpu, 1.0)}))
        return
    if args.decode_only:
        models = ("synthetic", "whistle") if args.decode_model == "both" else (args.decode_model,)
        print(json.dumps({"decode": decode_leg(gw, torch, args.decode_tokens, args.cpu_seconds, not args.no_cpu,
                                               models)}))
        return

    g = gw.synth.rng(20261201)
    packs = [gw.synth.random_packed(g, o, i, GROUP, b, sigma=0.05) for b in BITS for (o, i) in SHAPES]
    sweep_bytes = sum(weight_bytes(p.Out, p.In, p.Bits) for p in packs)
    copies = args.copies or max(1, math.ceil(2 * 256 * 2 ** 20 / sweep_bytes))
    mats = [[gw.cq.New(p) for p in packs] for _ in range(copies)]
    xs = {i: torch.from_numpy(gw.synth.activations(g, 1, i)).to(dev) for i in {p.In for p in packs}}
    ys = [[torch.zeros(p.Out, dtype=torch.float32, device=dev) for p in packs] for _ in range(copies)]

    def timed(fn, reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps  # ms

    by_bits = {b: [(c, k) for c in range(copies) for k, p in enumerate(packs) if p.Bits == b] for b in BITS}
    plans = {b: gw.cq.Batch([mats[c][k] for c, k in jobs], [ys[c][k] for c, k in jobs],
                            [xs[packs[k].In] for c, k in jobs]) for b, jobs in by_bits.items()}

    def step():
        for b in BITS:
            plans[b].run()

    if args.roofline_only:
        src = torch.empty(128 * 2 ** 20, dtype=torch.float32, device=dev).uniform_()
        dst = torch.empty_like(src)
        # ~50 ms of copies first, so that the clocks have settled before the
        # first lut launch (a profiler's average then covers steady launches)
        for _ in range(250):
            dst.copy_(src)
        for _ in range(args.steps):  # the launches the roofline leg times: 4 of 4 bits, then one of 2
            for _ in range(ROOF_REPS):
                plans[4].run()
            plans[2].run()
        for _ in range(4):
            dst.copy_(src)  # calibration: 512 MiB read, 512 MiB written
        torch.cuda.synchronize()
        print(json.dumps({"roofline_only": True, "launches_4bit": args.steps * ROOF_REPS, "copy_bytes": src.numel() * 4,
                          "algorithmic_bytes_4bit_launch": sum(algorithmic_bytes(packs[k].Out, packs[k].In, 4)
                                                               for c, k in by_bits[4])}))
        return

    for _ in range(args.warmup):
        step()
    prewarm_ms = prewarm(torch, step)
    ms = timed(step, args.steps)
    value = sweep_bytes * copies / (ms / 1e3) / 1e9

    # Roofline: the step's 4-bit launch, HIP events on the plans' stream
    # around ROOF_REPS back-to-back launches inside each step (the copies
    # exceed the MALL, so repeats stream from HBM too).
    def roof_step():
        for _ in range(ROOF_REPS):
            plans[4].run()
        plans[2].run()

    roof_prewarm_ms = prewarm(torch, roof_step)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    for e0, e1 in ev:
        e0.record()
        for _ in range(ROOF_REPS):
            plans[4].run()
        e1.record()
        plans[2].run()
    torch.cuda.synchronize()
    dur_s = sum(e0.elapsed_time(e1) for e0, e1 in ev) / len(ev) / ROOF_REPS / 1e3
    alg = sum(algorithmic_bytes(packs[k].Out, packs[k].In, 4) for c, k in by_bits[4])
    achieved = alg / dur_s / 1e9
    traffic = pmc_traffic()

    # One launch per GEMV: a captured graph of the whole sweep.
    def per_launch():
        for c in range(copies):
            for k, p in enumerate(packs):
                mats[c][k].gemm_dev(ys[c][k], xs[p.In], 1)

    per_launch()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        per_launch()
    graph.replay()
    ms_launch = timed(graph.replay, max(2, args.steps // 4))

    detail = {"one_launch_per_gemv": {"ms_per_step": round(ms_launch, 4),
                                      "weight_GBps": round(sweep_bytes * copies / ms_launch / 1e6, 1)}}
    for k, p in enumerate(packs):
        plan = gw.cq.Batch([mats[c][k] for c in range(copies)], [ys[c][k] for c in range(copies)],
                           [xs[p.In]] * copies)
        plan.run()
        msk = timed(plan.run, max(2, args.steps // 2))
        wb = weight_bytes(p.Out, p.In, p.Bits)
        detail[f"{p.Out}x{p.In}_cq{p.Bits}"] = {"us_per_gemv": round(msk * 1e3 / copies, 3),
                                                 "weight_GBps": round(wb * copies / msk / 1e6, 1)}

    # Config 1 on its own: the single 4-bit 2048x512 GEMV, one launch per
    # GEMV (cq_gemm_dev), 64 launches per captured graph: cold, a different
    # device copy each launch (weights from HBM), and warm, the same copy
    # every launch (weights in the caches, as the reference's repeated
    # BenchmarkGEMM calls have them).
    k1 = next(k for k, p in enumerate(packs) if (p.Out, p.In, p.Bits) == (2048, 512, 4))
    one = {}
    for kind, cs in (("cold", list(range(copies))), ("warm", [0] * copies)):
        def launches(cs=cs):
            for c in cs:
                mats[c][k1].gemm_dev(ys[c][k1], xs[512], 1)

        launches()
        torch.cuda.synchronize()
        g1 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g1):
            launches()
        prewarm(torch, g1.replay, 20.0)
        msg = timed(g1.replay, 10)
        us = msg * 1e3 / len(cs)
        wb1 = weight_bytes(2048, 512, 4)
        one[kind] = {"us_per_gemv": round(us, 3), "gemv_per_s": round(1e6 / us, 1),
                     "weight_GBps": round(wb1 / us / 1e3, 1)}
        del g1
    detail["config1_2048x512_cq4_one_launch"] = one

    line = {
        "metric": "CQ LUT GEMV HBM GB/s (% of peak) + decode tokens/sec, batch 1 and 256",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "prewarm_ms": round(prewarm_ms, 1),
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic",
        "config": {"workload": "batch-1 CQ LUT GEMV sweep, 2/4-bit x {512x512, 2048x512, 512x2048, 16384x512}, "
                               "group 128",
                   "copies": copies, "gemvs_per_step": copies * len(packs),
                   "weight_bytes_per_step": sweep_bytes * copies, "hbm_frac": round(value / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "lut_kernel<4,64,dev>: the step's 4-bit batch launch",
                     "launch_us": round(dur_s * 1e6, 3), "algorithmic_bytes": alg,
                     "prewarm_ms": round(roof_prewarm_ms, 1)},
        "detail": detail,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(gw, packs, args.cpu_seconds)
    if not args.no_gemm:
        line["batched_gemm"] = batched_gemm_leg(gw, torch)
        if not args.no_cpu:
            line["batched_gemm"]["cpu_baseline"] = batched_gemm_cpu(0.5)
    if not args.no_ref_shapes:
        line["ref_shapes"] = ref_shapes_leg(gw, torch, not args.no_cpu, 0.25)
    if not args.no_attention:
        line["attention"] = attention_leg(gw, torch, not args.no_cpu, 1.0)
    if not args.no_aux:
        line["aux"] = aux_leg(gw, torch, not args.no_cpu, 0.3)
    if not args.no_decode:
        del plans, mats
        torch.cuda.empty_cache()
        line["decode"] = decode_leg(gw, torch, args.decode_tokens, args.cpu_seconds, not args.no_cpu)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
