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
kernel (oracle/), one thread, on a bounded sample of the same sweep.
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


def batched_gemm_leg(gw, torch, reps=5):
    """The encoder's batched CQ GEMMs: X [M x In] ~N(0, 1) times 4/2-bit
    2048x512 and 512x2048 (FFN up/down), M in {375, 1500, 12000}, through
    cq_gemm_dev (which picks the lut kernel or its MFMA form). Flops are the
    dense equivalent 2*M*Out*In; for the MFMA form, mfma_util is the int8 MFMA
    work it issues (one 32x32x32 product per 64-row block, 64-activation tile,
    position and 32x32 quadrant) over the time, against 5.0 POP/s."""
    g = gw.synth.rng(31)
    out = {}
    for bits in (4, 2):
        for (o, i) in ((2048, 512), (512, 2048)):
            m = gw.cq.New(gw.synth.random_packed(g, o, i, GROUP, bits, sigma=0.05))
            for M in (375, 1500, 12000):
                x = torch.randn(M, i, device="cuda")
                y = torch.empty(M, o, device="cuda")
                m.gemm_dev(y, x, M)
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(reps):
                    m.gemm_dev(y, x, M)
                e1.record()
                torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / reps
                path = m.gemm_path(M)
                rec = {"path": path, "us": round(us, 2), "dense_TFLOPs": round(2.0 * M * o * i / us / 1e6, 2)}
                if path in ("lut-mfma", "lut-mfma-split"):
                    # one 32x32x32 int8 product per 32 weight rows, 32 activations and table position
                    # (the 512-row form pads activations to its 64-wide tiles, the split form to 32)
                    positions = (i // GROUP) * (2 * GROUP * bits // 8)
                    tile = 64 if path == "lut-mfma" else 32
                    mfmas = -(-o // 64) * 2 * (-(-M // tile) * tile // 32) * positions
                    ops = mfmas * 2 * 32 * 32 * 32
                    rec["mfma_TOPs"] = round(ops / us / 1e6, 1)
                    rec["mfma_util"] = round(ops / (us * 1e-6) / INT8_PEAK_OPS, 4)
                out[f"cq{bits}_{o}x{i}_M{M}"] = rec
                del x, y
    return out


def decode_leg(gw, torch, tokens, cpu_seconds, with_cpu):
    """Greedy decode of the synthetic 8-layer decoder (d 512, 8 heads, FFN
    2048, vocab 16384, 1500-frame int8 cross memory per stream), 200 tokens
    at batch 1 and 256: one captured step graph replayed per token."""
    from go_whistle_amd import decoder as dec

    cfg = dec.DecoderConfig()
    model = dec.make_model(7, cfg)
    res = {"model": "synthetic Whistle-shaped decoder: 8 layers, d 512, 8x64 heads, FFN 2048 (CQ2), attention "
                    "CQ4 (self q/k/v/gate/o, cross q/gate/o: sigmoid output gates), tied CQ4 head 16384x512, int8 "
                    "self/cross KV; cross memory: 1500 random encoder states through CQ4 K/V projections",
           "tokens": tokens}
    for batch in (1, 256):
        d = dec.Decoder(model, batch)
        d.set_memory(7, "numpy" if batch == 1 else "device")
        first = list(range(1, batch + 1))
        d.reset(first)
        g = d.capture()
        for _ in range(3):
            g.replay()
        d.reset(first)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(tokens):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1)
        res[f"batch{batch}"] = {"tokens_per_s": round(batch * tokens / ms * 1e3, 1),
                                "ms_per_step": round(ms / tokens, 4)}
        del d, g
        torch.cuda.empty_cache()
    if with_cpu:
        if ROOT not in sys.path:
            sys.path.insert(0, ROOT)
        from oracle import decoder_ref

        from oracle import binding as orc

        ref = decoder_ref.RefDecoder(model)
        avx2, threads = orc.have_avx2(), cpu_threads()
        orc.set_cpu(avx2, threads)
        ref.memory(dec.encoder_states(7, cfg, 0))  # untimed: the memory is built once per clip
        n, t0 = 0, time.perf_counter()
        while True:
            n += len(ref.decode(1, 10))
            el = time.perf_counter() - t0
            if el >= cpu_seconds:
                break
        orc.set_cpu(False, 1)
        res["cpu_baseline"] = {"value": round(n / el, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
                               "host": cpu_host(),
                               "sample": f"{n} greedy tokens at batch 1 (runs of 10 from position 0), oracle "
                                         f"decoder, lut products and int8 attention {'AVX2' if avx2 else 'generic'}, products split over "
                                         f"{threads} threads as the reference splits them, {el:.1f} s"}
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--copies", type=int, default=0, help="device copies of the sweep (0: > 2x MALL)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-tokens", type=int, default=200)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-gemm", action="store_true", help="skip the batched GEMM leg")
    ap.add_argument("--gemm-only", action="store_true", help="run only the batched GEMM leg (prints its JSON)")
    ap.add_argument("--decode-only", action="store_true", help="run only the decode leg (prints its JSON)")
    ap.add_argument("--roofline-only", action="store_true",
                    help="run only the step's 4-bit launch and a 512 MiB device copy (for rocprofv3 counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus above 1 is not supported"}))
        sys.exit(2)

    import numpy as np
    import torch

    gw = _package()
    torch.cuda.set_device(0)
    dev = torch.device("cuda:0")
    if args.gemm_only:
        print(json.dumps({"batched_gemm": batched_gemm_leg(gw, torch)}))
        return
    if args.decode_only:
        print(json.dumps({"decode": decode_leg(gw, torch, args.decode_tokens, args.cpu_seconds, not args.no_cpu)}))
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
        for _ in range(args.steps):
            plans[4].run()
            plans[2].run()
            dst.copy_(src)  # calibration: 512 MiB read, 512 MiB written
        torch.cuda.synchronize()
        print(json.dumps({"roofline_only": True, "launches": args.steps, "copy_bytes": src.numel() * 4,
                          "algorithmic_bytes_4bit_launch": sum(algorithmic_bytes(packs[k].Out, packs[k].In, 4)
                                                               for c, k in by_bits[4])}))
        return

    for _ in range(args.warmup):
        step()
    ms = timed(step, args.steps)
    value = sweep_bytes * copies / (ms / 1e3) / 1e9

    # Roofline: the step's 4-bit launch, HIP events on the plans' stream
    # around ROOF_REPS back-to-back launches inside each step (the copies
    # exceed the MALL, so repeats stream from HBM too).
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

    line = {
        "metric": "CQ LUT GEMV HBM GB/s (% of peak) + decode tokens/sec, batch 1 and 256",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
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
                     "launch_us": round(dur_s * 1e6, 3), "algorithmic_bytes": alg},
        "detail": detail,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(gw, packs, args.cpu_seconds)
    if not args.no_gemm:
        line["batched_gemm"] = batched_gemm_leg(gw, torch)
    if not args.no_decode:
        del plans, mats
        torch.cuda.empty_cache()
        line["decode"] = decode_leg(gw, torch, args.decode_tokens, args.cpu_seconds, not args.no_cpu)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
