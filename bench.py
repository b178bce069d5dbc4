#!/usr/bin/env python3
"""Benchmark of the phobos leaf kernels on one MI355X.

A "step" is one pass of the phobos-bench suite at the BASELINE configs:
saxpy_fp32 (n = 4096^2), gemm_fp32, gemm_fp16tc_fp32acc and gemm_fp16
(4096^3), flash_fp32 and flash_fp16 (B4 x H16 x 4096 x 4096 x D64), each
launched REPS[kernel] times back to back through libphobos_hip on one
stream, inputs resident in HBM.

Each kernel's run of launches is bracketed by HIP events on that stream, so
its average launch duration (run time / launches, dispatch gaps included)
is measured live; a run of several launches keeps the few microseconds of
event and dispatch overhead from dominating the 30-microsecond saxpy.  `value` is the headline metric's first
figure: gemm_fp16tc_fp32acc TFLOP/s (FLOP formula 2MNK + MN, main.rs:591); the
other kernels' figures are reported under "kernels".  saxpy rotates over four
input sets (512 MiB) so that it streams from HBM, not the 256 MB MALL.

Prints one JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "phobos-lang_amd"))

# MI355X published peaks (dense): HBM3E 8 TB/s; fp16 MFMA 2516.6 TFLOP/s;
# fp32 matrix 157.3 TFLOP/s.
PEAK_HBM_GBS = 8000.0
PEAK_FP16_TFLOPS = 2516.6
PEAK_FP32_TFLOPS = 157.3

GEMM_FLOP = 2 * 4096 ** 3 + 4096 ** 2          # main.rs:591
FLASH_FLOP = 4 * 4096 * 4096 * 64 * 64         # main.rs:1032, x 64 heads
FLASH_EXPS = 4096 * 4096 * 64                  # one exp per score (secondary bound)
SAXPY_BYTES = 12 * 4096 * 4096                 # read x, read y, write y
# back-to-back launches per kernel per step, between two HIP events: enough
# that the few microseconds an event pair adds stay small against the run
# (saxpy's launch is 32 us, so it runs 32 times)
REPS = {"saxpy_fp32": 32, "gemm_fp32": 2, "gemm_fp16tc_fp32acc": 2, "gemm_fp16": 2,
        "flash_fp32": 2, "flash_fp16": 2}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--kernels", default="all",
                    help="comma list of saxpy_fp32,gemm_fp32,gemm_fp16tc_fp32acc,gemm_fp16,"
                         "flash_fp32,flash_fp16")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--no-cluster", action="store_true",
                    help="skip the one-pod matmul_cluster job (16384^3 f32 from 3 GiB of files)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--csv", nargs="?", const="phobos-bench.csv", default=None, metavar="PATH",
                    help="also write the reference's results CSV (benchmark,impl,precision,gflops,"
                         "peak_gflops,pct_of_peak; default path phobos-bench.csv)")
    ap.add_argument("--peak-fp32", type=float, default=None, metavar="TFLOPS",
                    help="override the f32 peak of the CSV (default: MI355X 157.3)")
    ap.add_argument("--peak-fp16tc", type=float, default=None, metavar="TFLOPS",
                    help="override the f16 matrix peak of the CSV (default: MI355X 2516.6)")
    ap.add_argument("--peak-fp16tcf32acc", type=float, default=None, metavar="TFLOPS",
                    help="override the f16/f32-accumulate matrix peak of the CSV (default 2516.6)")
    ap.add_argument("--vendor", action="store_true",
                    help="add the vendor-library rows of the CSV (the reference's cuBLAS rows): "
                         "saxpy, sgemm and hgemm through torch on ROCm")
    ap.add_argument("--vendor-only", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--hold", type=float, default=0.0,
                    help="only launch the --kernels back to back for this many seconds and print "
                         "the launch count (a steady load for reading power and clocks with amd-smi)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 3 device-to-device copies of 256 MiB (the plain copy the "
                         "FETCH_SIZE/WRITE_SIZE counters are scaled by) and exit")
    ap.add_argument("--bench", default=None, metavar="NAME",
                    help="run only one benchmark, as phobos-bench --bench NAME: one of "
                         + ", ".join(BENCHES))
    ap.add_argument("--autotune", default=None, metavar="SPEC",
                    help="pin the launch plan instead of searching it, as phobos-bench's "
                         "--autotune pins its tile dims (needs --bench): \"splits=N variant=V\", for "
                         "gemm_fp32 also \"TILE_M=128 TILE_N=128 TILE_K=16\"")
    ap.add_argument("--pin", action="append", default=[], metavar="NAME=SPLITS,VARIANT",
                    help="pin one benchmark's launch plan instead of searching it (repeatable), "
                         "e.g. gemm_fp32=1,1: a profiling pass then runs the plans an earlier "
                         "run's search picked")
    ap.add_argument("--no-autotune", action="store_true",
                    help="skip the launch-plan search and use the runtime's built-in plans")
    ap.add_argument("--shapes", action="store_true",
                    help="only time the non-BASELINE shapes that run split (GEMMs at 512^3 and "
                         "1024^3, one-head flash at 4096 queries, through the .ph entries) and exit")
    args = ap.parse_args()
    if args.bench is not None:
        # phobos-bench/src/main.rs:62-67, 109-115: one name from the list
        if args.bench not in BENCHES:
            ap.error(f"unknown --bench '{args.bench}'; available: {', '.join(BENCHES)}")
        args.kernels = args.bench
    args.fixed = {}
    for tok in args.pin:
        name, eq, val = tok.partition("=")
        parts = val.split(",")
        if name not in BENCHES or name == "saxpy_fp32" or not eq or len(parts) != 2 or \
                not all(p.strip().isdigit() for p in parts):
            ap.error(f"bad --pin '{tok}', expected NAME=SPLITS,VARIANT for a kernel with plans")
        args.fixed[name] = (int(parts[0]), int(parts[1]))
    args.pins = {}
    if args.autotune is not None:
        # phobos-bench/src/main.rs:68-72, 118-119, 149-160: NAME=VALUE pins, one benchmark
        if args.bench is None:
            ap.error("--autotune pins are kernel-specific; pass --bench to pick one")
        for tok in args.autotune.replace(",", " ").split():
            name, eq, val = tok.partition("=")
            if not eq:
                ap.error(f"bad autotune pin '{tok}', expected NAME=VALUE")
            dims = ("splits", "variant") + (("TILE_M", "TILE_N", "TILE_K")
                                            if args.bench == "gemm_fp32" else ())
            if name not in dims:
                # autotune.rs:42-51
                ap.error(f"autotune pin '{name}' is not a search dim of this kernel "
                         f"(dims: {', '.join(dims)})")
            try:
                args.pins[name] = int(val)
            except ValueError:
                ap.error(f"autotune pin '{name}' has a non-integer value '{val}'")
    return args


# phobos-bench's benchmark names (phobos-bench/src/main.rs:26-33)
BENCHES = ["saxpy_fp32", "gemm_fp32", "gemm_fp16tc_fp32acc", "gemm_fp16", "flash_fp32", "flash_fp16"]


class Kernel:
    def __init__(self, name, launch, work, unit, bound, peak):
        self.name, self.launch, self.work, self.unit = name, launch, work, unit
        self.bound, self.peak = bound, peak
        self.times = []


def _need(buf, nbytes, what):
    """Host-side check that a device buffer holds what the kernel will touch."""
    if buf.nbytes < nbytes:
        raise RuntimeError(f"{what}: buffer of {buf.nbytes} B < {nbytes} B the kernel accesses")


def setup(px, stream, wanted):
    """Allocates and fills the BASELINE-config inputs on the device.  Every
    launch closure binds its own buffers (no late-bound names) and the sizes
    are checked against what the kernel reads and writes."""
    ks = []
    N = 4096

    def gemm_kernel(name, kid, a, b, c, esz, alpha, beta, peak):
        for buf, what in ((a, "A"), (b, "B"), (c, "C")):
            _need(buf, N * N * esz, f"{name} {what}")

        def launch():
            px.launch_gemm(stream, kid, a, b, c, N, N, N, alpha, beta)
        k = Kernel(name, launch, GEMM_FLOP / 1e12, "TFLOP/s", "mfma", peak)
        k.keep = (a, b, c)
        return k

    if "saxpy_fp32" in wanted:
        n = N * N
        sets = []
        for r in range(4):
            x = px.DeviceBuffer.from_array(px.lcg_f32(1 + 10 * r, n))
            y = px.DeviceBuffer.from_array(px.lcg_f32(2 + 10 * r, n))
            _need(x, 4 * n, "saxpy x")
            _need(y, 4 * n, "saxpy y")
            sets.append((x, y))

        def saxpy(sets=sets, state={"i": 0}):
            x, y = sets[state["i"] % 4]
            state["i"] += 1
            px.launch_saxpy(stream, x, y, y, n, 2.5)
        k = Kernel("saxpy_fp32", saxpy, SAXPY_BYTES / 1e9, "GB/s", "hbm", PEAK_HBM_GBS)
        k.keep = sets
        ks.append(k)
    if "gemm_fp32" in wanted:
        ks.append(gemm_kernel("gemm_fp32", px.GEMM_FP32,
                              px.DeviceBuffer.from_array(px.lcg_f32(1, N * N)),
                              px.DeviceBuffer.from_array(px.lcg_f32(2, N * N)),
                              px.DeviceBuffer.from_array(px.lcg_f32(3, N * N)),
                              4, 0.125, 1.5, PEAK_FP32_TFLOPS))
    if "gemm_fp16tc_fp32acc" in wanted or "gemm_fp16" in wanted:
        a32 = px.from_f16_bits(px.to_f16_bits(px.normal_f32(1, N * N, 1 / 64.0)))
        b32 = px.from_f16_bits(px.to_f16_bits(px.normal_f32(2, N * N, 1 / 64.0)))
    if "gemm_fp16tc_fp32acc" in wanted:
        c = px.DeviceBuffer(N * N * 4)
        c.zero(stream)
        ks.append(gemm_kernel("gemm_fp16tc_fp32acc", px.GEMM_FP16TC_FP32ACC,
                              px.DeviceBuffer.from_array(a32), px.DeviceBuffer.from_array(b32),
                              c, 4, 1.0, 0.0, PEAK_FP16_TFLOPS))
    if "gemm_fp16" in wanted:
        c = px.DeviceBuffer(N * N * 2)
        c.zero(stream)
        ks.append(gemm_kernel("gemm_fp16", px.GEMM_FP16,
                              px.DeviceBuffer.from_array(px.to_f16_bits(a32)),
                              px.DeviceBuffer.from_array(px.to_f16_bits(b32)),
                              c, 2, 1.0, 0.0, PEAK_FP16_TFLOPS))
    BH, S, D = 64, 4096, 64
    for name, kid, peak, esz in (("flash_fp32", px.FLASH_FP32_BH, PEAK_FP32_TFLOPS, 4),
                                 ("flash_fp16", px.FLASH_FP16_BH, PEAK_FP16_TFLOPS, 2)):
        if name not in wanted:
            continue
        ts = [px.normal_f32(s, BH * S * D) for s in (1, 2, 3)]
        if esz == 2:
            ts = [px.to_f16_bits(t) for t in ts]
        q, k, v = (px.DeviceBuffer.from_array(t) for t in ts)
        o = px.DeviceBuffer(BH * S * D * esz)
        for buf, what in ((q, "Q"), (k, "K"), (v, "V"), (o, "O")):
            _need(buf, BH * S * D * esz, f"{name} {what}")

        def fl(q=q, k=k, v=v, o=o, kid=kid):
            px.launch_flash_bh(stream, kid, q, k, v, o, BH, S, S, D, 0.125)
        kk = Kernel(name, fl, FLASH_FLOP / 1e12, "TFLOP/s", "mfma", peak)
        kk.keep = (q, k, v, o)
        ks.append(kk)
    px.synchronize()
    return ks


# Split launches keep their partial results in the workspace bound to their
# stream (the launches never allocate): a buffer this host allocates once,
# enough for 16 chunks of a 4096 x 4096 f32 output or of the 64-head flash
# state.  The autotuner binds a larger one if its search needs it.
WORKSPACE_BYTES = 2 << 30


def shapes_leg(px, stream, reps=20, tune=True):
    """Time the shapes that run split (phx_split_plan): each GEMM at 512^3 and
    1024^3, and the one-head flash .ph entry (main.rs:334-371) at 4096 x 4096.
    Inputs as in the BASELINE configs, average of `reps` launches after 3,
    under the built-in plan; with tune, also the autotuner's winner and its
    fastest launch (the pin is removed again afterwards)."""
    from phobos_amd import autotune
    out = []

    def tuned(kid, dims, fn):
        if not tune:
            return None
        r = fn()
        px.plan_pin(kid, dims, None)
        return {"plan": list(r["winner"]), "us": round(r["us"], 2)}

    ev0, ev1 = px.Event(), px.Event()

    def timed(fn):
        for _ in range(3):
            fn()
        ev0.record(stream)
        for _ in range(reps):
            fn()
        ev1.record(stream)
        ev1.synchronize()
        return ev0.elapsed_ms(ev1) / reps

    for name, kid, esz in (("gemm_fp32", px.GEMM_FP32, 4),
                           ("gemm_fp16tc_fp32acc", px.GEMM_FP16TC_FP32ACC, 4),
                           ("gemm_fp16", px.GEMM_FP16, 2)):
        for n in (512, 1024):
            a = px.normal_f32(1, n * n, 1 / np.sqrt(n))
            b = px.normal_f32(2, n * n, 1 / np.sqrt(n))
            if esz == 2:
                a, b = px.to_f16_bits(a), px.to_f16_bits(b)
            da, db = px.DeviceBuffer.from_array(a), px.DeviceBuffer.from_array(b)
            dc = px.DeviceBuffer(n * n * esz)
            dc.zero(stream)
            ms = timed(lambda: px.launch_gemm(stream, kid, da, db, dc, n, n, n, 1.0, 0.0))
            sp, ws = px.split_plan(kid, [n, n, n])
            out.append({"kernel": name, "shape": [n, n, n], "splits": sp, "workspace_bytes": ws,
                        "us": round(ms * 1e3, 2),
                        "tflops": round((2 * n ** 3 + n * n) / (ms / 1e3) / 1e12, 2),
                        "autotuned": tuned(kid, [n, n, n],
                                           lambda: autotune.tune_gemm(stream, kid, n, n, n))})
    S, D = 4096, 64
    for name, kid, esz in (("flash_fp32", px.FLASH_FP32, 4), ("flash_fp16", px.FLASH_FP16, 2)):
        ts = [px.normal_f32(sd, S * D) for sd in (1, 2, 3)]
        if esz == 2:
            ts = [px.to_f16_bits(t) for t in ts]
        q, k, v = (px.DeviceBuffer.from_array(t) for t in ts)
        o = px.DeviceBuffer(S * D * esz)
        ms = timed(lambda: px.launch_flash(stream, kid, q, k, v, o, S, S, D, 0.125))
        sp, ws = px.split_plan(kid, [S, S, D])
        out.append({"kernel": name + " (one head)", "shape": [S, S, D], "splits": sp,
                    "workspace_bytes": ws, "us": round(ms * 1e3, 2),
                    "tflops": round(4 * S * S * D / (ms / 1e3) / 1e12, 2),
                    "autotuned": tuned(kid, [S, S, D],
                                       lambda: autotune.tune_flash(stream, kid, 1, S, S))})
    return out


def hbm_ceiling_leg(px, sets=4, nbytes=256 << 20, reps=3):
    """The box's practical HBM ceiling next to saxpy's figure: hipMemcpy
    device-to-device (phx_memcpy_d2d) of 256 MiB, rotating over `sets`
    source/destination pairs (1 GiB each way, past the 256 MB MALL), timed
    with HIP events on the legacy stream; bytes read + written per second."""
    bufs = [(px.DeviceBuffer(nbytes), px.DeviceBuffer(nbytes)) for _ in range(sets)]
    for src, dst in bufs:  # first touch
        px.check(px.lib().phx_memcpy_d2d(dst.ptr, src.ptr, nbytes))
    px.synchronize()
    e0, e1 = px.Event(), px.Event()
    best = None
    for _ in range(reps):
        e0.record(None)
        for src, dst in bufs:
            px.check(px.lib().phx_memcpy_d2d(dst.ptr, src.ptr, nbytes))
        e1.record(None)
        e1.synchronize()
        ms = e0.elapsed_ms(e1)
        best = ms if best is None else min(best, ms)
    for src, dst in bufs:
        src.free()
        dst.free()
    return {"what": "hipMemcpy device-to-device, 256 MiB x %d sets" % sets,
            "value": round(2 * nbytes * sets / (best / 1e3) / 1e9, 1), "unit": "GB/s"}


def autotune_leg(px, stream, wanted, pins, fixed=None):
    """The launch-plan search of every benchmark kernel at its BASELINE
    shape and arguments, before the timed steps, as phobos-bench tunes each
    benchmark before it times it (main.rs:461-530); the winners stay pinned
    for the timed launches.  With pins (--autotune, one benchmark) the plan is
    pinned without a search, and so is a kernel's (splits, variant) in fixed
    (--pin)."""
    from phobos_amd import autotune
    N = 4096
    jobs = {"gemm_fp32": ("gemm", px.GEMM_FP32, (N, N, N), dict(alpha=0.125, beta=1.5)),
            "gemm_fp16tc_fp32acc": ("gemm", px.GEMM_FP16TC_FP32ACC, (N, N, N), {}),
            "gemm_fp16": ("gemm", px.GEMM_FP16, (N, N, N), {}),
            "flash_fp32": ("flash", px.FLASH_FP32_BH, (64, N, N), {}),
            "flash_fp16": ("flash", px.FLASH_FP16_BH, (64, N, N), {})}
    out = {}
    for name in wanted:
        if name not in jobs:
            continue  # saxpy has no plan choices
        kind, kid, dims, kw = jobs[name]
        pdims = list(dims) + ([64] if kind == "flash" else [])
        if fixed and name in fixed:
            try:
                px.plan_pin(kid, pdims, *fixed[name])
            except px.PhxError as e:  # a variant the kernel lacks, splits outside 1..16
                sys.exit(f"bench.py: --pin {name}={fixed[name][0]},{fixed[name][1]}: {e}")
            out[name] = {"pinned": list(px.plan_get(kid, pdims)),
                         "plan": autotune.plan_name(kid, fixed[name])}
            continue
        if pins:
            plan = autotune.plan_from_pins(kid, pins)
            px.plan_pin(kid, pdims, *plan)
            out[name] = {"pinned": list(px.plan_get(kid, pdims)),
                         "plan": autotune.plan_name(kid, plan)}
            continue
        t0 = time.perf_counter()
        try:
            if kind == "gemm":
                r = autotune.tune_gemm(stream, kid, *dims, **kw)
            else:
                r = autotune.tune_flash(stream, kid, *dims)
        except px.PhxError as e:  # keep the built-in plan; the timed steps still run
            px.plan_pin(kid, pdims, None)
            out[name] = {"error": str(e), "plan": list(px.plan_get(kid, pdims))}
            log(f"autotune {name} failed ({e}); built-in plan {out[name]['plan']}")
            continue
        out[name] = {"winner": list(r["winner"]), "plan": autotune.plan_name(kid, r["winner"]),
                     "us": round(r["us"], 2),
                     "finalists": [[list(f["plan"]), round(f["us"], 2)] for f in r["stage2"]],
                     "plans_tried": len(r["stage1"]), "s": round(time.perf_counter() - t0, 2)}
        log(f"autotune {name}: winner {out[name]['plan']}, {r['us']:.1f} us; "
            f"finalists {out[name]['finalists']}")
    return out


def cpu_baseline(seconds):
    """The CPU counterpart of the headline: the oracle's blocked f32 GEMM
    (OpenMP, every host core) over the gemm_fp16tc_fp32acc inputs, i.e.
    f16-valued A and B in f32 storage, at the full 4096^3 config with C = 0,
    alpha = 1, beta = 0; repeated for about `seconds`."""
    import oracle
    M = 4096
    A = oracle.f16_round(oracle.normal_f32(1, M * M, 1 / 64)).reshape(M, M)
    B = oracle.f16_round(oracle.normal_f32(2, M * M, 1 / 64)).reshape(M, M)
    C = np.zeros((M, M), np.float32)
    flop = 2 * M ** 3 + M * M
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.sgemm_f32(1.0, A, B, 0.0, C)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= 30:
            break
    return {"value": round(flop * reps / el / 1e12, 4), "unit": "TFLOP/s",
            "cores": oracle.num_threads(), "kind": "port",
            "sample": f"oracle orc_sgemm_f32 (f32 FMA, blocked, OpenMP on "
                      f"{oracle.num_threads()} threads) over the gemm_fp16tc inputs "
                      f"(f16-valued, f32 storage), full {M}^3, {reps} reps in {el:.1f} s"}


def cpu_other_legs():
    """The other configs' CPU counterparts (oracle, every host core) at their
    full BASELINE sizes, plus the reference-style 64-sample f64 GEMM check
    (main.rs:386-445)."""
    import oracle
    thr = oracle.num_threads()
    out = {"nproc": os.cpu_count(), "omp_threads": thr}
    n = 4096 * 4096
    x, y = oracle.lcg_f32(1, n), oracle.lcg_f32(2, n)
    oracle.saxpy_mt(np.float32(2.5), x, y)
    t0 = time.perf_counter()
    for _ in range(5):
        oracle.saxpy_mt(np.float32(2.5), x, y)
    el = (time.perf_counter() - t0) / 5
    out["saxpy_fp32"] = {"value": round(12 * n / el / 1e9, 2), "unit": "GB/s", "cores": thr,
                         "kind": "port", "sample": f"orc_saxpy_mt (OpenMP, mul and add "
                                                   f"separately rounded), full n = {n}, 5 runs"}
    M = 4096
    A = oracle.lcg_f32(1, M * M).reshape(M, M)
    B = oracle.lcg_f32(2, M * M).reshape(M, M)
    C = oracle.lcg_f32(3, M * M).reshape(M, M)
    t0 = time.perf_counter()
    oracle.sgemm_f32(0.125, A, B, 1.5, C)
    el = time.perf_counter() - t0
    out["gemm_fp32"] = {"value": round((2 * M ** 3 + M * M) / el / 1e12, 4), "unit": "TFLOP/s",
                        "cores": thr, "kind": "port",
                        "sample": f"orc_sgemm_f32, full {M}^3, alpha 0.125, beta 1.5, "
                                  f"in {el:.2f} s"}
    heads, S, D = 64, 4096, 64
    q, k, v = (oracle.normal_f32(s, heads * S * D).reshape(heads, S, D) for s in (1, 2, 3))
    t0 = time.perf_counter()
    oracle.flash_f32(q, k, v, 0.125)
    el = time.perf_counter() - t0
    out["flash_fp32"] = {"value": round(4 * S * S * D * heads / el / 1e12, 4), "unit": "TFLOP/s",
                         "cores": thr, "kind": "port",
                         "sample": f"orc_flash_f32 (f32, OpenMP), all {heads} heads "
                                   f"of 4096x4096x64 in {el:.2f} s"}
    r, c = oracle.sample_points(M, M, 64)
    t0 = time.perf_counter()
    oracle.gemm_points(r, c, A, B, C, 0.125, 1.5)
    out["gemm_check_64_samples_s"] = round(time.perf_counter() - t0, 4)
    return out


def cluster_leg(px):
    """One pod running the matmul_cluster segment: 16384^3 f32, supertiles
    4096 / 8192 / 4096, A/B/C from Lcg-seeded files.  COMPUTE-only TFLOP/s
    from the pod's per-launch events; end-to-end wall time separately."""
    import shutil
    import tempfile
    from phobos_amd import cluster
    M = N = K = 16384
    work = tempfile.mkdtemp(prefix="phx_bench_cluster_")
    try:
        t0 = time.perf_counter()
        stats, _, instrs = cluster.run_matmul_job(work, M, N, K, 4096, 8192, 4096, 0.125, 1.5)
        job_s = time.perf_counter() - t0
    finally:
        shutil.rmtree(work, ignore_errors=True)
    flop = 2 * M * N * K
    return {"workload": "matmul_cluster, one pod: C = 0.125*A@B + 1.5*C, 16384^3 f32, "
                        "supertiles 4096/8192/4096, Lcg seeds 1/2/3 in file:// tensors",
            "compute_tflops": round(flop / (stats["compute_ns"] / 1e9) / 1e12, 2),
            "compute_ms": round(stats["compute_ns"] / 1e6, 2),
            "segment_wall_ms": round(stats["wall_ns"] / 1e6, 2),
            "io_ms": round(stats["io_ns"] / 1e6, 2),
            "job_wall_s_incl_input_files": round(job_s, 2),
            "ops": {k: stats[k] for k in ("alloc", "load", "compute", "store", "free")}}


# CSV rows (phobos-bench/src/main.rs): benchmark name, precision label and
# GFLOP per launch.  saxpy counts 2 flops per element (main.rs:1284), the GEMMs
# 2MNK + MN (main.rs:591, 824), flash 4 Nq Nk D per head (main.rs:1032, 1160).
CSV_ROWS = {
    "saxpy_fp32": ("saxpy_fp32", "f32", 2 * 4096 * 4096 / 1e9),
    "gemm_fp32": ("gemm_fp32", "f32", GEMM_FLOP / 1e9),
    "gemm_fp16tc_fp32acc": ("gemm_fp16tc_fp32acc", "f16-tc-f32-acc", GEMM_FLOP / 1e9),
    "gemm_fp16": ("gemm_fp16", "f16-tc", GEMM_FLOP / 1e9),
    "flash_fp32": ("flash_fp32", "f32", FLASH_FLOP / 1e9),
    "flash_fp16": ("flash_fp16tc_fp32acc", "f16-tc-f32-acc", FLASH_FLOP / 1e9),
}


def vendor_rows(wanted, reps=20):
    """The reference's cuBLAS comparison rows (main.rs:611-622, 837-848,
    1295-1306) from the ROCm libraries torch calls: saxpy as y += 2.5 x, the f32
    GEMM (also the baseline row of gemm_fp16tc_fp32acc, as in the reference) and
    the f16 GEMM, on the BASELINE shapes.  Timed with torch's events over
    `reps` launches after 5 warmups.  Returns [(benchmark, impl, precision,
    gflops)]."""
    import torch
    lib = str(torch.backends.cuda.preferred_blas_library()).split(".")[-1].lower()
    blas = "hipBLASLt" if "lt" in lib else "rocBLAS"
    N = 4096
    g = torch.Generator(device="cuda").manual_seed(1)

    def timed(fn):
        for _ in range(5):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps / 1e3  # s

    rows = []
    if "saxpy_fp32" in wanted:
        xs = [torch.rand(N * N, device="cuda", generator=g) for _ in range(4)]
        ys = [torch.rand(N * N, device="cuda", generator=g) for _ in range(4)]
        it = iter(range(1 << 30))

        def saxpy():
            i = next(it) % 4
            ys[i].add_(xs[i], alpha=2.5)
        rows.append(("saxpy_fp32", "torch", "f32", CSV_ROWS["saxpy_fp32"][2] / timed(saxpy)))
    if "gemm_fp32" in wanted or "gemm_fp16tc_fp32acc" in wanted:
        a, b = (torch.randn(N, N, device="cuda", generator=g) for _ in range(2))
        t = timed(lambda: torch.mm(a, b))
        for name in ("gemm_fp32", "gemm_fp16tc_fp32acc"):
            if name in wanted:
                rows.append((name, blas, "f32", GEMM_FLOP / 1e9 / t))
    if "gemm_fp16" in wanted:
        a, b = (torch.randn(N, N, device="cuda", generator=g, dtype=torch.float16)
                for _ in range(2))
        rows.append(("gemm_fp16", blas, "f16-tc", GEMM_FLOP / 1e9 / timed(lambda: torch.mm(a, b))))
    return rows


def write_results_csv(args, kern, wanted):
    from phobos_amd import report
    res = report.Results()
    for name, (bench, prec, gflop) in CSV_ROWS.items():
        if name in kern:
            res.push(bench, "phobos", prec, gflop / (kern[name]["ms_avg"] / 1e3))
    if args.vendor:
        # torch brings its own HIP runtime, which cannot share a process with
        # the library's: the vendor rows are timed in a child process
        cp = subprocess.run([sys.executable, os.path.abspath(__file__), "--vendor-only",
                             "--kernels", ",".join(wanted)], capture_output=True, text=True,
                            timeout=600)
        if cp.returncode != 0:
            raise RuntimeError(f"vendor rows failed: {cp.stderr[-2000:]}")
        for row in json.loads(cp.stdout.strip().splitlines()[-1]):
            res.push(*row)
    peaks = report.Peaks(args.peak_fp32, args.peak_fp16tc, args.peak_fp16tcf32acc)
    n = res.write_csv(args.csv, peaks)
    log(f"theoretical peak: {peaks.describe()}")
    log(f"wrote {n} rows to {args.csv}")


def load_traffic():
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f)
    return {}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this backend has no multi-GPU path)", file=sys.stderr)
        sys.exit(2)
    if args.vendor_only:
        wanted = args.kernels.split(",")
        print(json.dumps(vendor_rows(wanted)), flush=True)
        return
    import phobos_amd as px
    px.init(0)
    if args.copy_calibration:
        nbytes = 256 << 20
        src, dst = px.DeviceBuffer(nbytes), px.DeviceBuffer(nbytes)
        for _ in range(3):
            px.check(px.lib().phx_memcpy_d2d(dst.ptr, src.ptr, nbytes))
        px.synchronize()
        print(json.dumps({"copy_calibration_bytes": nbytes, "copies": 3}))
        return
    info = px.device_info()
    log(f"device: {info}")
    if args.shapes:
        sstream = px.Stream()
        px.bind_workspace(sstream, WORKSPACE_BYTES)
        res = shapes_leg(px, sstream, tune=not args.no_autotune)
        for r in res:
            log(f"{r['kernel']:28s} {str(r['shape']):18s} splits {r['splits']:2d}  "
                f"{r['us']:8.2f} us  {r['tflops']:8.2f} TFLOP/s  autotuned {r['autotuned']}")
        print(json.dumps({"shapes": res, "device": info}), flush=True)
        return
    all_names = ["saxpy_fp32", "gemm_fp32", "gemm_fp16tc_fp32acc", "gemm_fp16", "flash_fp32",
                 "flash_fp16"]
    wanted = all_names if args.kernels == "all" else args.kernels.split(",")
    stream = px.Stream()
    px.bind_workspace(stream, WORKSPACE_BYTES)
    tuned = None
    if not args.no_autotune and not args.hold:
        tuned = autotune_leg(px, stream, wanted, args.pins, args.fixed)
    ks = setup(px, stream, wanted)
    if args.hold > 0:
        t0, n = time.perf_counter(), 0
        while time.perf_counter() - t0 < args.hold:
            for k in ks:
                for _ in range(REPS[k.name]):
                    k.launch()
            stream.synchronize()
            n += 1
        dt = time.perf_counter() - t0
        print(json.dumps({"hold_s": round(dt, 2), "rounds": n,
                          "kernels": [k.name for k in ks],
                          "us_per_round": round(dt / n * 1e6, 1)}))
        return
    ev = [px.Event() for _ in range(len(ks) + 1)]
    # per-step events: ev[i] before kernel i, ev[-1] after the last
    for _ in range(args.warmup):
        for k in ks:
            for _ in range(REPS[k.name]):
                k.launch()
    stream.synchronize()
    px.synchronize()
    step_events = []
    t0 = time.perf_counter()
    for s in range(args.steps):
        evs = [px.Event() for _ in range(len(ks) + 1)]
        for i, k in enumerate(ks):
            evs[i].record(stream)
            for _ in range(REPS[k.name]):
                k.launch()
        evs[-1].record(stream)
        step_events.append(evs)
    stream.synchronize()
    px.synchronize()
    wall = time.perf_counter() - t0
    for evs in step_events:
        for i, k in enumerate(ks):
            k.times.append(evs[i].elapsed_ms(evs[i + 1]) / REPS[k.name])
    gpu_ms = sum(evs[0].elapsed_ms(evs[-1]) for evs in step_events)
    for evs in step_events:
        for e in evs:
            e.destroy()

    traffic = load_traffic()
    kern = {}
    for k in ks:
        t = np.array(k.times)
        avg = float(t.mean())
        val = k.work / (avg / 1e3)
        kern[k.name] = {
            "value": round(val, 2), "unit": k.unit, "ms_avg": round(avg, 4),
            "launches_per_step": REPS[k.name],
            "ms_min": round(float(t.min()), 4), "ms_median": round(float(np.median(t)), 4),
            "roofline": {"bound": k.bound, "achieved": round(val, 2), "peak": k.peak,
                         "unit": "GB/s" if k.bound == "hbm" else "TFLOP/s",
                         "frac": round(val / k.peak, 4),
                         "traffic": traffic.get(k.name)},
        }
        if k.name.startswith("flash"):
            kern[k.name]["exp_rate"] = {"exps": FLASH_EXPS,
                                        "value": round(FLASH_EXPS / (avg / 1e3) / 1e9, 1),
                                        "unit": "Gexp/s"}
        log(f"{k.name:22s} avg {avg:8.4f} ms  min {t.min():8.4f} ms  "
            f"{val:10.2f} {k.unit}  ({100 * val / k.peak:5.1f}% of peak)")

    if "saxpy_fp32" in kern:
        try:
            ceil = hbm_ceiling_leg(px)
            ceil["saxpy_frac_of_it"] = round(kern["saxpy_fp32"]["value"] / ceil["value"], 3)
        except px.PhxError as e:
            ceil = {"error": str(e)}
        kern["saxpy_fp32"]["hbm_copy_ceiling"] = ceil
        log(f"hbm ceiling on this box: {ceil}")
    if args.csv:
        write_results_csv(args, kern, wanted)
    head = "gemm_fp16tc_fp32acc"
    hk = kern.get(head) or next(iter(kern.values()))
    cluster_res = None
    if not args.no_cluster:
        log("matmul_cluster one-pod job ...")
        try:
            cluster_res = cluster_leg(px)
        except Exception as e:  # e.g. no room for its 4 GiB of files: the headline still prints
            cluster_res = {"error": repr(e)}
        log(f"matmul_cluster: {cluster_res}")
    cpu = cpu_more = None
    if not args.no_cpu:
        log("cpu baseline ...")
        try:
            cpu = cpu_baseline(args.cpu_seconds)
        except Exception as e:  # the GPU figures still print
            cpu = {"error": repr(e)}
        log(f"cpu baseline: {cpu}")
        try:
            cpu_more = cpu_other_legs()
        except Exception as e:
            cpu_more = {"error": repr(e)}
        log(f"cpu legs: {cpu_more}")
    out = {
        "metric": "achieved TFLOPS & % peak: gemm_fp16tc 4096^3, flash_fp16; saxpy HBM GB/s",
        "value": hk["value"],
        "unit": hk["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gpu_ms / args.steps, 4),
        "wall_ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 (f32 accumulate)",
        "data": "synthetic (Lcg / Box-Muller seeded inputs of the BASELINE shapes)",
        "config": {"workload": "gemm_fp16tc_fp32acc M=N=K=4096, A,B=f16(N(0,1)/64) in f32 "
                               "storage, C=0, alpha=1, beta=0; step = phobos-bench suite "
                               "(saxpy 2^24, gemm_fp32/fp16tc/fp16 4096^3, flash fp32/fp16 "
                               "B4xH16x4096x4096xD64)",
                   "global_batch": 1, "seq_len": 4096, "parallelism": "none (1 GPU)"},
        "roofline": hk["roofline"],
        "cpu_baseline": cpu,
        "cpu_legs": cpu_more,
        "kernels": kern,
        "autotune": tuned,
        "matmul_cluster": cluster_res,
        "device": info,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
