"""Two-stage launch-plan autotuner for the built-in GEMM and flash kernels.

The reference's autotuner (phobos-bench/src/autotune.rs:98-192) compiles
every point of a kernel's @autotune space (TILE_M / TILE_N / TILE_K, BR / BC),
verifies it on its first launch, ranks all of them by a few short probes,
then times the fastest few round-robin, one launch each per round after a
joint warmup, so every finalist sees the same clocks, and keeps the
fastest minimum.  Here a probe is the average of enough back-to-back
launches for about 200 us (one launch when that is longer), timed with HIP
events on the launch stream; in the round-robin each probe follows one
untimed launch of the same plan, so it does not inherit the previous plan's
cache contents (a split plan's partial sums can push the operands out of
the 256 MB MALL, which the next plan would then pay for).  The space here
is the launch plan (phx_plan): the number of K chunks of a GEMM or key
chunks of a flash launch, gemm_fp32's tile dims (TILE_M x TILE_N x TILE_K
over the reference's ranges), and for gemm_fp16tc_fp32acc which of its
two kernel families (eight-wave or one-wave) runs.  The winner is pinned
with phx_plan_pin, so every later launch of that kernel at that shape uses
it.

A candidate is verified on its first launch against the unsplit plan's
output (a split changes only the order of the f32 sums): relative to the
largest output magnitude, within 1e-4 for f32 outputs and 2e-3 for f16
outputs (two f16 roundings apart at most).
"""
import math

import numpy as np

from . import (FLASH_FP16, FLASH_FP16_BH, FLASH_FP32_BH, GEMM_FP16, GEMM_FP16TC_FP32ACC,
               GEMM_FP32, GEMM_FP32_TILINGS,
               DeviceBuffer, Event, PhxError, bind_workspace, get_workspace, launch_flash,
               launch_flash_bh, launch_gemm, normal_f32, plan_pin, to_f16_bits)

SPLITS = (1, 2, 3, 4, 6, 8, 12, 16)  # the split counts a search tries
MAX_WORKSPACE = 4 << 30               # skip splits whose partial sums need more
WARMUP = 10                           # autotune.rs WARMUP


def _effective(units, sp):
    """The chunk count a launch really uses for sp chunks of units steps
    (whole steps per chunk, no empty chunk), as the runtime rounds it."""
    sp = min(sp, units)
    if sp < 2:
        return 1
    per = -(-units // sp)
    return -(-units // per)


def gemm_space(kernel, M, N, K):
    """[(splits, variant)] for a GEMM: every distinct split count; for
    gemm_fp32 every other tiling (TILE_M x TILE_N x TILE_K, the @autotune
    dims of examples/gemm_fp32.ph:1), unsplit; for gemm_fp16tc_fp32acc the
    one-wave kernel, unsplit, too."""
    steps = -(-K // 32)
    space = []
    for sp in SPLITS:
        e = _effective(steps, sp)
        if (e, 0) not in space and (e == 1 or e * M * N * 4 <= MAX_WORKSPACE):
            space.append((e, 0))
    if kernel == GEMM_FP32:
        space += [(1, v) for v in range(1, len(GEMM_FP32_TILINGS))]
    if kernel == GEMM_FP16TC_FP32ACC:
        space.append((1, 1))
    return space


def search_dims(kernel):
    """Names a --autotune pin may set for kernel (autotune.rs:38-58 checks
    pins against the kernel's @autotune dims)."""
    if kernel == GEMM_FP32:
        return ("splits", "variant", "TILE_M", "TILE_N", "TILE_K")
    return ("splits", "variant")


def plan_from_pins(kernel, pins):
    """The (splits, variant) plan that NAME=VALUE pins name.  For gemm_fp32
    TILE_M / TILE_N / TILE_K select the tiling (dims not given keep the
    built-in 256 x 256 x 16's value); PhxError if no tiling has them."""
    sp, v = pins.get("splits", 1), pins.get("variant", 0)
    tile = [pins.get(d) for d in ("TILE_M", "TILE_N", "TILE_K")]
    if kernel == GEMM_FP32 and any(t is not None for t in tile):
        want = tuple(t if t is not None else b for t, b in zip(tile, GEMM_FP32_TILINGS[0]))
        if want not in GEMM_FP32_TILINGS:
            raise PhxError(-1, f"no gemm_fp32 tiling TILE_M={want[0]} TILE_N={want[1]} "
                               f"TILE_K={want[2]}; tilings: " +
                               ", ".join("%dx%dx%d" % t for t in GEMM_FP32_TILINGS))
        v = GEMM_FP32_TILINGS.index(want)
    return sp, v


def plan_name(kernel, plan):
    """A readable name of a (splits, variant) plan: gemm_fp32's tiling dims."""
    sp, v = plan
    if kernel == GEMM_FP32:
        tm, tn, tk = GEMM_FP32_TILINGS[v]
        return f"TILE_M={tm} TILE_N={tn} TILE_K={tk} splits={sp}"
    return f"splits={sp} variant={v}"


def flash_space(BH, Nq, Nk):
    """[(splits, 0)] for a flash launch: every distinct key-chunk count."""
    nkb = -(-Nk // 64)
    space = []
    for sp in SPLITS:
        e = _effective(nkb, sp)
        if (e, 0) not in space and (e == 1 or e * BH * Nq * 66 * 4 <= MAX_WORKSPACE):
            space.append((e, 0))
    return space


class Autotuner:
    """autotune.rs Autotuner: launch() runs the kernel once on stream under
    the pinned plan; verify() is called after a plan's first launch and
    raises AssertionError if that plan's output is wrong (it may launch again
    from restored inputs, as the GEMM's C is read and written); reset(), if
    given, restores the inputs before each timed probe, outside the timing
    (a GEMM with beta != 0 would otherwise grow C by beta every launch)."""

    def __init__(self, stream, kernel, dims, launch, verify, short_probes=3, long_probes=10,
                 finalists=3, reset=None):
        self.stream, self.kernel, self.dims = stream, kernel, list(dims)
        self.launch, self.verify, self.reset = launch, verify, reset
        self.short_probes, self.long_probes, self.finalists = short_probes, long_probes, finalists
        self.e0, self.e1 = Event(), Event()

    def _time(self, reps=1):
        """Average seconds per launch over reps back-to-back launches."""
        if self.reset is not None:
            self.stream.synchronize()  # nothing may still be writing what reset() restores
            self.reset()
        self.e0.record(self.stream)
        for _ in range(reps):
            self.launch()
        self.e1.record(self.stream)
        self.e1.synchronize()
        return self.e0.elapsed_ms(self.e1) / 1e3 / reps

    def _reps(self):
        """Launches per probe: enough for about 200 us of work, so the events'
        own overhead (a few us) does not rank short launches."""
        t = self._time()
        return max(1, min(50, math.ceil(200e-6 / max(t, 1e-7))))

    def run(self, space):
        """Returns {"winner": plan, "us": its fastest launch, "stage1": [...],
        "stage2": [...]}, and leaves the winner pinned."""
        stage1 = []
        for plan in space:  # stage 1: verify (first launch) and short-probe each plan
            plan_pin(self.kernel, self.dims, *plan)
            try:
                self.launch()
                self.stream.synchronize()
                self.verify()
                reps = self._reps()
                best = min(self._time(reps) for _ in range(max(1, self.short_probes)))
            except (PhxError, AssertionError) as e:
                stage1.append({"plan": plan, "skipped": str(e)})
                continue
            stage1.append({"plan": plan, "us": best * 1e6, "reps": reps})
        ranked = sorted((r for r in stage1 if "us" in r), key=lambda r: r["us"])
        if not ranked:
            plan_pin(self.kernel, self.dims, None)
            raise PhxError(-1, "autotune: no plan works")
        fin = [{"plan": r["plan"], "reps": r["reps"], "min": math.inf, "max": 0.0}
               for r in ranked[:self.finalists]]
        for f in fin:  # one joint warmup ramps the clocks before the timed probes
            plan_pin(self.kernel, self.dims, *f["plan"])
            for _ in range(WARMUP):
                self.launch()
        self.stream.synchronize()
        for _ in range(max(1, self.long_probes)):  # stage 2: round-robin, one launch each
            for f in fin:
                plan_pin(self.kernel, self.dims, *f["plan"])
                self.launch()  # untimed: the caches then hold this plan's data, not the last one's
                t = self._time(f["reps"])
                f["min"], f["max"] = min(f["min"], t), max(f["max"], t)
        win = min(fin, key=lambda f: f["min"])
        plan_pin(self.kernel, self.dims, *win["plan"])
        return {"winner": win["plan"], "us": win["min"] * 1e6, "stage1": stage1,
                "stage2": [{"plan": f["plan"], "us": f["min"] * 1e6,
                            "spread_us": (f["max"] - f["min"]) * 1e6} for f in fin]}


def ensure_workspace(stream, nbytes):
    """Split launches take their partial results from the workspace bound to
    their stream and run unsplit without one; the search binds one large
    enough for every plan it times (replacing a smaller one), and the winner
    then runs with it."""
    if get_workspace(stream)[1] < nbytes:
        bind_workspace(stream, nbytes)


def _close(got, want, tol):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(float(np.max(np.abs(want))), 1e-30)
    err = float(np.max(np.abs(got - want))) / scale
    assert np.isfinite(got).all() and err <= tol, f"output differs from the unsplit plan by {err:.3g}"


def tune_gemm(stream, kernel, M, N, K, alpha=1.0, beta=0.0, seed=1, **kw):
    """Searches gemm_space for kernel at M x N x K (row-major, alpha, beta as
    the caller launches it) on seeded inputs and pins the winner."""
    f16 = kernel == GEMM_FP16
    esz = 2 if f16 else 4
    conv = (lambda x: to_f16_bits(x)) if f16 else (lambda x: x.astype(np.float32))
    if kernel == GEMM_FP16TC_FP32ACC:  # f16-valued inputs in f32 storage
        conv = lambda x: x.astype(np.float16).astype(np.float32)  # noqa: E731
    a = conv(normal_f32(seed, M * K, 1 / math.sqrt(K)))
    b = conv(normal_f32(seed + 1, K * N, 1 / math.sqrt(K)))
    c0 = conv(normal_f32(seed + 2, M * N))
    A, B = DeviceBuffer.from_array(a), DeviceBuffer.from_array(b)
    C = DeviceBuffer(M * N * esz)
    dims = [M, N, K]
    out_dtype = np.uint16 if f16 else np.float32

    def run_once():
        launch_gemm(stream, kernel, A, B, C, M, N, K, alpha, beta)

    def result():
        r = C.download(out_dtype, M * N)
        return r.view(np.float16).astype(np.float32) if f16 else r

    plan_pin(kernel, dims, 1, 0)
    C.upload(c0)
    run_once()
    stream.synchronize()
    want = result()
    tol = 2e-3 if f16 else 1e-4

    def verify():
        C.upload(c0)
        run_once()
        stream.synchronize()
        _close(result(), want, tol)

    reset = None if beta == 0.0 else (lambda: C.upload(c0))
    space = gemm_space(kernel, M, N, K)
    ensure_workspace(stream, max(sp for sp, _ in space) * M * N * 4)
    tuner = Autotuner(stream, kernel, dims, run_once, verify, reset=reset, **kw)
    return tuner.run(space)


def tune_flash(stream, kernel, BH, Nq, Nk, D=64, scale=0.125, seed=1, **kw):
    """Searches flash_space for kernel (one-head or batched, f16 or f32) at
    BH heads x Nq queries x Nk keys on seeded N(0,1) inputs; pins the winner
    (shared by the one-head and batched kernels of the precision)."""
    f16 = kernel in (FLASH_FP16, FLASH_FP16_BH)
    bh = kernel in (FLASH_FP16_BH, FLASH_FP32_BH)
    if not bh and BH != 1:
        raise PhxError(-1, "the one-head flash kernels take BH = 1")
    dims = [BH, Nq, Nk, D] if bh else [Nq, Nk, D]
    conv = to_f16_bits if f16 else (lambda x: x.astype(np.float32))
    Q = DeviceBuffer.from_array(conv(normal_f32(seed, BH * Nq * D)))
    K = DeviceBuffer.from_array(conv(normal_f32(seed + 1, BH * Nk * D)))
    V = DeviceBuffer.from_array(conv(normal_f32(seed + 2, BH * Nk * D)))
    O = DeviceBuffer(BH * Nq * D * (2 if f16 else 4))

    def launch():
        if bh:
            launch_flash_bh(stream, kernel, Q, K, V, O, BH, Nq, Nk, D, scale)
        else:
            launch_flash(stream, kernel, Q, K, V, O, Nq, Nk, D, scale)

    def result():
        r = O.download(np.uint16 if f16 else np.float32, BH * Nq * D)
        return r.view(np.float16).astype(np.float32) if f16 else r

    plan_pin(kernel, dims, 1, 0)
    launch()
    stream.synchronize()
    want = result()
    tol = 2e-3 if f16 else 1e-4

    def verify():
        _close(result(), want, tol)

    space = flash_space(BH, Nq, Nk)
    ensure_workspace(stream, max(sp for sp, _ in space) * BH * Nq * (D + 2) * 4)
    tuner = Autotuner(stream, kernel, dims, launch, verify, **kw)
    return tuner.run(space)

