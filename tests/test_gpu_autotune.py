"""The launch-plan autotuner (phobos_amd.autotune) and the plan pins it sets
(phx_plan_get / phx_plan_pin), against the f64 oracle.

The reference's autotuner (phobos-bench/src/autotune.rs:98-192) searches
tile sizes; this backend searches the split count and, for
gemm_fp16tc_fp32acc, which of its two kernel families runs.  Every
plan computes the same products and differs only in the order of the f32
sums, so each is held to the same bounds as the unsplit launch: f32 GEMM
1e-4 relative (floored at 1% of the RMS), f16 paths 2e-2 RMS-normalised,
flash |err| / max(|want|, 0.1) (main.rs:912-917) within 1e-4 (f32) or 2e-2
(f16).
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _unpin(px_gpu):
    px_gpu.plan_unpin_all()
    yield
    px_gpu.plan_unpin_all()


def _gemm_case(px, stream, kern, M, N, K, seed=61):
    r16 = kern != px.GEMM_FP32
    A = oracle.normal_f32(seed, M * K, 1 / np.sqrt(K)).reshape(M, K)
    B = oracle.normal_f32(seed + 1, K * N, 1 / np.sqrt(K)).reshape(K, N)
    C = oracle.normal_f32(seed + 2, M * N).reshape(M, N)
    if r16:
        A, B, C = oracle.f16_round(A), oracle.f16_round(B), oracle.f16_round(C)
    f16 = kern == px.GEMM_FP16
    conv = oracle.f16_bits if f16 else (lambda t: np.ascontiguousarray(t, np.float32))
    da, db, dc = (px.DeviceBuffer.from_array(conv(t)) for t in (A, B, C))

    def run():
        dc.upload(conv(C))
        px.launch_gemm(stream, kern, da, db, dc, M, N, K, 0.5, 0.25)
        stream.synchronize()
        if f16:
            return oracle.f16_to_f32(dc.download(np.uint16, M * N)).reshape(M, N)
        return dc.download(np.float32, (M, N))
    want = oracle.gemm_full(A, B, C, 0.5, 0.25, round16=r16)
    return run, want


def _gemm_ok(px, kern, got, want):
    if kern == px.GEMM_FP32:
        floor = 1e-2 * np.sqrt(np.mean(want ** 2))
        assert (np.abs(got - want) / np.maximum(np.abs(want), floor)).max() < 1e-4
    else:
        assert np.abs(got - want).max() / np.sqrt(np.mean(want ** 2)) < 2e-2


def test_plan_get_reports_the_built_in_rule(px_gpu):
    px = px_gpu
    for kern in (px.GEMM_FP32, px.GEMM_FP16TC_FP32ACC, px.GEMM_FP16):
        assert px.plan_get(kern, [4096, 4096, 4096]) == (1, 0)
        assert px.plan_get(kern, [512, 512, 4096])[0] == px.split_plan(kern, [512, 512, 4096])[0]
    assert px.plan_get(px.GEMM_FP32, [1024, 1024, 1024]) == (1, 7)  # the 64 x 64 tiling
    assert px.plan_get(px.GEMM_FP32, [256, 256, 8192]) == (16, 0)  # long K, few tiles: split
    assert px.plan_get(px.FLASH_FP16_BH, [64, 4096, 4096, 64]) == (1, 0)
    assert px.plan_get(px.FLASH_FP16, [4096, 4096, 64])[0] > 1


def test_pins_take_effect_and_come_off(px_gpu, stream):
    px = px_gpu
    kern, dims = px.GEMM_FP32, [1024, 1024, 1024]
    run, want = _gemm_case(px, stream, kern, *dims)  # built-in: 64 x 64 x 16, unsplit
    auto = px.plan_get(kern, dims)
    for sp in (1, 3, 16):
        px.plan_pin(kern, dims, sp)
        assert px.plan_get(kern, dims) == (sp, 0)
        assert px.split_plan(kern, dims)[0] == sp
        _gemm_ok(px, kern, run(), want)
    px.plan_pin(kern, dims, None)
    assert px.plan_get(kern, dims) == auto
    # a pin is per shape and per kernel
    other_shape = px.plan_get(kern, [1024, 1024, 2048])
    other_kernel = px.plan_get(px.GEMM_FP16, dims)
    px.plan_pin(kern, dims, 2)
    assert px.plan_get(kern, dims) == (2, 0)
    assert px.plan_get(kern, [1024, 1024, 2048]) == other_shape == (1, 7)
    assert px.plan_get(px.GEMM_FP16, dims) == other_kernel
    px.plan_unpin_all()
    assert px.plan_get(kern, dims) == auto


def test_invalid_pins_are_refused(px_gpu):
    px = px_gpu
    dims = [512, 512, 512]
    for sp, var, kern in ((0, 0, px.GEMM_FP32), (17, 0, px.GEMM_FP32), (1, 8, px.GEMM_FP32),
                          (2, 1, px.GEMM_FP32),
                          (1, 2, px.GEMM_FP16TC_FP32ACC), (1, 1, px.GEMM_FP16)):
        with pytest.raises(px.PhxError):
            px.plan_pin(kern, dims, sp, var)
    with pytest.raises(px.PhxError):
        px.plan_pin(px.SAXPY_FP32, [1024], 1)
    for bad in ([0, 512, 512], [512, 512]):  # shapes the kernel refuses
        with pytest.raises(px.PhxError):
            px.plan_pin(px.GEMM_FP32, bad, 1)


def test_tc_variant_pin_runs_the_one_wave_kernel(px_gpu, stream):
    # variant 1 = the one-wave kernel; both kernels sum each output's K
    # products in the same order, so the outputs are bit-identical.
    px = px_gpu
    kern, dims = px.GEMM_FP16TC_FP32ACC, [1024, 512, 2048]
    run, want = _gemm_case(px, stream, kern, *dims)
    px.plan_pin(kern, dims, 1, 0)
    w8 = run()
    px.plan_pin(kern, dims, 1, 1)
    assert px.plan_get(kern, dims) == (1, 1)
    one = run()
    assert np.array_equal(w8.view(np.uint32), one.view(np.uint32))
    _gemm_ok(px, kern, one, want)


@pytest.mark.parametrize("kern_name", ["GEMM_FP32", "GEMM_FP16TC_FP32ACC", "GEMM_FP16"])
def test_tune_gemm_pins_a_correct_winner(px_gpu, stream, kern_name):
    from phobos_amd import autotune
    px = px_gpu
    kern = getattr(px, kern_name)
    dims = [512, 512, 2048]
    r = autotune.tune_gemm(stream, kern, *dims, short_probes=1, long_probes=3, finalists=2)
    space = autotune.gemm_space(kern, *dims)
    assert tuple(r["winner"]) in space and len(r["stage1"]) == len(space)
    assert all("us" in s for s in r["stage1"]), r["stage1"]
    assert px.plan_get(kern, dims) == tuple(r["winner"])
    assert r["us"] == min(f["us"] for f in r["stage2"])
    run, want = _gemm_case(px, stream, kern, *dims)
    _gemm_ok(px, kern, run(), want)


@pytest.mark.parametrize("bits", [16, 32])
def test_tune_flash_pins_a_correct_winner(px_gpu, stream, bits):
    from phobos_amd import autotune
    px = px_gpu
    one, bh = (px.FLASH_FP16, px.FLASH_FP16_BH) if bits == 16 else (px.FLASH_FP32, px.FLASH_FP32_BH)
    Nq, Nk, D = 1024, 3000, 64
    r = autotune.tune_flash(stream, one, 1, Nq, Nk, short_probes=1, long_probes=3, finalists=2)
    assert tuple(r["winner"]) in autotune.flash_space(1, Nq, Nk)
    # one pin for the one-head kernel and the batched kernel at one head
    assert px.plan_get(one, [Nq, Nk, D]) == tuple(r["winner"])
    assert px.plan_get(bh, [1, Nq, Nk, D]) == tuple(r["winner"])
    q = oracle.normal_f32(71, Nq * D).reshape(Nq, D)
    k = oracle.normal_f32(72, Nk * D).reshape(Nk, D)
    v = oracle.normal_f32(73, Nk * D).reshape(Nk, D)
    if bits == 16:
        q, k, v = (oracle.f16_round(t) for t in (q, k, v))
        up = lambda t: px.DeviceBuffer.from_array(oracle.f16_bits(t))  # noqa: E731
    else:
        up = lambda t: px.DeviceBuffer.from_array(np.ascontiguousarray(t, np.float32))  # noqa: E731
    dq, dk, dv = up(q), up(k), up(v)
    do = px.DeviceBuffer(Nq * D * bits // 8)
    px.launch_flash(stream, one, dq, dk, dv, do, Nq, Nk, D, 0.125)
    stream.synchronize()
    if bits == 16:
        got = oracle.f16_to_f32(do.download(np.uint16, Nq * D)).reshape(Nq, D)
    else:
        got = do.download(np.float32, (Nq, D))
    rows = np.unique(np.linspace(0, Nq - 1, 32).astype(np.int64))
    want = oracle.flash_rows(rows, q, k, v, 0.125)
    assert (np.abs(got[rows] - want) / np.maximum(np.abs(want), 0.1)).max() < (2e-2 if bits == 16 else 1e-4)
