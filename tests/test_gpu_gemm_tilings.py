"""gemm_fp32's tilings (the launch plan's variant: TILE_M x TILE_N x TILE_K
over the reference's @autotune ranges, examples/gemm_fp32.ph:1) against the
f64 oracle, each pinned with phx_plan_pin and launched through the same
entry point as the built-in plan.

Bounds (the gemm_fp32 contract): max relative error <= 1e-4, floored at 1%
of the output RMS on zero-mean data (cancellation) and at f64::MIN_POSITIVE
on the all-negative Lcg inputs of the BASELINE config (main.rs:398-402);
bit-exact on small-integer data, where every order of the f32 sums is exact
(the masking.rs:108-110 idea).  A guard after C catches stores past it.
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

GUARD, SENTINEL = 4096, 12345.0
VARIANTS = range(8)


def _gemm(px, stream, A, B, C, alpha, beta, variant):
    M, K = A.shape
    N = B.shape[1]
    px.plan_pin(px.GEMM_FP32, [M, N, K], 1, variant)
    try:
        assert px.plan_get(px.GEMM_FP32, [M, N, K]) == (1, variant)
        c = np.concatenate([C.ravel(), np.full(GUARD, SENTINEL, np.float32)])
        da, db, dc = (px.DeviceBuffer.from_array(np.ascontiguousarray(t, np.float32))
                      for t in (A, B, c))
        px.launch_gemm(stream, px.GEMM_FP32, da, db, dc, M, N, K, alpha, beta)
        stream.synchronize()
        out = dc.download(np.float32, M * N + GUARD)
    finally:
        px.plan_pin(px.GEMM_FP32, [M, N, K], None)
    assert np.all(out[M * N:] == SENTINEL), "write past C"
    return out[:M * N].reshape(M, N)


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (300, 200, 100), (64, 64, 8),
                                   (129, 132, 36), (520, 388, 1004)])
def test_tiling_against_oracle(px_gpu, stream, variant, M, N, K):
    # Lcg operands (all of one sign within a row product, as the BASELINE
    # config): 1e-4 relative, floored at 1% of the RMS where 0.125*dot +
    # 1.5*c cancels; zero-mean operands: 1e-5 of the output RMS
    A = oracle.lcg_f32(1, M * K).reshape(M, K)
    B = oracle.lcg_f32(2, K * N).reshape(K, N)
    C = oracle.lcg_f32(3, M * N).reshape(M, N)
    got = _gemm(px_gpu, stream, A, B, C, 0.125, 1.5, variant)
    want = oracle.gemm_full(A, B, C, 0.125, 1.5)
    floor = 1e-2 * np.sqrt(np.mean(want ** 2))
    rel = np.abs(got - want) / np.maximum(np.abs(want), floor)
    assert rel.max() < 1e-4, (px_gpu.GEMM_FP32_TILINGS[variant], rel.max())
    A = oracle.normal_f32(41, M * K).reshape(M, K)
    B = oracle.normal_f32(42, K * N).reshape(K, N)
    C = oracle.normal_f32(43, M * N).reshape(M, N)
    got = _gemm(px_gpu, stream, A, B, C, 0.75, -0.5, variant)
    want = oracle.gemm_full(A, B, C, 0.75, -0.5)
    err = np.abs(got - want).max() / np.sqrt(np.mean(want ** 2))
    assert err < 1e-5, (px_gpu.GEMM_FP32_TILINGS[variant], err)


@pytest.mark.parametrize("variant", VARIANTS)
def test_tiling_exact_on_integers(px_gpu, stream, variant):
    M, N, K = 192, 320, 1000
    rng = np.random.default_rng(9)
    A = rng.integers(-3, 4, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    C = rng.integers(-5, 6, (M, N)).astype(np.float32)
    got = _gemm(px_gpu, stream, A, B, C, 1.0, 2.0, variant)
    want = oracle.gemm_full(A, B, C, 1.0, 2.0)
    assert np.array_equal(got.astype(np.float64), want)


@pytest.mark.parametrize("variant", VARIANTS)
def test_tiling_baseline_config_sampled(px_gpu, stream, variant):
    # the BASELINE gemm_fp32 config: 4096^3, Lcg inputs, alpha 0.125, beta 1.5,
    # checked at the reference's 64 xorshift points with its floor
    px = px_gpu
    M = N = K = 4096
    A = px.lcg_f32(1, M * K).reshape(M, K)
    B = px.lcg_f32(2, K * N).reshape(K, N)
    C = px.lcg_f32(3, M * N).reshape(M, N)
    got = _gemm(px, stream, A, B, C, 0.125, 1.5, variant)
    r, c = oracle.sample_points(M, N, 64)
    want = oracle.gemm_points(r, c, A, B, C, 0.125, 1.5)
    g = got[r.astype(int), c.astype(int)]
    rel = np.abs(g - want) / np.maximum(np.abs(want), np.finfo(np.float64).tiny)
    assert rel.max() < 1e-4, rel.max()


def test_autotuner_searches_the_tilings(px_gpu, stream):
    # the search's space holds every tiling; the winner is verified and pinned
    from phobos_amd import autotune
    px = px_gpu
    r = autotune.tune_gemm(stream, px.GEMM_FP32, 512, 512, 512, alpha=0.125, beta=1.5,
                           short_probes=1, long_probes=2)
    tried = {tuple(s["plan"]) for s in r["stage1"] if "us" in s}
    assert {(1, v) for v in range(1, 8)} <= tried, tried
    assert px.plan_get(px.GEMM_FP32, [512, 512, 512]) == tuple(r["winner"])
    px.plan_pin(px.GEMM_FP32, [512, 512, 512], None)
