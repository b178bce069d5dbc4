"""GEMM leaf kernels on gfx950 vs the f64 oracle.

Tolerances (written here):
  gemm_fp32 / matmul:      max relative error <= 1e-4, rel = |got-want| /
                           max(|want|, floor) with the reference's floor of
                           f64::MIN_POSITIVE (main.rs:398-402) on Lcg inputs
                           (all-negative, so no cancellation) and an RMS-
                           normalised 1e-5 bound on zero-mean inputs;
                           bit-exact on the exact-integer fixture.
  gemm_fp16tc / gemm_fp16: max |got-want| / rms(want) <= 2e-2 ("normalised
                           outputs"), want = f64 over f16-rounded inputs
                           (main.rs:417-427); exact on integer data (tc).
"""
import os

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _gemm(px, stream, kernel, A, B, C, alpha, beta, f16=False):
    M, K = A.shape
    N = B.shape[1]
    if f16:
        A, B, C = oracle.f16_bits(A).reshape(M, K), oracle.f16_bits(B).reshape(K, N), \
            oracle.f16_bits(C).reshape(M, N)
    da, db, dc = (px.DeviceBuffer.from_array(t) for t in (A, B, C))
    px.launch_gemm(stream, kernel, da.ptr, db.ptr, dc.ptr, M, N, K, alpha, beta)
    stream.synchronize()
    if f16:
        return oracle.f16_to_f32(dc.download(np.uint16, M * N)).reshape(M, N)
    return dc.download(np.float32, (M, N))


def _norm_err(got, want):
    return np.abs(got - want).max() / np.sqrt(np.mean(want ** 2))


@pytest.mark.parametrize("M,N,K", [(128, 128, 32), (256, 384, 96), (512, 256, 1024)])
def test_gemm_fp32_full_small(px_gpu, stream, M, N, K):
    A = oracle.lcg_f32(1, M * K).reshape(M, K)
    B = oracle.lcg_f32(2, K * N).reshape(K, N)
    C = oracle.lcg_f32(3, M * N).reshape(M, N)
    got = _gemm(px_gpu, stream, px_gpu.GEMM_FP32, A, B, C, 0.125, 1.5)
    want = oracle.gemm_full(A, B, C, 0.125, 1.5)
    # 0.125*dot + 1.5*c can cancel at small K, so the relative error is floored
    # at 1% of the output RMS (at 4096^3 nothing cancels and the floor is unused).
    floor = 1e-2 * np.sqrt(np.mean(want ** 2))
    rel = np.abs(got - want) / np.maximum(np.abs(want), floor)
    assert rel.max() < 1e-4, rel.max()
    # zero-mean operands (cancellation): RMS-normalised bound
    A2 = oracle.normal_f32(4, M * K).reshape(M, K)
    B2 = oracle.normal_f32(5, K * N).reshape(K, N)
    got = _gemm(px_gpu, stream, px_gpu.GEMM_FP32, A2, B2, C, 0.125, 1.5)
    assert _norm_err(got, oracle.gemm_full(A2, B2, C, 0.125, 1.5)) < 1e-5


def test_gemm_fp32_beta_zero_and_alpha(px_gpu, stream):
    M = N = K = 256
    A = oracle.lcg_f32(7, M * K).reshape(M, K)
    B = oracle.lcg_f32(8, K * N).reshape(K, N)
    C = oracle.lcg_f32(9, M * N).reshape(M, N)
    got = _gemm(px_gpu, stream, px_gpu.GEMM_FP32, A, B, C, -2.0, 0.0)
    want = oracle.gemm_full(A, B, None, -2.0, 0.0)
    assert (np.abs(got - want) / np.abs(want)).max() < 1e-4


def test_gemm_integer_fixture_exact(px_gpu, stream):
    # masking.rs:108-110-style integers: any summation order is exact.
    g = np.load(os.path.join(GOLD, "int_gemm.npz"))
    a, b = g["a"], g["b"]
    # pad to the kernels' tile multiples with zeros (exact)
    M, K, N = 256, 256, 256
    A = np.zeros((M, K), np.float32)
    A[:96, :64] = a
    B = np.zeros((K, N), np.float32)
    B[:64, :100] = b
    C0 = np.zeros((M, N), np.float32)
    want = g["c"]
    for kern in (px_gpu.GEMM_FP32, px_gpu.GEMM_FP16TC_FP32ACC):
        got = _gemm(px_gpu, stream, kern, A, B, C0, 1.0, 0.0)
        assert np.array_equal(got[:96, :100], want), kern
        assert not got[96:].any() and not got[:, 100:].any()
    got = _gemm(px_gpu, stream, px_gpu.GEMM_FP16, A, B, C0, 1.0, 0.0, f16=True)
    assert np.array_equal(got[:96, :100], oracle.f16_round(want))


# K = 32 and 96 are one and three K steps (the pipelines' tail paths), 320 is
# ten; 768 columns are three tile columns.
@pytest.mark.parametrize("M,N,K", [(256, 256, 32), (256, 256, 64), (256, 512, 96), (512, 768, 320),
                                   (256, 512, 2048)])
def test_gemm_fp16tc_full_small(px_gpu, stream, M, N, K):
    A = oracle.f16_round(oracle.normal_f32(1, M * K, 1 / np.sqrt(K))).reshape(M, K)
    B = oracle.f16_round(oracle.normal_f32(2, K * N, 1 / np.sqrt(K))).reshape(K, N)
    C = np.zeros((M, N), np.float32)
    got = _gemm(px_gpu, stream, px_gpu.GEMM_FP16TC_FP32ACC, A, B, C, 1.0, 0.0)
    want = oracle.gemm_full(A, B, None, 1.0, 0.0, round16=True)
    assert _norm_err(got, want) < 2e-2
    # f32 accumulate of exact f16 products: far inside the bound
    assert _norm_err(got, want) < 1e-4


def test_gemm_fp16tc_rounds_f32_inputs_to_f16(px_gpu, stream):
    M = N = K = 256
    A = oracle.lcg_f32(1, M * K).reshape(M, K)          # not f16-exact
    B = oracle.lcg_f32(2, K * N).reshape(K, N)
    C = oracle.lcg_f32(3, M * N).reshape(M, N)
    got = _gemm(px_gpu, stream, px_gpu.GEMM_FP16TC_FP32ACC, A, B, C, 1.0, 1.0)
    want16 = oracle.gemm_full(A, B, C, 1.0, 1.0, round16=True)
    want32 = oracle.gemm_full(A, B, C, 1.0, 1.0, round16=False)
    e16 = np.abs(got - want16).max()
    e32 = np.abs(got - want32).max()
    assert e16 < 1e-3 and e16 < e32 / 10


@pytest.mark.parametrize("M,N,K", [(256, 256, 32), (256, 256, 64), (512, 256, 96), (768, 512, 160),
                                   (512, 256, 1024)])
def test_gemm_fp16_full_small(px_gpu, stream, M, N, K):
    A = oracle.normal_f32(3, M * K, 1 / np.sqrt(K)).reshape(M, K)
    B = oracle.normal_f32(4, K * N, 1 / np.sqrt(K)).reshape(K, N)
    C = oracle.normal_f32(5, M * N).reshape(M, N)
    got = _gemm(px_gpu, stream, px_gpu.GEMM_FP16, A, B, C, 0.5, 0.25, f16=True)
    Cr = oracle.f16_round(C)
    want = oracle.gemm_full(A, B, Cr, 0.5, 0.25, round16=True)
    assert _norm_err(got, want) < 2e-2
    # the reference's f16-accumulate model, informational distance
    i, j = 3, 5
    ref16 = oracle.gemm_fp16acc_point(i, j, A, B, Cr, 0.5, 0.25)
    assert abs(ref16 - got[i, j]) < 0.15 * max(abs(want[i, j]), np.sqrt(K) / 3)


def _baseline_inputs(px):
    M = N = K = 4096
    A = oracle.f16_round(oracle.normal_f32(1, M * K, 1 / 64.0)).reshape(M, K)
    B = oracle.f16_round(oracle.normal_f32(2, K * N, 1 / 64.0)).reshape(K, N)
    return A, B


def test_gemm_fp16tc_baseline_config_sampled(px_gpu, stream):
    A, B = _baseline_inputs(px_gpu)
    C = np.zeros((4096, 4096), np.float32)
    got = _gemm(px_gpu, stream, px_gpu.GEMM_FP16TC_FP32ACC, A, B, C, 1.0, 0.0)
    r, c = oracle.sample_points(4096, 4096, 256)
    want = oracle.gemm_points(r, c, A, B, None, 1.0, 0.0, round16=True)
    g = got[r.astype(int), c.astype(int)]
    assert np.abs(g - want).max() < 1e-4          # |C| ~ N(0,1): absolute = normalised
    assert np.isfinite(got).all()
    # checksum of checksums: column sums of C equal (row-sum of A) @ B in f64
    colsum = got.astype(np.float64).sum(axis=0)
    want_cs = A.astype(np.float64).sum(axis=0) @ B.astype(np.float64)
    assert np.abs(colsum - want_cs).max() < 1e-3


def test_gemm_fp16_baseline_config_sampled(px_gpu, stream):
    A, B = _baseline_inputs(px_gpu)
    C = np.zeros((4096, 4096), np.float32)
    got = _gemm(px_gpu, stream, px_gpu.GEMM_FP16, A, B, C, 1.0, 0.0, f16=True)
    r, c = oracle.sample_points(4096, 4096, 256)
    want = oracle.gemm_points(r, c, A, B, None, 1.0, 0.0, round16=True)
    rms = np.sqrt(np.mean(want ** 2))
    assert np.abs(got[r.astype(int), c.astype(int)] - want).max() / rms < 2e-2


def test_gemm_fp32_baseline_config_sampled(px_gpu, stream):
    M = N = K = 4096
    A = px_gpu.lcg_f32(1, M * K).reshape(M, K)
    B = px_gpu.lcg_f32(2, K * N).reshape(K, N)
    C = px_gpu.lcg_f32(3, M * N).reshape(M, N)
    got = _gemm(px_gpu, stream, px_gpu.GEMM_FP32, A, B, C, 0.125, 1.5)
    r, c = oracle.sample_points(M, N, 64)
    want = oracle.gemm_points(r, c, A, B, C, 0.125, 1.5)
    g = got[r.astype(int), c.astype(int)]
    rel = np.abs(g - want) / np.maximum(np.abs(want), np.finfo(np.float64).tiny)
    assert rel.max() < 1e-4, rel.max()


def test_gemm_fp16_operand_past_4gib(px_gpu, stream):
    # A of 2^21 x 1024 f16 (4 GiB): tiles past the 4 GiB mark address A
    # through 64-bit tile bases.  A's rows repeat with period 3001 (built by
    # device copies), which does not divide the 2^21 rows, so a row fetched
    # through a wrapped 32-bit offset would come from the wrong phase.
    px = px_gpu
    M, N, K, P = 1 << 21, 256, 1024, 3001
    Ap = oracle.f16_round(oracle.normal_f32(61, P * K, 1 / 32)).reshape(P, K)
    B = oracle.f16_round(oracle.normal_f32(62, K * N, 1 / 32)).reshape(K, N)
    dA = px.DeviceBuffer(M * K * 2)
    blk = oracle.f16_bits(Ap)
    dA.upload(blk)
    rows = P
    while rows < M:  # double the filled prefix
        m = min(rows, M - rows)
        assert px.lib().phx_memcpy_d2d(dA.ptr + rows * K * 2, dA.ptr, m * K * 2) == 0
        rows += m
    dB = px.DeviceBuffer.from_array(oracle.f16_bits(B))
    dC = px.DeviceBuffer(M * N * 2)
    print(f"gemm_fp16 M={M} N={N} K={K}", flush=True)
    px.launch_gemm(stream, px.GEMM_FP16, dA, dB, dC, M, N, K, 1.0, 0.0)
    stream.synchronize()
    want = oracle.gemm_full(Ap, B, None, 1.0, 0.0, round16=True)   # one period
    rms = np.sqrt(np.mean(want ** 2))
    out = np.empty(N, np.uint16)
    for r in [0, 1, P - 1, P, (1 << 20) + 7, (1 << 21) - 4097, M - 2, M - 1]:
        assert px.lib().phx_memcpy_d2h(out.ctypes.data, dC.ptr + r * N * 2, N * 2) == 0
        got = oracle.f16_to_f32(out)
        assert np.abs(got - want[r % P]).max() / rms < 2e-2, r
    for b in (dA, dB, dC):
        b.free()


# Every output of the BASELINE configs against the CPU's f32 GEMM (oracle
# sgemm_f32, OpenMP; itself checked against the f64 oracle across its
# blocking in test_oracle.py).  The sampled tests above hold the reference's
# f64 points; these cover all 16.7 M outputs.
def test_gemm_fp32_baseline_config_every_output(px_gpu, stream):
    M = N = K = 4096
    A = px_gpu.lcg_f32(1, M * K).reshape(M, K)
    B = px_gpu.lcg_f32(2, K * N).reshape(K, N)
    C = px_gpu.lcg_f32(3, M * N).reshape(M, N)
    got = _gemm(px_gpu, stream, px_gpu.GEMM_FP32, A, B, C, 0.125, 1.5)
    want = oracle.sgemm_f32(0.125, A, B, 1.5, C)
    assert _norm_err(got, want) < 2e-5  # two f32 summation orders


def test_gemm_fp16tc_baseline_config_every_output(px_gpu, stream):
    A, B = _baseline_inputs(px_gpu)
    C = np.zeros((4096, 4096), np.float32)
    got = _gemm(px_gpu, stream, px_gpu.GEMM_FP16TC_FP32ACC, A, B, C, 1.0, 0.0)
    want = oracle.sgemm_f32(1.0, A, B, 0.0, C)
    assert np.abs(got - want).max() < 1e-4  # |C| ~ N(0,1): absolute = normalised


def test_gemm_fp16_baseline_config_every_output(px_gpu, stream):
    # both sides sum in f32 and round once to f16, so every output is within
    # one f16 step (at either value) of the f32 oracle's rounded result, or,
    # near zero where the two f32 sums' own rounding (~1e-7 here) exceeds
    # the f16 step, within 1e-5 of the RMS
    A, B = _baseline_inputs(px_gpu)
    C = np.zeros((4096, 4096), np.float32)
    got = _gemm(px_gpu, stream, px_gpu.GEMM_FP16, A, B, C, 1.0, 0.0, f16=True)
    want = oracle.f16_round(oracle.sgemm_f32(1.0, A, B, 0.0, C))
    assert _norm_err(got, want) < 2e-2
    step = np.maximum(np.spacing(np.abs(want).astype(np.float16)),
                      np.spacing(np.abs(got).astype(np.float16))).astype(np.float32)
    bad = np.abs(got - want) > np.maximum(step, 1e-5 * np.sqrt(np.mean(want ** 2)))
    assert not bad.any(), (int(bad.sum()), got[bad][:5], want[bad][:5])


@pytest.mark.parametrize("M,N,K", [(128, 128, 32), (256, 384, 96), (512, 256, 1024), (300, 200, 100)])
def test_gemm_fp32_small_strict_relative(px_gpu, stream, M, N, K):
    # non-negative operands and scalars: no output cancels, so every output
    # is held to BASELINE's 1e-4 relative error with the reference's own
    # floor, f64::MIN_POSITIVE (main.rs:398-402), at the built-in plan and at
    # every tiling
    px = px_gpu
    A = np.abs(oracle.lcg_f32(11, M * K)).reshape(M, K)
    B = np.abs(oracle.lcg_f32(12, K * N)).reshape(K, N)
    C = np.abs(oracle.lcg_f32(13, M * N)).reshape(M, N)
    want = oracle.gemm_full(A, B, C, 0.125, 1.5)
    for variant in [None] + list(range(8)):
        if variant is not None:
            px.plan_pin(px.GEMM_FP32, [M, N, K], 1, variant)
        try:
            got = _gemm(px, stream, px.GEMM_FP32, A, B, C, 0.125, 1.5)
        finally:
            px.plan_pin(px.GEMM_FP32, [M, N, K], None)
        rel = np.abs(got - want) / np.maximum(np.abs(want), np.finfo(np.float64).tiny)
        assert rel.max() < 1e-4, (variant, rel.max())
