"""Ragged shapes on gfx950: extents that are not multiples of the kernels'
tiles, against the f64 oracle, with a sentinel guard after every output.

The reference's kernels take any M, N that its smallest tile (32) divides and
any K its K tile divides (phobos-bench/src/main.rs:500-508 rejects only tiles
that do not divide M or N; search_choices expands [32, 256] to 32..256); its
own masking check is examples/masking.rs:96-160 (a 96x64 @ 64x100 f32 matmul
of exact integers, a sentinel guard after C).  These kernels take M of any
size, N and K in whole 16-byte chunks (K % 8 for gemm_fp16tc), and flash
attention at any Nq and Nk.

Tolerances as in the full-tile tests: f32 paths 1e-4, f16 paths 2e-2,
exact-integer inputs bit-exact.
"""
import os

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SENTINEL = -12345.0
GUARD = 64  # elements after the output, as in masking.rs


def _norm_err(got, want):
    return np.abs(got - want).max() / np.sqrt(np.mean(want ** 2))


def _gemm_guarded(px, stream, kernel, A, B, C, alpha, beta, f16=False):
    """Runs the gemm with C followed by GUARD sentinel elements; returns C and
    asserts the guard is intact."""
    M, K = A.shape
    N = B.shape[1]
    if f16:
        a, b = oracle.f16_bits(A), oracle.f16_bits(B)
        c = np.concatenate([oracle.f16_bits(C).ravel(),
                            np.full(GUARD, oracle.f16_bits(np.float32([SENTINEL]))[0], np.uint16)])
    else:
        a, b = np.ascontiguousarray(A, np.float32), np.ascontiguousarray(B, np.float32)
        c = np.concatenate([np.ascontiguousarray(C, np.float32).ravel(),
                            np.full(GUARD, SENTINEL, np.float32)])
    da, db, dc = (px.DeviceBuffer.from_array(t) for t in (a, b, c))
    print(f"gemm kernel={kernel} M={M} N={N} K={K}", flush=True)
    px.launch_gemm(stream, kernel, da.ptr, db.ptr, dc.ptr, M, N, K, alpha, beta)
    stream.synchronize()
    if f16:
        out = dc.download(np.uint16, M * N + GUARD)
        assert np.array_equal(out[M * N:], c[M * N:]), "store past C"
        return oracle.f16_to_f32(out[:M * N]).reshape(M, N)
    out = dc.download(np.float32, M * N + GUARD)
    assert np.all(out[M * N:] == SENTINEL), "store past C"
    return out[:M * N].reshape(M, N)


def test_masking_example_exact_at_its_own_shape(px_gpu, stream):
    # masking.rs:96-160: A[96,64] (i%7-3) @ B[64,100] (i%5-2), no padding.
    g = np.load(os.path.join(GOLD, "int_gemm.npz"))
    a, b, want = g["a"], g["b"], g["c"]
    C0 = np.zeros((96, 100), np.float32)
    for kern in (px_gpu.GEMM_FP32, px_gpu.GEMM_FP16TC_FP32ACC, px_gpu.MATMUL):
        got = _gemm_guarded(px_gpu, stream, kern, a, b, C0, 1.0, 0.0 if kern != px_gpu.MATMUL else 1.0)
        assert np.array_equal(got, want), kern
    # gemm_fp16 needs N % 8: pad B with four zero columns (exact)
    b8 = np.zeros((64, 104), np.float32)
    b8[:, :100] = b
    got = _gemm_guarded(px_gpu, stream, px_gpu.GEMM_FP16, a, b8, np.zeros((96, 104), np.float32),
                        1.0, 0.0, f16=True)
    assert np.array_equal(got[:, :100], oracle.f16_round(want)) and not got[:, 100:].any()


# (M, N, K) per kernel: a single row and column chunk; a tile plus one in
# every direction with a partial last K step; a K that is one K step plus a
# partial one.  N and K respect each kernel's chunk multiple.
SHAPES = {
    "fp32": [(1, 4, 4), (257, 516, 1000), (300, 260, 36), (33, 8, 4)],
    "tc": [(1, 4, 8), (257, 516, 1000), (300, 260, 40), (33, 8, 8)],
    "f16": [(1, 8, 8), (257, 520, 1000), (300, 264, 40), (33, 8, 8)],
}


@pytest.mark.parametrize("M,N,K", SHAPES["fp32"])
def test_gemm_fp32_ragged(px_gpu, stream, M, N, K):
    A = oracle.normal_f32(11, M * K).reshape(M, K)
    B = oracle.normal_f32(12, K * N).reshape(K, N)
    C = oracle.normal_f32(13, M * N).reshape(M, N)
    got = _gemm_guarded(px_gpu, stream, px_gpu.GEMM_FP32, A, B, C, 0.125, 1.5)
    assert _norm_err(got, oracle.gemm_full(A, B, C, 0.125, 1.5)) < 1e-5
    got = _gemm_guarded(px_gpu, stream, px_gpu.MATMUL, A, B, C, 0.125, 1.5)   # C += 0.125 A@B
    assert _norm_err(got, oracle.gemm_full(A, B, C, 0.125, 1.0)) < 1e-5


@pytest.mark.parametrize("M,N,K", SHAPES["tc"])
def test_gemm_fp16tc_ragged(px_gpu, stream, M, N, K):
    A = oracle.f16_round(oracle.normal_f32(21, M * K, 1 / np.sqrt(K))).reshape(M, K)
    B = oracle.f16_round(oracle.normal_f32(22, K * N, 1 / np.sqrt(K))).reshape(K, N)
    C = oracle.normal_f32(23, M * N).reshape(M, N)
    got = _gemm_guarded(px_gpu, stream, px_gpu.GEMM_FP16TC_FP32ACC, A, B, C, 1.0, 0.5)
    assert _norm_err(got, oracle.gemm_full(A, B, C, 1.0, 0.5, round16=True)) < 1e-4


@pytest.mark.parametrize("M,N,K", SHAPES["f16"])
def test_gemm_fp16_ragged(px_gpu, stream, M, N, K):
    A = oracle.normal_f32(31, M * K, 1 / np.sqrt(K)).reshape(M, K)
    B = oracle.normal_f32(32, K * N, 1 / np.sqrt(K)).reshape(K, N)
    C = oracle.normal_f32(33, M * N).reshape(M, N)
    got = _gemm_guarded(px_gpu, stream, px_gpu.GEMM_FP16, A, B, C, 0.5, 0.25, f16=True)
    want = oracle.gemm_full(A, B, oracle.f16_round(C), 0.5, 0.25, round16=True)
    assert _norm_err(got, want) < 2e-2


@pytest.mark.parametrize("kern,K", [("GEMM_FP32", 36), ("GEMM_FP16TC_FP32ACC", 40),
                                    ("GEMM_FP16", 40)])
def test_gemm_partial_k_step_reads_nothing_past_k(px_gpu, stream, kern, K):
    # A row r's elements past K are row r+1's first elements.  A NaN at
    # A[1, 0] must reach row 1 of C only, not row 0 through the partial last
    # K step (which would happen if A's chunks past K were multiplied by B's
    # zero rows instead of being read as zeros).
    M, N = 64, 64
    A = oracle.normal_f32(41, M * K, 1 / np.sqrt(K)).reshape(M, K)
    B = oracle.normal_f32(42, K * N, 1 / np.sqrt(K)).reshape(K, N)
    if kern != "GEMM_FP32":
        A, B = oracle.f16_round(A), oracle.f16_round(B)
    A[1, 0] = np.nan
    f16 = kern == "GEMM_FP16"
    got = _gemm_guarded(px_gpu, stream, getattr(px_gpu, kern), A, B, np.zeros((M, N), np.float32),
                        1.0, 0.0, f16=f16)
    assert np.isnan(got[1]).all()
    rest = np.delete(np.arange(M), 1)
    assert np.isfinite(got[rest]).all()
    want = oracle.gemm_full(A[rest], B, None, 1.0, 0.0, round16=kern != "GEMM_FP32")
    assert _norm_err(got[rest], want) < (2e-2 if f16 else 1e-4)


# ------------------------------------------------------------------- flash
TOL = {16: 2e-2, 32: 1e-4}


def _rel(got, want):
    return (np.abs(got - want) / np.maximum(np.abs(want), 0.1)).max()


def _flash_inputs(Nq, Nk, bits, seed, qscale=1.0):
    D = 64
    q = oracle.normal_f32(seed, Nq * D, qscale).reshape(Nq, D)
    k = oracle.normal_f32(seed + 1, Nk * D).reshape(Nk, D)
    v = oracle.normal_f32(seed + 2, Nk * D).reshape(Nk, D)
    if bits == 16:
        q, k, v = oracle.f16_round(q), oracle.f16_round(k), oracle.f16_round(v)
    return q, k, v


def _flash_guarded(px, stream, bits, q, k, v, scale):
    Nq, D = q.shape
    Nk = k.shape[0]
    kern = px.FLASH_FP16 if bits == 16 else px.FLASH_FP32
    if bits == 16:
        up = [oracle.f16_bits(t) for t in (q, k, v)]
        o0 = np.full(Nq * D + GUARD, 0x7bff, np.uint16)  # f16 max, never a softmax output
    else:
        up = [np.ascontiguousarray(t, np.float32) for t in (q, k, v)]
        o0 = np.full(Nq * D + GUARD, SENTINEL, np.float32)
    dq, dk, dv = (px.DeviceBuffer.from_array(t) for t in up)
    do = px.DeviceBuffer.from_array(o0)
    print(f"flash bits={bits} Nq={Nq} Nk={Nk} scale={scale}", flush=True)
    px.launch_flash(stream, kern, dq.ptr, dk.ptr, dv.ptr, do.ptr, Nq, Nk, D, scale)
    stream.synchronize()
    out = do.download(o0.dtype, Nq * D + GUARD)
    assert np.array_equal(out[Nq * D:], o0[Nq * D:]), "store past O"
    if bits == 16:
        return oracle.f16_to_f32(out[:Nq * D]).reshape(Nq, D)
    return out[:Nq * D].reshape(Nq, D)


@pytest.mark.parametrize("bits", [16, 32])
# Nk < 64 (the first block is partial), and Nk with 1, 2, 3 and 4 full blocks
# before a partial one (each stage of the f16 copy ring holds the last block
# once); Nq not a multiple of either precision's workgroup rows.
@pytest.mark.parametrize("Nq,Nk", [(1, 1), (100, 37), (130, 81), (300, 130), (77, 200), (129, 261),
                                   (64, 1000)])
def test_flash_ragged(px_gpu, stream, bits, Nq, Nk):
    q, k, v = _flash_inputs(Nq, Nk, bits, 61)
    got = _flash_guarded(px_gpu, stream, bits, q, k, v, 0.125)
    want = oracle.flash_rows(np.arange(Nq), q, k, v, 0.125)
    assert _rel(got, want) < TOL[bits], _rel(got, want)


@pytest.mark.parametrize("bits", [16, 32])
@pytest.mark.parametrize("scale", [-0.125, 0.0, -1.0])
def test_flash_negative_and_zero_scale(px_gpu, stream, bits, scale):
    # softmax(s * scale) for any sign of scale; scale 0 gives the mean of V.
    # -1.0 makes |s * scale| up to ~34 with the sign flipped.  (At ~200 the
    # f32 rounding of the scores alone exceeds the 1e-4 bound: numpy's f32
    # softmax of the same inputs is 1.9e-4 away from the f64 oracle.)
    Nq, Nk = 128, 200
    q, k, v = _flash_inputs(Nq, Nk, bits, 71)
    got = _flash_guarded(px_gpu, stream, bits, q, k, v, scale)
    want = oracle.flash_rows(np.arange(Nq), q, k, v, scale)
    assert _rel(got, want) < TOL[bits], _rel(got, want)
    if scale == 0.0:
        assert _rel(got, np.broadcast_to(v.astype(np.float64).mean(axis=0), got.shape)) < TOL[bits]


@pytest.mark.parametrize("bits", [16, 32])
def test_flash_partial_block_with_very_negative_scores(px_gpu, stream, bits):
    # Every score is about -72 (q = 3, k = -3 on 64 dims, scale 1/8): masked
    # keys past Nk must not count as score 0 in the row max or as p in l.
    D, Nq, Nk = 64, 128, 100
    q = np.full((Nq, D), 3.0, np.float32)
    k = np.full((Nk, D), -3.0, np.float32)
    k[:, 0] += oracle.normal_f32(81, Nk).astype(np.float32) * 0.5
    v = oracle.normal_f32(82, Nk * D).reshape(Nk, D)
    if bits == 16:
        k, v = oracle.f16_round(k), oracle.f16_round(v)
    got = _flash_guarded(px_gpu, stream, bits, q, k, v, 0.125)
    want = oracle.flash_rows(np.arange(Nq), q, k, v, 0.125)
    assert _rel(got, want) < TOL[bits], _rel(got, want)


@pytest.mark.parametrize("bits", [16, 32])
def test_flash_bh_ragged_equals_per_head(px_gpu, stream, bits):
    px = px_gpu
    BH, Nq, Nk, D = 3, 100, 75, 64
    q = oracle.normal_f32(91, BH * Nq * D).reshape(BH, Nq, D)
    k = oracle.normal_f32(92, BH * Nk * D).reshape(BH, Nk, D)
    v = oracle.normal_f32(93, BH * Nk * D).reshape(BH, Nk, D)
    if bits == 16:
        q, k, v = oracle.f16_round(q), oracle.f16_round(k), oracle.f16_round(v)
        up = [oracle.f16_bits(t) for t in (q, k, v)]
        esz, dt = 2, np.uint16
    else:
        up = [np.ascontiguousarray(t, np.float32) for t in (q, k, v)]
        esz, dt = 4, np.uint32
    dq, dk, dv = (px.DeviceBuffer.from_array(t) for t in up)
    do = px.DeviceBuffer(BH * Nq * D * esz)
    kb = px.FLASH_FP16_BH if bits == 16 else px.FLASH_FP32_BH
    k1 = px.FLASH_FP16 if bits == 16 else px.FLASH_FP32
    print(f"flash_bh bits={bits} BH={BH} Nq={Nq} Nk={Nk}", flush=True)
    px.launch_flash_bh(stream, kb, dq.ptr, dk.ptr, dv.ptr, do.ptr, BH, Nq, Nk, D, 0.125)
    stream.synchronize()
    batched = do.download(dt, BH * Nq * D).reshape(BH, Nq * D)
    do1 = px.DeviceBuffer(Nq * D * esz)
    for h in range(BH):
        px.launch_flash(stream, k1, dq.ptr + h * Nq * D * esz, dk.ptr + h * Nk * D * esz,
                        dv.ptr + h * Nk * D * esz, do1.ptr, Nq, Nk, D, 0.125)
        stream.synchronize()
        assert np.array_equal(do1.download(dt, Nq * D), batched[h]), h
    if bits == 16:
        got = oracle.f16_to_f32(batched.astype(np.uint16).ravel()).reshape(BH, Nq, D)
    else:
        got = batched.view(np.float32).reshape(BH, Nq, D)
    want = np.stack([oracle.flash_rows(np.arange(Nq), q[h], k[h], v[h], 0.125) for h in range(BH)])
    assert _rel(got, want) < TOL[bits]
