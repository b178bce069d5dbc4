"""Shape-adaptive launches: GEMMs split over K and flash attention split over
the keys when the problem has too few tiles or query blocks to fill the GPU
(phx_split_plan), against the f64 oracle.

The reference picks per-shape tile sizes with its autotuner
(phobos-bench/src/autotune.rs:98-192) instead; its kernels' arithmetic is the
same at every tiling, and so is this backend's: a split only changes the
order of the f32 sums.  Tolerances as in the full-tile tests: f32 paths
1e-4 (relative, floored at 1% of the RMS) or 1e-5 (RMS-normalised), f16
paths 2e-2 (RMS-normalised); exact-integer inputs bit-exact; flash by the
reference's metric |err| / max(|want|, 0.1) (main.rs:912-917).
"""
import os

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

SENTINEL = -12345.0
GUARD = 64


def _norm_err(got, want):
    return np.abs(got - want).max() / np.sqrt(np.mean(want ** 2))


class _Env:
    """Sets an environment variable for the duration of a with-block."""

    def __init__(self, name, value):
        self.name, self.value = name, value

    def __enter__(self):
        self.old = os.environ.get(self.name)
        os.environ[self.name] = str(self.value)

    def __exit__(self, *a):
        if self.old is None:
            os.environ.pop(self.name, None)
        else:
            os.environ[self.name] = self.old


def _gemm(px, stream, kern, A, B, C, alpha, beta):
    """C followed by GUARD sentinels; returns C after the launch and checks
    the guard."""
    f16 = kern == px.GEMM_FP16
    M, K = A.shape
    N = B.shape[1]
    if f16:
        a, b = oracle.f16_bits(A), oracle.f16_bits(B)
        c = np.concatenate([oracle.f16_bits(C).ravel(),
                            oracle.f16_bits(np.full(GUARD, SENTINEL, np.float32))])
    else:
        a, b = A, B
        c = np.concatenate([C.ravel(), np.full(GUARD, SENTINEL, np.float32)])
    da, db, dc = (px.DeviceBuffer.from_array(np.ascontiguousarray(t)) for t in (a, b, c))
    px.launch_gemm(stream, kern, da.ptr, db.ptr, dc.ptr, M, N, K, alpha, beta)
    stream.synchronize()
    if f16:
        out = oracle.f16_to_f32(dc.download(np.uint16, M * N + GUARD))
    else:
        out = dc.download(np.float32, M * N + GUARD)
    guard = oracle.f16_round(np.full(GUARD, SENTINEL, np.float32)) if f16 else SENTINEL
    assert np.all(out[M * N:] == guard), "write past C"
    return out[:M * N].reshape(M, N)


def _check(kern_name, got, want):
    if kern_name == "GEMM_FP32":
        floor = 1e-2 * np.sqrt(np.mean(want ** 2))
        rel = np.abs(got - want) / np.maximum(np.abs(want), floor)
        assert rel.max() < 1e-4, rel.max()
    else:
        assert _norm_err(got, want) < 2e-2


GEMM_SHAPES = [(512, 512, 512), (1024, 1024, 1024), (256, 512, 4096), (300, 200, 5000),
               (64, 64, 8192)]


@pytest.mark.parametrize("kern_name", ["GEMM_FP32", "GEMM_FP16TC_FP32ACC", "GEMM_FP16"])
@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_small_gemms_against_oracle(px_gpu, stream, kern_name, M, N, K):
    px = px_gpu
    kern = getattr(px, kern_name)
    sp, ws = px.split_plan(kern, [M, N, K])
    if kern_name == "GEMM_FP32":
        # the 64 x 64 tiling where it fills the GPU at this K, else the split
        small = px.plan_get(kern, [M, N, K])[1] == 7
        assert (sp == 1) == small and ws == (0 if small else sp * M * N * 4), (sp, ws)
    elif K >= 4096:
        assert sp > 1 and ws == sp * M * N * 4, (sp, ws)
    A = oracle.normal_f32(21, M * K, 1 / np.sqrt(K)).reshape(M, K)
    B = oracle.normal_f32(22, K * N, 1 / np.sqrt(K)).reshape(K, N)
    C = oracle.normal_f32(23, M * N).reshape(M, N)
    r16 = kern_name != "GEMM_FP32"
    if r16:
        A, B, C = oracle.f16_round(A), oracle.f16_round(B), oracle.f16_round(C)
    got = _gemm(px, stream, kern, A, B, C, 0.5, 0.25)
    want = oracle.gemm_full(A, B, C, 0.5, 0.25, round16=r16)
    _check(kern_name, got, want)


@pytest.mark.parametrize("kern_name", ["GEMM_FP32", "GEMM_FP16TC_FP32ACC", "GEMM_FP16"])
def test_split_gemm_exact_on_integers(px_gpu, stream, kern_name):
    # Small-integer operands (the exact-integer idea of masking.rs:108-110):
    # every partial sum is an integer far below 2^24, so any split and any
    # summation order gives the f64 result exactly; the outputs also stay
    # below 2048, where every integer is an f16.
    px = px_gpu
    kern = getattr(px, kern_name)
    M, N, K = 128, 256, 2048
    rng = np.random.default_rng(5)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-1, 2, (K, N)).astype(np.float32)
    assert px.split_plan(kern, [M, N, K])[0] > 1
    C = np.zeros((M, N), np.float32)
    got = _gemm(px, stream, kern, A, B, C, 1.0, 0.0)
    want = oracle.gemm_full(A, B, None, 1.0, 0.0)
    assert 100 < np.abs(want).max() < 2048
    assert np.array_equal(got.astype(np.float64), want)


@pytest.mark.parametrize("kern_name", ["GEMM_FP32", "GEMM_FP16TC_FP32ACC", "GEMM_FP16"])
def test_forced_splits_agree(px_gpu, stream, kern_name):
    # The same GEMM with the split off, at the automatic choice and at the
    # maximum: each within the kernel's bound of the oracle.
    px = px_gpu
    kern = getattr(px, kern_name)
    M, N, K = 256, 256, 2048
    r16 = kern_name != "GEMM_FP32"
    A = oracle.normal_f32(31, M * K, 1 / np.sqrt(K)).reshape(M, K)
    B = oracle.normal_f32(32, K * N, 1 / np.sqrt(K)).reshape(K, N)
    C = oracle.normal_f32(33, M * N).reshape(M, N)
    if r16:
        A, B, C = oracle.f16_round(A), oracle.f16_round(B), oracle.f16_round(C)
    want = oracle.gemm_full(A, B, C, 1.0, -0.5, round16=r16)
    for sp in (1, 16, None):
        if sp is None:
            got = _gemm(px, stream, kern, A, B, C, 1.0, -0.5)
        else:
            with _Env("PHX_GEMM_SPLIT", sp):
                assert px.split_plan(kern, [M, N, K])[0] == sp
                got = _gemm(px, stream, kern, A, B, C, 1.0, -0.5)
        _check(kern_name, got, want)


def _flash_inputs(BH, Nq, Nk, bits, seed):
    D = 64
    q = oracle.normal_f32(seed, BH * Nq * D).reshape(BH, Nq, D)
    k = oracle.normal_f32(seed + 1, BH * Nk * D).reshape(BH, Nk, D)
    v = oracle.normal_f32(seed + 2, BH * Nk * D).reshape(BH, Nk, D)
    if bits == 16:
        q, k, v = (oracle.f16_round(t) for t in (q, k, v))
    return q, k, v


def _upload(px, t, bits):
    if bits == 16:
        return px.DeviceBuffer.from_array(oracle.f16_bits(t))
    return px.DeviceBuffer.from_array(np.ascontiguousarray(t, np.float32))


def _flash_rel(got, want):
    return (np.abs(got - want) / np.maximum(np.abs(want), 0.1)).max()


TOL = {16: 2e-2, 32: 1e-4}


@pytest.mark.parametrize("bits", [16, 32])
@pytest.mark.parametrize("Nq,Nk,scale", [(4096, 4096, 0.125), (1000, 4133, 0.125),
                                         (300, 2048, -0.2), (64, 16384, 0.125)])
def test_one_head_flash_split_over_keys(px_gpu, stream, bits, Nq, Nk, scale):
    # The .ph entry's one-head launch (main.rs:334-371) at shapes with a
    # handful of query blocks: the keys are split so the launch fills the GPU.
    px = px_gpu
    D = 64
    sp, ws = px.split_plan(px.FLASH_FP16 if bits == 16 else px.FLASH_FP32, [Nq, Nk, D])
    assert sp > 1 and ws == sp * Nq * (D + 2) * 4
    q, k, v = _flash_inputs(1, Nq, Nk, bits, 41)
    dq, dk, dv = (_upload(px, t[0], bits) for t in (q, k, v))
    esz = 2 if bits == 16 else 4
    do = px.DeviceBuffer(Nq * D * esz + 256)
    do.upload(np.full((Nq * D * esz + 256) // 4, 0x7fc00001, np.uint32))  # NaN sentinels
    kern = px.FLASH_FP16 if bits == 16 else px.FLASH_FP32
    px.launch_flash(stream, kern, dq.ptr, dk.ptr, dv.ptr, do.ptr, Nq, Nk, D, scale)
    stream.synchronize()
    raw = do.download(np.uint32, (Nq * D * esz + 256) // 4)
    assert np.all(raw[Nq * D * esz // 4:] == 0x7fc00001), "write past O"
    if bits == 16:
        got = oracle.f16_to_f32(do.download(np.uint16, Nq * D)).reshape(Nq, D)
    else:
        got = do.download(np.float32, (Nq, D))
    rows = np.unique(np.linspace(0, Nq - 1, 48).astype(np.int64))
    want = oracle.flash_rows(rows, q[0], k[0], v[0], scale)
    assert _flash_rel(got[rows], want) < TOL[bits]


@pytest.mark.parametrize("bits", [16, 32])
def test_bh_flash_split_matches_unsplit(px_gpu, stream, bits):
    # A small batched launch (4 heads x 512 queries) split over the keys, the
    # same launch with the split off, and the oracle.
    px = px_gpu
    BH, Nq, Nk, D = 4, 512, 4096, 64
    kern = px.FLASH_FP16_BH if bits == 16 else px.FLASH_FP32_BH
    assert px.split_plan(kern, [BH, Nq, Nk, D])[0] > 1
    q, k, v = _flash_inputs(BH, Nq, Nk, bits, 51)
    dq, dk, dv = (_upload(px, t, bits) for t in (q, k, v))
    esz = 2 if bits == 16 else 4
    outs = []
    for force in (None, 1):
        do = px.DeviceBuffer(BH * Nq * D * esz)
        if force is None:
            px.launch_flash_bh(stream, kern, dq.ptr, dk.ptr, dv.ptr, do.ptr, BH, Nq, Nk, D, 0.125)
        else:
            with _Env("PHX_FLASH_SPLIT", force):
                px.launch_flash_bh(stream, kern, dq.ptr, dk.ptr, dv.ptr, do.ptr, BH, Nq, Nk, D,
                                   0.125)
        stream.synchronize()
        if bits == 16:
            outs.append(oracle.f16_to_f32(do.download(np.uint16, BH * Nq * D)).reshape(BH, Nq, D))
        else:
            outs.append(do.download(np.float32, (BH, Nq, D)))
    rows = np.array([0, 1, 255, 256, 511])
    for h in range(BH):
        want = oracle.flash_rows(rows, q[h], k[h], v[h], 0.125)
        for o in outs:
            assert _flash_rel(o[h][rows], want) < TOL[bits]
    assert _flash_rel(outs[0], outs[1]) < TOL[bits]


@pytest.mark.parametrize("kern_name", ["GEMM_FP16TC_FP32ACC"])
@pytest.mark.parametrize("split", [1, 3])
@pytest.mark.parametrize("M,N,K", [(512, 768, 2048), (1024, 256, 96), (256, 256, 32),
                                   (300, 200, 104), (520, 388, 1000), (257, 260, 40),
                                   (1000, 1000, 1000)])
def test_eight_wave_kernel_matches_one_wave_kernel(px_gpu, stream, kern_name, M, N, K, split):
    # gemm_fp16tc_fp32acc launches run the eight-wave kernels (gemm_w8, two
    # waves per SIMD, and gemm_w8_splitk); PHX_GEMM_W8=0 runs the one-wave
    # kernels.  Whole tiles and ragged edges (rows, columns and the last K
    # step), unsplit and split in three: both sum each output's K products in
    # the same order, so they agree bit for bit, and both meet the oracle.
    # The guard past C catches stores beyond the last row.
    px = px_gpu
    kern = getattr(px, kern_name)
    A = oracle.f16_round(oracle.normal_f32(61, M * K, 1 / np.sqrt(K))).reshape(M, K)
    B = oracle.f16_round(oracle.normal_f32(62, K * N, 1 / np.sqrt(K))).reshape(K, N)
    C = oracle.normal_f32(63, M * N).reshape(M, N)
    outs = []
    with _Env("PHX_GEMM_SPLIT", split):
        for w8 in (1, 0):
            with _Env("PHX_GEMM_W8", w8):
                outs.append(_gemm(px, stream, kern, A, B, C, 0.75, -0.5))
    if kern_name == "GEMM_FP16":
        C = oracle.f16_round(C)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    want = oracle.gemm_full(A, B, C, 0.75, -0.5, round16=True)
    _check(kern_name, outs[0], want)
