"""Seeded random shapes for every GEMM and both flash precisions, against the
f64 oracle, with sentinel guards after each output: extents anywhere in the
shape contract (any M; N and K in whole 16-byte chunks, K % 8 for the f16
GEMMs and gemm_fp16tc, N % 8 for gemm_fp16; any Nq and Nk), random alpha, beta
and scale; every third case pins a random split of the reduction (2-5 K or
key chunks) through phx_plan_pin, the rest run the plan the runtime picks.
Bounds as in the fixed-shape tests: max error over the output's RMS below
1e-5 for gemm_fp32, 1e-4 for gemm_fp16tc_fp32acc, 2e-2 for gemm_fp16; flash
|err| / max(|want|, 0.1) within 1e-4 (f32) or 2e-2 (f16) (main.rs:912-917)."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

SENTINEL = -12345.0
GUARD = 64
RULES = {"GEMM_FP32": (4, 4), "GEMM_FP16TC_FP32ACC": (4, 8), "GEMM_FP16": (8, 8)}  # N, K multiples


def _cases(name, n=24):
    rng = np.random.default_rng(sum(map(ord, name)))
    nm, km = RULES[name]
    out = []
    for _ in range(n):
        M = int(rng.integers(1, 321))
        N = nm * int(rng.integers(1, 320 // nm + 1))
        K = km * int(rng.integers(1, 1200 // km + 1))
        alpha = float(rng.uniform(-2, 2))
        beta = float(rng.choice([0.0, float(rng.uniform(-2, 2))]))
        split = int(rng.integers(2, 6)) if len(out) % 3 == 2 else 0
        out.append((M, N, K, alpha, beta, split))
    return out


@pytest.fixture(autouse=True)
def _no_pins_left(px_gpu):
    yield
    px_gpu.plan_unpin_all()


@pytest.mark.parametrize("name", list(RULES))
def test_random_gemm_shapes(px_gpu, stream, name):
    px = px_gpu
    kern = getattr(px, name)
    f16 = name == "GEMM_FP16"
    r16 = name != "GEMM_FP32"
    for i, (M, N, K, alpha, beta, split) in enumerate(_cases(name)):
        assert px.check_shape(kern, [M, N, K]) == 0, (M, N, K)
        px.plan_pin(kern, [M, N, K], split if split else None)
        A = oracle.normal_f32(100 + i, M * K, 1 / np.sqrt(K)).reshape(M, K)
        B = oracle.normal_f32(200 + i, K * N, 1 / np.sqrt(K)).reshape(K, N)
        C = oracle.normal_f32(300 + i, M * N).reshape(M, N)
        if r16:
            A, B, C = oracle.f16_round(A), oracle.f16_round(B), oracle.f16_round(C)
        if f16:
            a, b = oracle.f16_bits(A), oracle.f16_bits(B)
            guard = oracle.f16_bits(np.float32([SENTINEL]))[0]
            c = np.concatenate([oracle.f16_bits(C).ravel(), np.full(GUARD, guard, np.uint16)])
        else:
            a, b = np.ascontiguousarray(A), np.ascontiguousarray(B)
            c = np.concatenate([np.ascontiguousarray(C).ravel(), np.full(GUARD, SENTINEL, np.float32)])
        da, db, dc = (px.DeviceBuffer.from_array(t) for t in (a, b, c))
        print(f"{name} M={M} N={N} K={K} plan={px.plan_get(kern, [M, N, K])}", flush=True)
        px.launch_gemm(stream, kern, da, db, dc, M, N, K, alpha, beta)  # sizes host-checked
        stream.synchronize()
        raw = dc.download(c.dtype, M * N + GUARD)
        assert np.array_equal(raw[M * N:], c[M * N:]), f"store past C at {(M, N, K)}"
        got = (oracle.f16_to_f32(raw[:M * N]) if f16 else raw[:M * N]).reshape(M, N)
        want = oracle.gemm_full(A, B, C, alpha, beta, round16=r16)
        rms = np.sqrt(np.mean(want ** 2))
        err = np.abs(got - want).max() / rms
        assert err < (1e-5 if name == "GEMM_FP32" else 1e-4 if not f16 else 2e-2), (M, N, K, err)


@pytest.mark.parametrize("variant", range(1, 8))
def test_random_gemm_fp32_tiling_shapes(px_gpu, stream, variant):
    # every other gemm_fp32 tiling (TILE_M x TILE_N x TILE_K), pinned, over
    # 12 seeded shapes of the contract, a guard after C, the gemm_fp32 bound
    px = px_gpu
    for i, (M, N, K, alpha, beta, _) in enumerate(_cases("GEMM_FP32", 12 + variant)[variant:]):
        px.plan_pin(px.GEMM_FP32, [M, N, K], 1, variant)
        A = oracle.normal_f32(400 + i, M * K, 1 / np.sqrt(K)).reshape(M, K)
        B = oracle.normal_f32(500 + i, K * N, 1 / np.sqrt(K)).reshape(K, N)
        C = oracle.normal_f32(600 + i, M * N).reshape(M, N)
        c = np.concatenate([C.ravel(), np.full(GUARD, SENTINEL, np.float32)])
        da, db, dc = (px.DeviceBuffer.from_array(np.ascontiguousarray(t)) for t in (A, B, c))
        print(f"tiling {px.GEMM_FP32_TILINGS[variant]} M={M} N={N} K={K}", flush=True)
        px.launch_gemm(stream, px.GEMM_FP32, da, db, dc, M, N, K, alpha, beta)
        stream.synchronize()
        raw = dc.download(np.float32, M * N + GUARD)
        assert np.array_equal(raw[M * N:], c[M * N:]), f"store past C at {(M, N, K)}"
        want = oracle.gemm_full(A, B, C, alpha, beta)
        err = np.abs(raw[:M * N].reshape(M, N) - want).max() / np.sqrt(np.mean(want ** 2))
        assert err < 1e-5, (variant, M, N, K, err)


@pytest.mark.parametrize("bits", [16, 32])
def test_random_flash_shapes(px_gpu, stream, bits):
    px = px_gpu
    kern = px.FLASH_FP16_BH if bits == 16 else px.FLASH_FP32_BH
    rng = np.random.default_rng(4000 + bits)
    D = 64
    for i in range(12):
        BH = int(rng.integers(1, 4))
        Nq, Nk = int(rng.integers(1, 701)), int(rng.integers(1, 1501))
        scale = float(rng.choice([-1, 1]) * rng.uniform(0.05, 0.3))
        assert px.check_shape(kern, [BH, Nq, Nk, D]) == 0
        px.plan_pin(kern, [BH, Nq, Nk, D], int(rng.integers(2, 6)) if i % 3 == 2 else None)
        q = oracle.normal_f32(500 + i, BH * Nq * D).reshape(BH, Nq, D)
        k = oracle.normal_f32(600 + i, BH * Nk * D).reshape(BH, Nk, D)
        v = oracle.normal_f32(700 + i, BH * Nk * D).reshape(BH, Nk, D)
        if bits == 16:
            q, k, v = (oracle.f16_round(t) for t in (q, k, v))
            up = lambda t: px.DeviceBuffer.from_array(oracle.f16_bits(t))  # noqa: E731
            n_o = BH * Nq * D * 2 + 256
        else:
            up = lambda t: px.DeviceBuffer.from_array(np.ascontiguousarray(t, np.float32))  # noqa: E731
            n_o = BH * Nq * D * 4 + 256
        dq, dk, dv = up(q), up(k), up(v)
        do = px.DeviceBuffer(n_o)
        do.upload(np.full(n_o // 4, 0x7FC00001, np.uint32))  # NaN sentinels
        print(f"flash{bits} BH={BH} Nq={Nq} Nk={Nk} scale={scale:.3f} "
              f"plan={px.plan_get(kern, [BH, Nq, Nk, D])}", flush=True)
        px.launch_flash_bh(stream, kern, dq, dk, dv, do, BH, Nq, Nk, D, scale)
        stream.synchronize()
        raw = do.download(np.uint32, n_o // 4)
        used = (n_o - 256) // 4
        assert np.all(raw[used:] == 0x7FC00001), f"store past O at {(BH, Nq, Nk)}"
        if bits == 16:
            got = oracle.f16_to_f32(do.download(np.uint16, BH * Nq * D)).reshape(BH, Nq, D)
        else:
            got = do.download(np.float32, (BH, Nq, D))
        rows = np.unique(np.linspace(0, Nq - 1, min(Nq, 16)).astype(np.int64))
        for h in range(BH):
            want = oracle.flash_rows(rows, q[h], k[h], v[h], scale)
            err = (np.abs(got[h][rows] - want) / np.maximum(np.abs(want), 0.1)).max()
            assert err < (2e-2 if bits == 16 else 1e-4), (BH, Nq, Nk, h, err)
