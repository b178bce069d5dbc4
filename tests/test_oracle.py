"""Pins the CPU oracle against golden vectors and mathematics (no GPU)."""
import json
import os

import numpy as np
import pytest

import oracle

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _json(name):
    with open(os.path.join(GOLD, name)) as f:
        return json.load(f)


# ------------------------------------------------------------------ Lcg
def test_lcg_known_answers():
    kat = _json("lcg_kat.json")
    states = oracle.lcg_u64(1, 8)
    assert [int(s) for s in states] == [int(s) for s in kat["seed1_states"]]
    for seed in (1, 2, 3, 7):
        got = oracle.lcg_f32(seed, 8)
        want = np.array(kat[f"seed{seed}_unit"], np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_lcg_range_and_reproducible():
    # rng.rs:42-48 asserts (-1..1).contains; the expression actually lands in [-1, 0].
    x = oracle.lcg_f32(7, 4096)
    assert np.all(x >= -1.0) and np.all(x < 1.0)
    assert np.all(x <= 0.0)
    assert np.array_equal(oracle.lcg_f32(1, 64), oracle.lcg_f32(1, 64))
    assert not np.array_equal(oracle.lcg_f32(1, 16), oracle.lcg_f32(2, 16))


def test_normal_statistics():
    z = oracle.normal_f32(11, 1 << 20)
    assert abs(z.mean()) < 5e-3
    assert abs(z.std() - 1.0) < 5e-3
    # fourth moment of N(0,1) is 3
    assert abs((z.astype(np.float64) ** 4).mean() - 3.0) < 0.05
    s = oracle.normal_f32(11, 1000, 1.0 / 64.0)
    assert np.allclose(s, (z[:1000].astype(np.float64) / 64.0).astype(np.float32), rtol=1e-6)


# ------------------------------------------------------------------ f16
def test_f16_golden_pairs():
    g = _json("f16_pairs.json")
    f = np.array(g["f32_bits"], np.uint32).view(np.float32)
    want = np.array(g["f16_bits"], np.uint16)
    assert np.array_equal(oracle.f16_bits(f), want)


def test_f16_against_numpy_bulk():
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[~np.isnan(f)]
    with np.errstate(over="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f16_bits(f), want)
    # every f16 value round-trips exactly
    allh = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    fin = allh[~np.isnan(allh.view(np.float16))]
    assert np.array_equal(oracle.f16_to_f32(fin), fin.view(np.float16).astype(np.float32))
    assert np.array_equal(oracle.f16_bits(oracle.f16_to_f32(fin)), fin)


# ---------------------------------------------------------------- saxpy
def test_saxpy_is_uncontracted_mul_add():
    x = oracle.lcg_f32(1, 1 << 16)
    y = oracle.lcg_f32(2, 1 << 16)
    a = np.float32(2.5)
    want = (a * x) + y          # numpy: two separately rounded f32 ops
    got = oracle.saxpy(a, x, y)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # a case where fma and mul+add differ must take the mul+add value
    xs = np.array([1.0 + 2 ** -23], np.float32)
    ys = np.array([-(1.0 + 2 ** -22)], np.float32)
    al = np.float32(1.0 + 2 ** -23)
    exact = float(al) * float(xs[0]) + float(ys[0])
    got = oracle.saxpy(al, xs, ys)[0]
    assert got == np.float32(np.float32(al * xs[0]) + ys[0])
    assert got != np.float32(exact)


# ----------------------------------------------------------------- gemm
def _xorshift_points(M, N, count):
    st, mask = 0x243F6A8885A308D3, (1 << 64) - 1
    pts = []
    for s in range(count):
        if s == 0:
            pts.append((0, 0))
            continue
        if s == 1:
            pts.append((M - 1, N - 1))
            continue
        out = []
        for lim in (M, N):
            st ^= (st << 13) & mask
            st ^= st >> 7
            st ^= (st << 17) & mask
            out.append(st % lim)
        pts.append(tuple(out))
    return pts


def test_sample_points_match_xorshift():
    r, c = oracle.sample_points(4096, 4096, 64)
    assert list(zip(r.tolist(), c.tolist())) == _xorshift_points(4096, 4096, 64)


def test_gemm_full_against_numpy():
    rng = np.random.default_rng(3)
    A = rng.standard_normal((37, 53)).astype(np.float32)
    B = rng.standard_normal((53, 29)).astype(np.float32)
    C = rng.standard_normal((37, 29)).astype(np.float32)
    want = 0.125 * (A.astype(np.float64) @ B.astype(np.float64)) + 1.5 * C.astype(np.float64)
    got = oracle.gemm_full(A, B, C, 0.125, 1.5)
    assert np.allclose(got, want, rtol=1e-13, atol=1e-12)
    r, c = oracle.sample_points(37, 29, 64)
    pts = oracle.gemm_points(r, c, A, B, C, 0.125, 1.5)
    assert np.allclose(pts, want[r.astype(int), c.astype(int)], rtol=1e-13, atol=1e-12)
    # round16 rounds the operands exactly as f16_round does
    g16 = oracle.gemm_full(A, B, None, 1.0, 0.0, round16=True)
    want16 = oracle.f16_round(A).astype(np.float64) @ oracle.f16_round(B).astype(np.float64)
    assert np.allclose(g16, want16, rtol=1e-13, atol=1e-12)
    # swapped alpha/beta or a transposed operand must not pass
    assert not np.allclose(oracle.gemm_full(A, B, C, 1.5, 0.125), want, rtol=1e-3)
    Bsq = rng.standard_normal((53, 53)).astype(np.float32)
    Asq = A[:, :53]
    assert not np.allclose(oracle.gemm_full(Asq, Bsq, None, 1.0, 0.0),
                           Asq.astype(np.float64) @ Bsq.T.astype(np.float64), rtol=1e-3)


def test_gemm_integer_fixture_exact():
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "int_gemm.npz"))
    got = oracle.gemm_full(g["a"], g["b"], None, 1.0, 0.0)
    assert np.array_equal(got, g["c"].astype(np.float64))


def test_fp16acc_model_close_to_f64():
    A = oracle.normal_f32(1, 64 * 256, 1 / 16).reshape(64, 256)
    B = oracle.normal_f32(2, 256 * 64, 1 / 16).reshape(256, 64)
    want = oracle.gemm_full(A, B, None, 1.0, 0.0, round16=True)
    for (i, j) in [(0, 0), (5, 7), (63, 63)]:
        v = oracle.gemm_fp16acc_point(i, j, A, B, None, 1.0, 0.0)
        assert abs(v - want[i, j]) < 2e-2


def _fp16acc(a_row, b_col, K, alpha=1.0, beta=0.0, c=0.0):
    A = np.asarray(a_row, np.float32).reshape(1, K)
    B = np.asarray(b_col, np.float32).reshape(K, 1)
    C = np.full((1, 1), c, np.float32)
    return oracle.gemm_fp16acc_point(0, 0, A, B, C, alpha, beta)


def test_fp16acc_model_known_answers():
    """Known answers of main.rs:663-670's model (f16 accumulator rounded after
    every step, product and sum in f32, epilogue f16(alpha*acc + beta*c)),
    each chosen so that an f32-accumulating or product-rounding variant fails."""
    # 4096 ones: the f16 running sum stops at 2048 (2048 + 1 is a tie that
    # rounds to the even 2048); an f32 accumulator would give 4096.
    K = 4096
    assert _fp16acc(np.ones(K), np.ones(K), K) == 2048.0
    assert float(np.ones(K, np.float32).sum()) == 4096.0
    # 2048 + 1 + 1 stays 2048, whatever the order of the ones after it.
    assert _fp16acc([2048.0, 1.0, 1.0], [1.0, 1.0, 1.0], 3) == 2048.0
    assert _fp16acc([1.0, 1.0, 2048.0], [1.0, 1.0, 1.0], 3) == 2050.0
    # The product is added unrounded: (1+2^-10) + (1+2^-10)(1+3*2^-10) =
    # 2 + 5*2^-10 + 3*2^-20 is just above a tie and rounds up to 2 + 6*2^-10.
    # Rounding the product to f16 first (1 + 2^-8) lands on the tie itself,
    # which rounds to the even 2 + 4*2^-10.
    u = 2.0**-10
    assert _fp16acc([1 + u, 1 + u], [1.0, 1 + 3 * u], 2) == 2 + 6 * u
    assert float(np.float16(np.float32(1 + u) + np.float32(np.float16((1 + u) * (1 + 3 * u))))) \
        == 2 + 4 * u
    # Inputs are rounded to f16 (RNE) before the product: 1 + 2^-12 -> 1.
    assert _fp16acc([1.0 + 2.0**-12], [3.0], 1) == 3.0
    # Epilogue: f16(fl(alpha*acc) + fl(beta*c)); 0.5*2048 + 0.25*4 = 1025 is
    # exact in f16, 1024 + 0.5 (beta*c = 0.5) is a tie that rounds to 1024.
    assert _fp16acc([2048.0], [1.0], 1, 0.5, 0.25, 4.0) == 1025.0
    assert _fp16acc([2048.0], [1.0], 1, 0.5, 0.25, 2.0) == 1024.0
    assert _fp16acc([2048.0], [1.0], 1, 0.5, 0.25, 2.0 + 2.0**-10) == 1025.0


# ---------------------------------------------------------------- flash
def _softmax_attention(q, k, v, scale):
    s = q.astype(np.float64) @ k.astype(np.float64).T * scale
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    return p @ v.astype(np.float64)


def test_flash_tiny_fixture():
    g = _json("flash_tiny.json")
    q, k, v = (np.array(g[n], np.float32) for n in "qkv")
    got = oracle.flash_rows(np.arange(4), q, k, v, g["scale"])
    assert np.allclose(got, np.array(g["o"]), rtol=1e-12, atol=1e-12)


def test_flash_against_closed_form_and_invariants():
    rng = np.random.default_rng(9)
    H, N, D = 2, 96, 16
    q = rng.standard_normal((H, N, D)).astype(np.float32)
    k = rng.standard_normal((H, N, D)).astype(np.float32)
    v = rng.standard_normal((H, N, D)).astype(np.float32)
    got = oracle.flash_heads(q, k, v, 0.25)
    for h in range(H):
        assert np.allclose(got[h], _softmax_attention(q[h], k[h], v[h], 0.25), rtol=1e-11,
                           atol=1e-12)
    # convex combination of V rows
    assert np.all(np.abs(got) <= np.abs(v).max() + 1e-12)
    # permuting keys together with values leaves O unchanged
    perm = rng.permutation(N)
    got_p = oracle.flash_heads(q, k[:, perm], v[:, perm], 0.25)
    assert np.allclose(got, got_p, rtol=1e-11, atol=1e-12)
    # a single key gives O = v
    one = oracle.flash_heads(q[:, :5], k[:, :1], v[:, :1], 0.25)
    assert np.allclose(one, np.broadcast_to(v[:, :1], one.shape), rtol=0, atol=1e-15)
    # the f32 CPU baseline agrees
    o32 = oracle.flash_f32(q, k, v, 0.25)
    assert np.allclose(o32, got, rtol=1e-4, atol=1e-5)


def test_flash_any_scale_sign_and_ragged_keys():
    # negative and zero scales and key counts that are not block multiples:
    # the replay is per key, so it must match the closed form for any of them
    rng = np.random.default_rng(10)
    D = 16
    for Nq, Nk, scale in [(7, 37, -0.5), (3, 1, 0.25), (5, 65, 0.0), (4, 130, -3.0)]:
        q = rng.standard_normal((Nq, D)).astype(np.float32)
        k = rng.standard_normal((Nk, D)).astype(np.float32)
        v = rng.standard_normal((Nk, D)).astype(np.float32)
        got = oracle.flash_rows(np.arange(Nq), q, k, v, scale)
        assert np.allclose(got, _softmax_attention(q, k, v, scale), rtol=1e-10, atol=1e-12), scale
    # scale 0: every key weighs the same
    got = oracle.flash_rows(np.arange(Nq), q, k, v, 0.0)
    assert np.allclose(got, np.broadcast_to(v.astype(np.float64).mean(0), got.shape), atol=1e-12)
    # a sign error in the scale would pick the opposite softmax
    assert not np.allclose(oracle.flash_rows(np.arange(Nq), q, k, v, -3.0),
                           _softmax_attention(q, k, v, 3.0), atol=1e-3)


# ------------------------------------------------------- cluster chain
def test_cluster_chain_matches_direct_evaluation():
    rng = np.random.default_rng(4)
    M, N, K, TK = 16, 24, 64, 16
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    C = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    c = oracle.matmul_init(1.5, C)
    assert np.array_equal(c, (np.float32(1.5) * C))
    for k0 in range(0, K, TK):
        acc = (A[:, k0:k0 + TK].astype(np.float64) @ B[k0:k0 + TK].astype(np.float64)).astype(
            np.float32)
        c = oracle.matmul_step_epilogue(0.125, acc, c)
    want = 0.125 * (A.astype(np.float64) @ B.astype(np.float64)) + 1.5 * C.astype(np.float64)
    assert np.allclose(c, want, rtol=1e-5, atol=1e-5)


def test_sgemm_baseline_agrees():
    A = oracle.lcg_f32(1, 130 * 70).reshape(130, 70)
    B = oracle.lcg_f32(2, 70 * 300).reshape(70, 300)
    C = oracle.lcg_f32(3, 130 * 300).reshape(130, 300)
    got = oracle.sgemm_f32(0.125, A, B, 1.5, C)
    want = oracle.gemm_full(A, B, C, 0.125, 1.5)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5)


def test_sgemm_baseline_agrees_across_its_blocks():
    # M, N and K each cross the CPU GEMM's 64 x 256 x 256 blocking, with a
    # ragged last block: the full-size GPU checks use it as their checker
    A = oracle.normal_f32(7, 130 * 600).reshape(130, 600)
    B = oracle.normal_f32(8, 600 * 300).reshape(600, 300)
    C = oracle.normal_f32(9, 130 * 300).reshape(130, 300)
    got = oracle.sgemm_f32(0.75, A, B, -0.5, C)
    want = oracle.gemm_full(A, B, C, 0.75, -0.5)
    # f32 rounding of 600-term sums: a few 1e-6 of the RMS; a dropped or
    # misplaced block would be O(1)
    assert np.abs(got - want).max() / np.sqrt(np.mean(want ** 2)) < 2e-5


def test_saxpy_mt_matches_scalar_saxpy():
    # the multi-core CPU baseline computes the same bits as the scalar oracle
    n = 1_000_003
    x, y = oracle.lcg_f32(11, n), oracle.lcg_f32(12, n)
    a = oracle.saxpy_mt(np.float32(2.5), x, y)
    assert np.array_equal(a.view(np.uint32), oracle.saxpy(np.float32(2.5), x, y).view(np.uint32))
