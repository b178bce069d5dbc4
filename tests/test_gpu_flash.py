"""Flash-attention leaf kernels on gfx950 vs the f64 online-softmax oracle.

Metric (main.rs:912-917): rel = |got - want| / max(|want|, 0.1) per element.
Bounds: flash_fp16 <= 2e-2 (north-star fp16 tolerance); flash_fp32 <= 1e-4
(exact-f32 semantics, no f16 rounding).  want is computed over the
dtype-rounded inputs (main.rs:1079-1081).
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

TOL = {16: 2e-2, 32: 1e-4}


def _rel(got, want):
    return (np.abs(got - want) / np.maximum(np.abs(want), 0.1)).max()


def _upload(px, t, bits):
    if bits == 16:
        return px.DeviceBuffer.from_array(oracle.f16_bits(t).reshape(t.shape))
    return px.DeviceBuffer.from_array(np.ascontiguousarray(t, np.float32))


def _download(buf, shape, bits):
    n = int(np.prod(shape))
    if bits == 16:
        return oracle.f16_to_f32(buf.download(np.uint16, n)).reshape(shape)
    return buf.download(np.float32, shape)


def _inputs(shape, bits, seed0=1, scale=1.0):
    n = int(np.prod(shape))
    ts = [oracle.normal_f32(seed0 + i, n, scale).reshape(shape) for i in range(3)]
    if bits == 16:
        ts = [oracle.f16_round(t) for t in ts]
    return ts


@pytest.mark.parametrize("bits", [16, 32])
# Nk/64 = 1, 2, 3, 5, 6, 7, 16 key blocks covers every tail of the 4-stage copy
# ring; Nq = 128, 384, 640 leaves the last 256-row f16 workgroup half full.
@pytest.mark.parametrize("Nq,Nk", [(128, 64), (128, 128), (256, 192), (128, 320), (128, 384), (640, 448),
                                   (384, 1024)])
def test_flash_one_head_full(px_gpu, stream, bits, Nq, Nk):
    D = 64
    q, _, _ = _inputs((Nq, D), bits, 1)
    _, k, v = _inputs((Nk, D), bits, 11)
    dq, dk, dv = (_upload(px_gpu, t, bits) for t in (q, k, v))
    do = px_gpu.DeviceBuffer(Nq * D * 4)
    kern = px_gpu.FLASH_FP16 if bits == 16 else px_gpu.FLASH_FP32
    px_gpu.launch_flash(stream, kern, dq.ptr, dk.ptr, dv.ptr, do.ptr, Nq, Nk, D, 0.125)
    stream.synchronize()
    got = _download(do, (Nq, D), bits)
    want = oracle.flash_rows(np.arange(Nq), q, k, v, 0.125)
    assert _rel(got, want) < TOL[bits]


@pytest.mark.parametrize("bits", [16, 32])
def test_flash_large_scores_and_single_block(px_gpu, stream, bits):
    # scores of magnitude ~100 exercise the running-max rescale; Nk = 64 is a
    # single key block, i.e. plain softmax.
    D = 64
    for Nk in (64, 512):
        q = _inputs((128, D), bits, 5, 3.0)[0]
        _, k, _ = _inputs((Nk, D), bits, 7, 3.0)
        v = _inputs((Nk, D), bits, 7, 1.0)[2]
        dq, dk, dv = (_upload(px_gpu, t, bits) for t in (q, k, v))
        do = px_gpu.DeviceBuffer(128 * D * 4)
        kern = px_gpu.FLASH_FP16 if bits == 16 else px_gpu.FLASH_FP32
        px_gpu.launch_flash(stream, kern, dq.ptr, dk.ptr, dv.ptr, do.ptr, 128, Nk, D, 0.125)
        stream.synchronize()
        got = _download(do, (128, D), bits)
        want = oracle.flash_rows(np.arange(128), q, k, v, 0.125)
        assert _rel(got, want) < TOL[bits], (Nk, _rel(got, want))
        assert np.all(np.abs(got) <= np.abs(v).max() * (1 + 1e-3) + 1e-6)


@pytest.mark.parametrize("bits", [16, 32])
def test_flash_bh_equals_per_head_bit_exact(px_gpu, stream, bits):
    BH, N, D = 6, 256, 64
    q, k, v = _inputs((BH, N, D), bits, 21)
    dq, dk, dv = (_upload(px_gpu, t, bits) for t in (q, k, v))
    esz = 2 if bits == 16 else 4
    do = px_gpu.DeviceBuffer(BH * N * D * esz)
    kb = px_gpu.FLASH_FP16_BH if bits == 16 else px_gpu.FLASH_FP32_BH
    k1 = px_gpu.FLASH_FP16 if bits == 16 else px_gpu.FLASH_FP32
    px_gpu.launch_flash_bh(stream, kb, dq.ptr, dk.ptr, dv.ptr, do.ptr, BH, N, N, D, 0.125)
    stream.synchronize()
    dt = np.uint16 if bits == 16 else np.uint32
    batched = do.download(dt, BH * N * D).reshape(BH, N * D)
    do1 = px_gpu.DeviceBuffer(N * D * esz)
    hs = N * D * esz
    for h in range(BH):
        px_gpu.launch_flash(stream, k1, dq.ptr + h * hs, dk.ptr + h * hs, dv.ptr + h * hs,
                            do1.ptr, N, N, D, 0.125)
        stream.synchronize()
        assert np.array_equal(do1.download(dt, N * D), batched[h]), h
    got = _download(do, (BH, N, D), bits)
    want = oracle.flash_heads(q, k, v, 0.125)
    assert _rel(got, want) < TOL[bits]


@pytest.mark.parametrize("bits", [16, 32])
def test_flash_baseline_config_sampled(px_gpu, stream, bits):
    # B=4, H=16, Nq=Nk=4096, D=64, N(0,1) inputs, scale 1/8
    BH, N, D = 64, 4096, 64
    q, k, v = _inputs((BH, N, D), bits, 1)
    dq, dk, dv = (_upload(px_gpu, t, bits) for t in (q, k, v))
    do = px_gpu.DeviceBuffer(BH * N * D * 4)
    kb = px_gpu.FLASH_FP16_BH if bits == 16 else px_gpu.FLASH_FP32_BH
    px_gpu.launch_flash_bh(stream, kb, dq.ptr, dk.ptr, dv.ptr, do.ptr, BH, N, N, D, 0.125)
    stream.synchronize()
    got = _download(do, (BH, N, D), bits)
    assert np.isfinite(got).all()
    rng = np.random.default_rng(0)
    worst = 0.0
    for h in (0, 17, 38, 63):
        rows = np.concatenate([[0, N - 1], rng.choice(N, 30, replace=False)]).astype(np.uint64)
        want = oracle.flash_rows(rows, q[h], k[h], v[h], 0.125)
        worst = max(worst, _rel(got[h][rows.astype(int)], want))
    assert worst < TOL[bits], worst


@pytest.mark.parametrize("bits", [16, 32])
def test_flash_baseline_config_every_row(px_gpu, stream, bits):
    # all 64 heads x 4096 rows of the BASELINE config against the f64
    # online-softmax replay (main.rs:894-911, OpenMP over rows), and the
    # convexity bound: each output row is a convex combination of V's rows
    BH, N, D = 64, 4096, 64
    q, k, v = _inputs((BH, N, D), bits, 1)
    dq, dk, dv = (_upload(px_gpu, t, bits) for t in (q, k, v))
    do = px_gpu.DeviceBuffer(BH * N * D * 4)
    kb = px_gpu.FLASH_FP16_BH if bits == 16 else px_gpu.FLASH_FP32_BH
    px_gpu.launch_flash_bh(stream, kb, dq.ptr, dk.ptr, dv.ptr, do.ptr, BH, N, N, D, 0.125)
    stream.synchronize()
    got = _download(do, (BH, N, D), bits)
    want = oracle.flash_heads(q, k, v, 0.125)
    assert _rel(got, want) < TOL[bits]
    vmax = np.abs(v).reshape(BH, -1).max(axis=1)
    vmin_col, vmax_col = v.min(axis=1), v.max(axis=1)  # per head and d
    slack = 1e-2 if bits == 16 else 1e-5
    assert (np.abs(got).reshape(BH, -1).max(axis=1) <= vmax * (1 + slack)).all()
    assert (got >= vmin_col[:, None, :] - slack).all() and (got <= vmax_col[:, None, :] + slack).all()


def test_flash16_rows_past_nq_untouched(px_gpu, stream):
    # A 256-row f16 workgroup with Nq = 128 computes rows 128..255 from zero
    # queries but must not store them.
    px = px_gpu
    Nq, Nk, D = 128, 128, 64
    q, _, _ = _inputs((Nq, D), 16, 21)
    _, k, v = _inputs((Nk, D), 16, 31)
    dq, dk, dv = (_upload(px, t, 16) for t in (q, k, v))
    sentinel = np.full(2 * Nq * D, 0x7bff, np.uint16)  # f16 max, not a softmax output
    do = px.DeviceBuffer.from_array(sentinel)
    px.launch_flash(stream, px.FLASH_FP16, dq.ptr, dk.ptr, dv.ptr, do.ptr, Nq, Nk, D, 0.125)
    stream.synchronize()
    out = do.download(np.uint16, 2 * Nq * D)
    assert np.array_equal(out[Nq * D:], sentinel[Nq * D:])
    got = oracle.f16_to_f32(out[:Nq * D]).reshape(Nq, D)
    assert _rel(got, oracle.flash_rows(np.arange(Nq), q, k, v, 0.125)) < TOL[16]


@pytest.mark.parametrize("grid_x", [1, 5])
def test_flash16_bh_any_grid(px_gpu, stream, grid_x):
    # The bh entry walks (head, row block) work items block-stride: a grid with
    # fewer workgroups than items (LDS ring reused across items) or more
    # (idle workgroups) gives the grid_for result bit for bit.
    px = px_gpu
    BH, N, D = 3, 512, 64
    q, k, v = _inputs((BH, N, D), 16, 41)
    dq, dk, dv = (_upload(px, t, 16) for t in (q, k, v))
    dref, dgot = px.DeviceBuffer(BH * N * D * 2), px.DeviceBuffer(BH * N * D * 2)
    px.launch_flash_bh(stream, px.FLASH_FP16_BH, dq.ptr, dk.ptr, dv.ptr, dref.ptr, BH, N, N, D, 0.125)
    fn = px.builtin_function(px.FLASH_FP16_BH)
    px.compute(fn, 64, [(t.ptr, (BH, N, D)) for t in (dq, dk, dv, dgot)],
               [(4, 4, px.f32_bits(0.125))], (grid_x, 1, 1), px.kernel_abi(px.FLASH_FP16_BH)[1],
               stream)
    stream.synchronize()
    assert np.array_equal(dgot.download(np.uint16, BH * N * D), dref.download(np.uint16, BH * N * D))


@pytest.mark.parametrize("bits", [16, 32])
def test_flash_block_sum_over_limit_without_raise(px_gpu, stream, bits):
    # Key block 0 scores 0, so the running max (log2 units) is 0 after it.
    # Block 1 scores s*scale*log2e = 4.0 on every key: each p = 16, a lane's
    # 32 of them sum to 512 > 2^8, which sends the f16 kernel down its slow
    # path, but the block max (4) is within the slack of 8, so nothing is
    # raised.  Block 2 scores -4.  Exact answer from the f64 oracle.
    D, Nq, Nk = 64, 128, 192
    q = np.zeros((Nq, D), np.float32)
    q[:, 0] = 1.0
    k = np.zeros((Nk, D), np.float32)
    k[64:128, 0] = 22.1875   # 22.1875 * 0.125 * log2(e) = 4.001
    k[128:, 0] = -22.1875
    v = _inputs((Nk, D), bits, 51)[2]
    dq, dk, dv = (_upload(px_gpu, t, bits) for t in (q, k, v))
    do = px_gpu.DeviceBuffer(Nq * D * 4)
    kern = px_gpu.FLASH_FP16 if bits == 16 else px_gpu.FLASH_FP32
    px_gpu.launch_flash(stream, kern, dq.ptr, dk.ptr, dv.ptr, do.ptr, Nq, Nk, D, 0.125)
    stream.synchronize()
    got = _download(do, (Nq, D), bits)
    want = oracle.flash_rows(np.arange(Nq), q, k, v, 0.125)
    assert _rel(got, want) < TOL[bits]


def _void_args(vals):
    import ctypes
    return vals, (ctypes.c_void_p * len(vals))(
        *[ctypes.cast(ctypes.pointer(v), ctypes.c_void_p) for v in vals])


@pytest.mark.parametrize("bits", [16, 32])
def test_flash_with_reference_bench_geometry(px_gpu, stream, bits):
    # launch_flash (main.rs:334-371): grid Nq/BR with the reference's BR, the
    # @launch(128) cta, i64 exploded memrefs, one head.  The backend replaces
    # grid and cta with its own; the result equals the typed launch bit for
    # bit and the oracle within the kernel's tolerance.
    import ctypes
    px = px_gpu
    Nq, Nk, D = 512, 384, 64
    q, k, v = _inputs((Nq, D), bits, 61)[0], *_inputs((Nk, D), bits, 62)[1:]
    dq, dk, dv = (_upload(px, t, bits) for t in (q, k, v))
    esz = 2 if bits == 16 else 4
    do, dr = px.DeviceBuffer(Nq * D * esz), px.DeviceBuffer(Nq * D * esz)
    vals = []
    for buf, n in ((dq, Nq), (dk, Nk), (dv, Nk), (do, Nq)):
        vals += [ctypes.c_void_p(buf.ptr), ctypes.c_void_p(buf.ptr), ctypes.c_int64(0),
                 ctypes.c_int64(n), ctypes.c_int64(D), ctypes.c_int64(D), ctypes.c_int64(1)]
    vals.append(ctypes.c_float(0.125))
    keep, args = _void_args(vals)
    stem = b"flash_attention_fp16" if bits == 16 else b"flash_attention_fp32"
    grid = (ctypes.c_uint32 * 3)(Nq // 64, 1, 1)
    block = (ctypes.c_uint32 * 3)(128, 1, 1)
    px.check(px.lib().phx_launch_by_name(stem, b"flash_attention", grid, block, stream.handle,
                                         args))
    kern = px.FLASH_FP16 if bits == 16 else px.FLASH_FP32
    px.launch_flash(stream, kern, dq.ptr, dk.ptr, dv.ptr, dr.ptr, Nq, Nk, D, 0.125)
    stream.synchronize()
    dt = np.uint16 if bits == 16 else np.uint32
    assert np.array_equal(do.download(dt, Nq * D), dr.download(dt, Nq * D))
    got = _download(do, (Nq, D), bits)
    assert _rel(got, oracle.flash_rows(np.arange(Nq), q, k, v, 0.125)) < TOL[bits]


def test_raw_launch_refuses_inconsistent_descriptors(px_gpu, stream):
    # A built-in launched with descriptors the kernel would refuse on entry
    # (here K's head dim differs from Q's) is refused on the host.
    import ctypes
    px = px_gpu
    bufs = [px.DeviceBuffer(256 * 64 * 2) for _ in range(4)]
    vals = []
    for i, b in enumerate(bufs):
        d = 32 if i == 1 else 64
        vals += [ctypes.c_void_p(b.ptr), ctypes.c_void_p(b.ptr), ctypes.c_int64(0),
                 ctypes.c_int64(256), ctypes.c_int64(d), ctypes.c_int64(d), ctypes.c_int64(1)]
    vals.append(ctypes.c_float(0.125))
    keep, args = _void_args(vals)
    grid = (ctypes.c_uint32 * 3)(4, 1, 1)
    block = (ctypes.c_uint32 * 3)(128, 1, 1)
    rc = px.lib().phx_launch_by_name(b"flash_attention_fp16", b"flash_attention", grid, block,
                                     stream.handle, args)
    assert rc == px.PHX_E_INVALID and "disagree" in px.lib().phx_last_error().decode()
    stream.synchronize()


@pytest.mark.parametrize("split", ["1", "4"])
def test_flash_fp16_row_sum_is_over_the_f32_p(px_gpu, stream, monkeypatch, split):
    # flash_attention_fp16.ph:33-38: p = exp(s - mnew) is f32; l sums the
    # f32 p, and only P.V sees p rounded to f16.  Known answer that tells the
    # two apart: the first key of every 64-key block scores 1 (the row max,
    # p = 1, in every block and so in every key chunk of a split launch),
    # every other key scores b = f16(0.000616...), so with scale*log2e = 1
    # each other p is 2^(b - 1) = 0.5 + 0.8747 * 2^-12, which f16 rounds down
    # to 0.5.  With V = 1, O = sum f16(p) / sum p = (64 + 4032 * 0.5) /
    # (64 + 4032 * p) = 0.999586, which rounds to the f16 1 - 2^-11.  A
    # kernel that summed l over the f16-rounded p would return exactly 1.0.
    px = px_gpu
    monkeypatch.setenv("PHX_FLASH_SPLIT", split)
    Nq, Nk, D = 64, 4096, 64
    b = np.float16(0.000616)
    scale = np.float32(1 / 1.4426950408889634)
    assert np.float32(scale * np.float32(1.4426950408889634)) == 1.0
    q = np.zeros((Nq, D), np.float32)
    q[:, 0] = 1.0
    k = np.zeros((Nk, D), np.float32)
    k[:, 0] = float(b)
    k[::64, 0] = 1.0
    v = np.ones((Nk, D), np.float32)
    p = 2.0 ** (float(b) - 1.0)
    assert 0.87 < (p - 0.5) / 2 ** -12 < 0.88 and np.float16(p) == 0.5
    n1, nb = Nk // 64, Nk - Nk // 64
    want = np.float16((n1 + nb * 0.5) / (n1 + nb * p))
    assert want == np.float16(1 - 2 ** -11)
    dq, dk, dv = (_upload(px, t, 16) for t in (q, k, v))
    do = px.DeviceBuffer(Nq * D * 2)
    assert px.split_plan(px.FLASH_FP16, [Nq, Nk, D])[0] == int(split)
    px.launch_flash(stream, px.FLASH_FP16, dq.ptr, dk.ptr, dv.ptr, do.ptr, Nq, Nk, D, float(scale))
    stream.synchronize()
    got = do.download(np.uint16, Nq * D).view(np.float16)
    assert (got == want).all(), np.unique(got)
