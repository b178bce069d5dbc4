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
@pytest.mark.parametrize("Nq,Nk", [(128, 64), (128, 320), (384, 1024)])
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
