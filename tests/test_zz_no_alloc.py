"""phx_flash_attention_bh_noalloc: the allocation-free variant of
phx_flash_attention_bh (a fixed device scratch array instead of the
workspace bound to the stream), called through the C ABI and checked bit for
bit against the existing entry point on the session stream, whose bound
workspace holds every split here: same split plan, same kernels, so the
outputs must be identical.  Two calls in a row, the second smaller, so the
second runs on scratch the first left behind; a size whose split needs more
than the scratch holds is refused; an unsplit size runs the batched kernel."""
import ctypes

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

D = 64


def _noalloc(px):
    L = px.lib()
    f = L.phx_flash_attention_bh_noalloc
    f.argtypes = [ctypes.c_void_p, ctypes.c_int] + [ctypes.c_uint64] * 4 + \
        [ctypes.c_int64] * 4 + [ctypes.c_float]
    f.restype = ctypes.c_int
    return f


def _case(px, stream, bits, BH, Nq, Nk, seed, scale=0.125):
    kern = px.FLASH_FP16_BH if bits == 16 else px.FLASH_FP32_BH
    q = oracle.normal_f32(seed, BH * Nq * D)
    k = oracle.normal_f32(seed + 1, BH * Nk * D)
    v = oracle.normal_f32(seed + 2, BH * Nk * D)
    if bits == 16:
        q, k, v = (oracle.f16_bits(t) for t in (q, k, v))
    dq, dk, dv = (px.DeviceBuffer.from_array(t) for t in (q, k, v))
    esz = 2 if bits == 16 else 4
    ref, got = px.DeviceBuffer(BH * Nq * D * esz), px.DeviceBuffer(BH * Nq * D * esz)
    px.launch_flash_bh(stream, kern, dq, dk, dv, ref, BH, Nq, Nk, D, scale)
    rc = _noalloc(px)(stream.handle, kern, dq.ptr, dk.ptr, dv.ptr, got.ptr, BH, Nq, Nk, D, scale)
    assert rc == 0, px.lib().phx_last_error().decode()
    stream.synchronize()
    dt = np.uint16 if bits == 16 else np.uint32
    a, b = ref.download(dt, BH * Nq * D), got.download(dt, BH * Nq * D)
    assert np.array_equal(a, b)
    # and the oracle, on a few rows of the last head
    if bits == 16:
        o = oracle.f16_to_f32(b).reshape(BH, Nq, D)
        qq, kk, vv = (oracle.f16_to_f32(t) for t in (q, k, v))
    else:
        o = b.view(np.float32).reshape(BH, Nq, D)
        qq, kk, vv = q, k, v
    rows = np.array([0, Nq // 2, Nq - 1])
    want = oracle.flash_rows(rows, qq.reshape(BH, Nq, D)[-1], kk.reshape(BH, Nk, D)[-1],
                             vv.reshape(BH, Nk, D)[-1], scale)
    err = (np.abs(o[-1][rows] - want) / np.maximum(np.abs(want), 0.1)).max()
    assert err < (2e-2 if bits == 16 else 1e-4)


@pytest.mark.parametrize("bits", [16, 32])
def test_noalloc_matches_flash_bh_on_two_calls(px_gpu, stream, bits):
    px = px_gpu
    kern = px.FLASH_FP16_BH if bits == 16 else px.FLASH_FP32_BH
    first, second = (1, 4096, 4096), (1, 700, 2113)
    for shape in (first, second):
        sp, ws = px.split_plan(kern, [shape[0], shape[1], shape[2], D])
        assert sp > 1 and 0 < ws <= 16 << 20, (shape, sp, ws)
    _case(px, stream, bits, *first, seed=71)
    _case(px, stream, bits, *second, seed=81)


def test_noalloc_unsplit_size_runs_the_batched_kernel(px_gpu, stream):
    px = px_gpu
    assert px.split_plan(px.FLASH_FP16_BH, [16, 4096, 1024, D])[0] == 1
    _case(px, stream, 16, 16, 4096, 1024, seed=91)


def test_noalloc_refuses_a_split_larger_than_its_scratch(px_gpu, stream):
    px = px_gpu
    BH, Nq, Nk = 1, 16384, 4096
    sp, ws = px.split_plan(px.FLASH_FP16_BH, [BH, Nq, Nk, D])
    assert ws > 16 << 20
    bufs = [px.DeviceBuffer(BH * max(Nq, Nk) * D * 2) for _ in range(4)]
    rc = _noalloc(px)(stream.handle, px.FLASH_FP16_BH, *(b.ptr for b in bufs), BH, Nq, Nk, D,
                      0.125)
    assert rc == px.PHX_E_INVALID
    assert "scratch" in px.lib().phx_last_error().decode()
    stream.synchronize()
