"""saxpy_fp32 on gfx950 vs the oracle: bit-exact (main.rs:1176-1188)."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def _run(px, stream, x, y, alpha, alias=True):
    n = x.size
    dx, dy = px.DeviceBuffer.from_array(x), px.DeviceBuffer.from_array(y)
    if alias:
        px.launch_saxpy(stream, dx.ptr, dy.ptr, dy.ptr, n, alpha)
        stream.synchronize()
        return dy.download(np.float32, n)
    do = px.DeviceBuffer(max(4, n * 4))
    px.launch_saxpy(stream, dx.ptr, dy.ptr, do.ptr, n, alpha)
    stream.synchronize()
    return do.download(np.float32, n)


@pytest.mark.parametrize("n", [0, 1, 3, 4, 5, 255, 4096, 4097, 100_003, 1 << 20])
def test_saxpy_ragged_sizes(px_gpu, stream, n):
    x, y = oracle.lcg_f32(1, n), oracle.lcg_f32(2, n)
    got = _run(px_gpu, stream, x, y, 2.5, alias=(n % 2 == 0))
    want = oracle.saxpy(np.float32(2.5), x, y)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_saxpy_baseline_config_bit_exact(px_gpu, stream):
    # BASELINE config: n = 4096*4096, alpha = 2.5, y = alpha*x + y (out aliases y)
    n = 4096 * 4096
    x, y = px_gpu.lcg_f32(1, n), px_gpu.lcg_f32(2, n)
    got = _run(px_gpu, stream, x, y, 2.5)
    want = oracle.saxpy(np.float32(2.5), x, y)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_saxpy_special_values_and_no_fma(px_gpu, stream):
    x = np.array([0.0, -0.0, 1e-45, -1e-45, 3.4e38, -3.4e38, np.inf, 1.0 + 2 ** -23, 7.0],
                 np.float32)
    y = np.array([-0.0, 0.0, 1e-45, 0.0, 3.4e38, 1.0, -np.inf, -(1.0 + 2 ** -22), np.nan],
                 np.float32)
    alpha = np.float32(1.0 + 2 ** -23)
    got = _run(px_gpu, stream, x, y, float(alpha), alias=False)
    want = oracle.saxpy(alpha, x, y)
    assert np.array_equal(got.view(np.uint32)[:-1], want.view(np.uint32)[:-1])
    assert np.isnan(got[-1])
    # the uncontracted result differs from the fused one at index 7
    assert got[7] == np.float32(np.float32(alpha * x[7]) + y[7])


def test_saxpy_unaligned_offset_path(px_gpu, stream):
    # a buffer starting 1 float past a 16-byte boundary takes the scalar path
    n = 10_001
    x, y = oracle.lcg_f32(3, n + 1), oracle.lcg_f32(4, n + 1)
    dx, dy = px_gpu.DeviceBuffer.from_array(x), px_gpu.DeviceBuffer.from_array(y)
    px_gpu.launch_saxpy(stream, dx.ptr + 4, dy.ptr + 4, dy.ptr + 4, n, -1.25)
    stream.synchronize()
    got = dy.download(np.float32, n + 1)
    want = oracle.saxpy(np.float32(-1.25), x[1:], y[1:])
    assert got[0] == y[0]
    assert np.array_equal(got[1:].view(np.uint32), want.view(np.uint32))
