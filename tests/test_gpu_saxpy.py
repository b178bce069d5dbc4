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


def test_saxpy_max_i32_extent(px_gpu, stream):
    # n = 2^31 - 1, the largest extent the i32 descriptor holds (three 8 GiB
    # vectors, which 288 GB of HBM takes easily): the chunks past 4 GiB get
    # their own buffer resources and the last 3 elements are the ragged tail.
    # x and y are byte-pattern fills, so every output is the same f32 value.
    px = px_gpu
    n = (1 << 31) - 1
    dx, dy, do = (px.DeviceBuffer(n * 4) for _ in range(3))
    for b, byte in ((dx, 0x3F), (dy, 0x40), (do, 0x00)):
        assert px.lib().phx_memset_async(b.ptr, byte, b.nbytes, stream.handle) == 0
    print(f"saxpy n={n}", flush=True)
    px.launch_saxpy(stream, dx, dy, do, n, 2.5)
    stream.synchronize()
    x = np.frombuffer(bytes([0x3F] * 4), np.float32)
    y = np.frombuffer(bytes([0x40] * 4), np.float32)
    want = oracle.saxpy(np.float32(2.5), x, y).view(np.uint32)[0]
    chunk = 1 << 26  # elements per download (256 MiB)
    buf = np.empty(chunk, np.uint32)
    for start in range(0, n, chunk):
        m = min(chunk, n - start)
        assert px.lib().phx_memcpy_d2h(buf.ctypes.data, do.ptr + 4 * start, 4 * m) == 0
        bad = np.flatnonzero(buf[:m] != want)
        assert bad.size == 0, (start + bad[:4], buf[bad[:4]], want)
    for b in (dx, dy, do):
        b.free()
