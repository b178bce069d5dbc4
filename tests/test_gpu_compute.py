"""The drop-in path: raw module loading and pod-style COMPUTE marshalling.

phx_compute builds the exploded-memref argument list exactly as
Engine::launch does (phobos-pod/src/engine.rs:582-647), with scalars placed by
ScalarArg.pos; the kernels accept the reference-derived grid and cta."""
import ctypes
import os

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def test_module_load_data_and_raw_launch_saxpy(px_gpu, stream):
    px = px_gpu
    import ctypes
    with open(os.path.join(px.LIB_DIR, "saxpy_fp32.hsaco"), "rb") as f:
        image = f.read()
    m = ctypes.c_void_p()
    px.check(px.lib().phx_module_load_data(ctypes.byref(m), image, len(image)))
    fn = ctypes.c_void_p()
    px.check(px.lib().phx_module_get_function(ctypes.byref(fn), m, b"saxpy"))
    n = 5000
    x, y = oracle.lcg_f32(1, n), oracle.lcg_f32(2, n)
    dx, dy = px.DeviceBuffer.from_array(x), px.DeviceBuffer.from_array(y)
    do = px.DeviceBuffer(n * 4)
    # a module loaded from bytes is the caller's own kernel to the backend:
    # it launches with the caller's geometry, here grid ceil(n/16), 256 threads
    px.compute(fn.value, 32, [(dx.ptr, (n,)), (dy.ptr, (n,)), (do.ptr, (n,))],
               [(3, 4, px.f32_bits(2.5))], ((n + 15) // 16, 1, 1), (256, 1, 1), stream)
    stream.synchronize()
    got = do.download(np.float32, n)
    assert np.array_equal(got.view(np.uint32), oracle.saxpy(np.float32(2.5), x, y).view(np.uint32))
    px.check(px.lib().phx_module_unload(m))


def test_cluster_leaves_via_compute_with_reference_grid(px_gpu, stream):
    # matmul_2x2x2 planner geometry scaled down: leaf grid = supertile / 32,
    # cta 256 (phobos-sched/src/lib.rs:380-429, 1022-1093).
    px = px_gpu
    M, N, K, TK = 256, 384, 512, 128
    A = oracle.lcg_f32(1, M * K).reshape(M, K)
    B = oracle.lcg_f32(2, K * N).reshape(K, N)
    C = oracle.lcg_f32(3, M * N).reshape(M, N)
    alpha, beta = 0.125, 1.5
    step = px.builtin_function(px.MATMUL)
    init = px.builtin_function(px.MATMUL_INIT)
    dc = px.DeviceBuffer.from_array(C)
    # init leaf: params (C, beta) -> beta at position 1
    px.compute(init, 32, [(dc.ptr, (M, N))], [(1, 4, px.f32_bits(beta))],
               (M // 32, N // 32, 1), (256, 1, 1), stream)
    want = oracle.matmul_init(beta, C)
    for k0 in range(0, K, TK):
        da = px.DeviceBuffer.from_array(np.ascontiguousarray(A[:, k0:k0 + TK]))
        db = px.DeviceBuffer.from_array(np.ascontiguousarray(B[k0:k0 + TK]))
        px.compute(step, 32, [(da.ptr, (M, TK)), (db.ptr, (TK, N)), (dc.ptr, (M, N))],
                   [(3, 4, px.f32_bits(alpha)), (4, 4, px.f32_bits(beta))],
                   (M // 32, N // 32, 1), (256, 1, 1), stream)
        stream.synchronize()
        acc = oracle.gemm_full(A[:, k0:k0 + TK], B[k0:k0 + TK], None, 1.0, 0.0).astype(np.float32)
        want = oracle.matmul_step_epilogue(alpha, acc, want)
    got = dc.download(np.float32, (M, N))
    # per-step acc differs from the f64-rounded acc only by f32 summation order
    rel = np.abs(got - want) / np.abs(want)
    assert rel.max() < 1e-5, rel.max()
    full = oracle.gemm_full(A, B, C, alpha, beta)
    assert (np.abs(got - full) / np.abs(full)).max() < 1e-4


def test_matmul_init_ragged_and_exact(px_gpu, stream):
    px = px_gpu
    for (M, N) in ((1, 1), (3, 5), (33, 1000), (512, 512)):
        C = oracle.lcg_f32(4, M * N).reshape(M, N)
        dc = px.DeviceBuffer.from_array(C)
        px.launch_matmul_init(stream, dc.ptr, M, N, 1.5)
        stream.synchronize()
        got = dc.download(np.float32, (M, N))
        assert np.array_equal(got.view(np.uint32), oracle.matmul_init(1.5, C).view(np.uint32))


def test_launches_reject_bad_shapes_and_null_operands(px_gpu, stream):
    # Shapes outside the kernels' contract and null operands are refused on
    # the host before anything is launched.  Real buffers throughout, so a
    # check that let one through could not reach a null address.
    px = px_gpu
    buf = px.DeviceBuffer(1 << 20)
    p = buf.ptr
    with pytest.raises(px.PhxError) as e:
        px.launch_gemm(stream, px.GEMM_FP16, p, p, p, 64, 100, 64, 1.0, 0.0)   # N % 8
    assert e.value.code == px.PHX_E_INVALID
    with pytest.raises(px.PhxError):
        px.launch_gemm(stream, px.GEMM_FP32, p, p, p, 64, 64, 30, 1.0, 0.0)    # K % 4
    with pytest.raises(px.PhxError):
        px.launch_flash(stream, px.FLASH_FP16, p, p, p, p, 16, 16, 128, 0.125)  # D != 64
    with pytest.raises(px.PhxError):
        px.launch_flash(stream, px.FLASH_FP32, p, p, p, p, 0, 16, 64, 0.125)   # Nq = 0
    with pytest.raises(px.PhxError):
        px.launch_gemm(stream, px.GEMM_FP32, p + 4, p, p, 64, 64, 64, 1.0, 0.0)  # misaligned
    for call in (lambda: px.lib().phx_gemm(stream.handle, px.GEMM_FP32, 0, p, p, 64, 64, 64,
                                           ctypes.c_float(1.0), ctypes.c_float(0.0)),
                 lambda: px.lib().phx_flash_attention(stream.handle, px.FLASH_FP16, p, p, 0, p,
                                                      16, 16, 64, ctypes.c_float(0.125)),
                 lambda: px.lib().phx_saxpy(stream.handle, p, 0, p, 16, ctypes.c_float(1.0))):
        assert call() == px.PHX_E_INVALID
        assert "null operand" in px.lib().phx_last_error().decode()
    stream.synchronize()


@pytest.mark.parametrize("kernel,grid", [("GEMM_FP16", 2), ("GEMM_FP16TC_FP32ACC", 4),
                                         ("GEMM_FP16", 17), ("GEMM_FP16TC_FP32ACC", 9)])
def test_f16_gemms_any_grid(px_gpu, stream, kernel, grid):
    # The reference derives the GEMM grid from its own tile sizes
    # (main.rs:500-508); these kernels walk their tiles block-stride, so a grid
    # smaller than the tile count (several tiles per workgroup, LDS reused
    # across tiles) or larger (idle workgroups) gives the same result.
    px = px_gpu
    k = getattr(px, kernel)
    f16 = kernel == "GEMM_FP16"
    M, N, K = 768, 512, 96   # 6 output tiles of 256x256
    A = oracle.f16_round(oracle.normal_f32(11, M * K, 1 / np.sqrt(K)))
    B = oracle.f16_round(oracle.normal_f32(12, K * N, 1 / np.sqrt(K)))
    if f16:
        dA, dB = px.DeviceBuffer.from_array(oracle.f16_bits(A)), px.DeviceBuffer.from_array(oracle.f16_bits(B))
        dC, dR = px.DeviceBuffer(M * N * 2), px.DeviceBuffer(M * N * 2)
    else:
        dA, dB = px.DeviceBuffer.from_array(A), px.DeviceBuffer.from_array(B)
        dC, dR = px.DeviceBuffer(M * N * 4), px.DeviceBuffer(M * N * 4)
    px.launch_gemm(stream, k, dA.ptr, dB.ptr, dR.ptr, M, N, K, 1.0, 0.0)
    fn = px.builtin_function(k)
    px.compute(fn, 64, [(dA.ptr, (M, K)), (dB.ptr, (K, N)), (dC.ptr, (M, N))],
               [(3, 4, px.f32_bits(1.0)), (4, 4, px.f32_bits(0.0))], (grid, 1, 1), (256, 1, 1),
               stream)
    stream.synchronize()
    dt = np.uint16 if f16 else np.uint32
    assert np.array_equal(dC.download(dt, M * N), dR.download(dt, M * N))


def test_launch_by_reference_names_with_void_args(px_gpu, stream):
    # phx_launch_by_name takes the reference's launch! argument list: one
    # pointer per kernel parameter, each memref exploded as (alloc, aligned,
    # offset, size, stride) at the kernel's index width (i32 for saxpy,
    # main.rs:1230-1235), then the f32 scalar.
    px = px_gpu
    n = 10_007
    x, y = oracle.lcg_f32(5, n), oracle.lcg_f32(6, n)
    dx, dy = px.DeviceBuffer.from_array(x), px.DeviceBuffer.from_array(y)
    do = px.DeviceBuffer(n * 4)
    vals = []
    for b in (dx, dy, do):
        vals += [ctypes.c_void_p(b.ptr), ctypes.c_void_p(b.ptr), ctypes.c_int32(0),
                 ctypes.c_int32(n), ctypes.c_int32(1)]
    vals.append(ctypes.c_float(2.5))
    args = (ctypes.c_void_p * len(vals))(*[ctypes.cast(ctypes.pointer(v), ctypes.c_void_p) for v in vals])
    grid = (ctypes.c_uint32 * 3)(*px.grid_for(px.SAXPY_FP32, [n])[0])
    assert px.lib().phx_launch_by_name(b"saxpy_fp32", b"saxpy", grid, None, stream.handle, args) == 0
    stream.synchronize()
    want = oracle.saxpy(np.float32(2.5), x, y)
    assert np.array_equal(do.download(np.float32, n).view(np.uint32), want.view(np.uint32))
    # the reference bench's own geometry (main.rs:1216-1235): grid
    # ceil(n/BLOCK) with BLOCK = 16 and 1024-thread blocks; the backend runs
    # saxpy on its own geometry, with y aliased as out (y = alpha*x + y)
    dy2 = px.DeviceBuffer.from_array(y)
    vals2 = []
    for b in (dx, dy2, dy2):
        vals2 += [ctypes.c_void_p(b.ptr), ctypes.c_void_p(b.ptr), ctypes.c_int32(0),
                  ctypes.c_int32(n), ctypes.c_int32(1)]
    vals2.append(ctypes.c_float(2.5))
    args2 = (ctypes.c_void_p * len(vals2))(*[ctypes.cast(ctypes.pointer(v), ctypes.c_void_p)
                                             for v in vals2])
    grid2 = (ctypes.c_uint32 * 3)((n + 15) // 16, 1, 1)
    block2 = (ctypes.c_uint32 * 3)(1024, 1, 1)
    assert px.lib().phx_launch_by_name(b"saxpy_fp32", b"saxpy", grid2, block2, stream.handle,
                                       args2) == 0
    # and through the caller's own load of the code object file, as
    # Module::from_ptx + get_function would
    m = ctypes.c_void_p()
    px.check(px.lib().phx_module_load_file(ctypes.byref(m),
                                           os.path.join(px.LIB_DIR, "saxpy_fp32.hsaco").encode()))
    fn = ctypes.c_void_p()
    px.check(px.lib().phx_module_get_function(ctypes.byref(fn), m, b"saxpy"))
    do3 = px.DeviceBuffer(n * 4)
    vals3 = vals2[:10] + [ctypes.c_void_p(do3.ptr), ctypes.c_void_p(do3.ptr), ctypes.c_int32(0),
                          ctypes.c_int32(n), ctypes.c_int32(1), ctypes.c_float(2.5)]
    args3 = (ctypes.c_void_p * len(vals3))(*[ctypes.cast(ctypes.pointer(v), ctypes.c_void_p)
                                             for v in vals3])
    px.check(px.lib().phx_launch(fn, grid2, block2, 0, stream.handle, args3))
    stream.synchronize()
    assert np.array_equal(dy2.download(np.float32, n).view(np.uint32), want.view(np.uint32))
    px.check(px.lib().phx_module_unload(m))
    # unknown names are refused before any launch
    assert px.lib().phx_launch_by_name(b"gemm_fp64", b"gemm", grid, None, stream.handle, args) \
        == px.PHX_E_INVALID


_THREADS_SCRIPT = r'''
import sys, threading
import numpy as np
sys.path[:0] = sys.argv[1:3]
import oracle
import phobos_amd as px
px.init(0)
errors = []
start = threading.Barrier(6)

def gemm(kern, f16):
    M, N, K = 300, 200, 512
    A = oracle.normal_f32(5, M * K, 1 / np.sqrt(K)).reshape(M, K)
    B = oracle.normal_f32(6, K * N, 1 / np.sqrt(K)).reshape(K, N)
    if kern != px.GEMM_FP32:
        A, B = oracle.f16_round(A), oracle.f16_round(B)
    conv = oracle.f16_bits if f16 else (lambda t: np.ascontiguousarray(t, np.float32))
    da, db = px.DeviceBuffer.from_array(conv(A)), px.DeviceBuffer.from_array(conv(B))
    dc = px.DeviceBuffer(M * N * (2 if f16 else 4))
    want = oracle.gemm_full(A, B, None, 1.0, 0.0, round16=kern != px.GEMM_FP32)
    def run(s):
        px.launch_gemm(s, kern, da, db, dc, M, N, K, 1.0, 0.0)
        s.synchronize()
        r = dc.download(np.uint16 if f16 else np.float32, M * N)
        return (oracle.f16_to_f32(r) if f16 else r).reshape(M, N)
    tol = 2e-2 if kern != px.GEMM_FP32 else 1e-4
    return run, lambda g: np.abs(g - want).max() / np.sqrt(np.mean(want ** 2)) < tol

def flash(kern, f16):
    Nq, Nk, D = 256, 1000, 64
    q, k, v = (oracle.normal_f32(s, n * D).reshape(n, D) for s, n in ((7, Nq), (8, Nk), (9, Nk)))
    if f16:
        q, k, v = (oracle.f16_round(t) for t in (q, k, v))
    conv = oracle.f16_bits if f16 else (lambda t: np.ascontiguousarray(t, np.float32))
    dq, dk, dv = (px.DeviceBuffer.from_array(conv(t)) for t in (q, k, v))
    do = px.DeviceBuffer(Nq * D * (2 if f16 else 4))
    rows = np.arange(0, Nq, 17)
    want = oracle.flash_rows(rows, q, k, v, 0.125)
    def run(s):
        px.launch_flash(s, kern, dq, dk, dv, do, Nq, Nk, D, 0.125)
        s.synchronize()
        r = do.download(np.uint16 if f16 else np.float32, Nq * D)
        return (oracle.f16_to_f32(r) if f16 else r).reshape(Nq, D)
    tol = 2e-2 if f16 else 1e-4
    return run, lambda g: (np.abs(g[rows] - want) / np.maximum(np.abs(want), 0.1)).max() < tol

def saxpy():
    n = 100003
    x, y = oracle.lcg_f32(1, n), oracle.lcg_f32(2, n)
    dx, dy, do = px.DeviceBuffer.from_array(x), px.DeviceBuffer.from_array(y), px.DeviceBuffer(4 * n)
    want = oracle.saxpy(2.5, x, y)
    def run(s):
        px.launch_saxpy(s, dx, dy, do, n, 2.5)
        s.synchronize()
        return do.download(np.float32, n)
    return run, lambda g: np.array_equal(g.view(np.uint32), want.view(np.uint32))

jobs = [saxpy(), gemm(px.GEMM_FP32, False), gemm(px.GEMM_FP16TC_FP32ACC, False),
        gemm(px.GEMM_FP16, True), flash(px.FLASH_FP32, False), flash(px.FLASH_FP16, True)]

def worker(i):
    try:
        s = px.Stream()
        run, ok = jobs[i]
        start.wait()  # every thread's first launch (and code-object load) at once
        first = run(s)
        assert ok(first), f"job {i}: wrong result"
        for _ in range(10):
            assert np.array_equal(run(s), first), f"job {i}: result changed"
    except Exception as e:
        errors.append(repr(e))

ts = [threading.Thread(target=worker, args=(i,)) for i in range(6)]
[t.start() for t in ts]
[t.join() for t in ts]
print("ERRORS" if errors else "OK", errors, flush=True)
sys.exit(1 if errors else 0)
'''


def test_concurrent_first_launches_from_threads(px_gpu):
    # Six host threads, each with its own stream, start at once in a fresh
    # process, so six code objects load concurrently on first use; each
    # result matches the oracle and stays the same over ten more launches.
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _THREADS_SCRIPT, root,
                        os.path.join(root, "phobos-lang_amd")],
                       capture_output=True, text=True, timeout=180)
    assert r.returncode == 0 and "OK" in r.stdout, (r.stdout, r.stderr[-2000:])
