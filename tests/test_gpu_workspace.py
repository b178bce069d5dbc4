"""Split launches draw their workspace from memory the caller owns.

The reference's kernels never allocate: every buffer a launch touches is the
caller's (phobos-bench's DeviceBuffers; a pod COMPUTE touches only arena
tiles, phobos-pod/src/tile_store.rs:14-83, engine.rs:582-647).  This
backend splits small launches over K or over the keys; the split's partial
results go to the workspace bound to the launch stream
(phx_stream_set_workspace), or, in a pod, to an arena slab.  Checked here:

  * the reference bench's own one-head 4096 x 4096 flash launch
    (phx_launch_by_name with the .ph geometry, main.rs:334-371) and a
    256 x 256 x 8192 gemm_fp32 through phx_compute run split inside the bound workspace (its
    sentinel bytes are overwritten), leave hipMemGetInfo's free bytes
    unchanged, and meet the oracle;
  * the same launches on a stream with no workspace run unsplit, allocate
    nothing and meet the oracle; with a workspace too small for the built-in
    plan they take fewer chunks;
  * a pod's split COMPUTE takes its slab through the arena (the bump pointer
    moves past the tiles) and leaves device memory unchanged.
"""
import ctypes
import gc

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

SENTINEL = 0x7F  # 0x7F7F7F7F: a large finite f32 no partial result equals


class _NoGc:
    """Collects garbage first and holds the cyclic collector off, so no
    buffer of an earlier test is freed while free memory is compared."""

    def __enter__(self):
        gc.collect()
        gc.disable()

    def __exit__(self, *exc):
        gc.enable()


def _free_bytes():
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def _flash_args(px, dq, dk, dv, do, Nq, Nk, D, scale):
    """The launch! argument list of flash_attention_fp16.ph: four i64
    exploded memrefs and the f32 scale (main.rs:352-367)."""
    vals = []
    for buf, n in ((dq, Nq), (dk, Nk), (dv, Nk), (do, Nq)):
        vals += [ctypes.c_uint64(buf.ptr), ctypes.c_uint64(buf.ptr), ctypes.c_int64(0),
                 ctypes.c_int64(n), ctypes.c_int64(D), ctypes.c_int64(D), ctypes.c_int64(1)]
    vals.append(ctypes.c_float(scale))
    arr = (ctypes.c_void_p * len(vals))(*[ctypes.cast(ctypes.byref(v), ctypes.c_void_p)
                                         for v in vals])
    return vals, arr


def _one_head_flash(px, stream, Nq=4096, Nk=4096, D=64, scale=0.125, seed=5):
    q, k, v = (oracle.f16_bits(oracle.normal_f32(seed + i, n * D)) for i, n in
               enumerate((Nq, Nk, Nk)))
    dq, dk, dv = (px.DeviceBuffer.from_array(t) for t in (q, k, v))
    do = px.DeviceBuffer(Nq * D * 2)
    keep, args = _flash_args(px, dq, dk, dv, do, Nq, Nk, D, scale)
    grid = (ctypes.c_uint32 * 3)(Nq // 128, 1, 1)  # @launch(128), BR = 128
    block = (ctypes.c_uint32 * 3)(128, 1, 1)

    def launch():
        px.check(px.lib().phx_launch_by_name(b"flash_attention_fp16", b"flash_attention", grid,
                                             block, px._sh(stream), args))

    def check():
        got = oracle.f16_to_f32(do.download(np.uint16, Nq * D)).reshape(Nq, D)
        rows = np.array([0, 1, Nq // 2, Nq - 1])
        qq, kk, vv = (oracle.f16_to_f32(t) for t in (q, k, v))
        want = oracle.flash_rows(rows, qq.reshape(Nq, D), kk.reshape(Nk, D), vv.reshape(Nk, D),
                                 scale)
        err = (np.abs(got[rows] - want) / np.maximum(np.abs(want), 0.1)).max()
        assert err < 2e-2, err
        assert np.isfinite(got).all()
        return got

    return launch, check, (dq, dk, dv, do, keep)


def _gemm_fp32_compute(px, stream, M=256, N=256, K=8192, alpha=0.125, beta=1.5, seed=11):
    a, b, c = (oracle.lcg_f32(seed + i, n) for i, n in enumerate((M * K, K * N, M * N)))
    da, db, dc = (px.DeviceBuffer.from_array(t) for t in (a, b, c))
    fn = px.builtin_function(px.GEMM_FP32)
    want = oracle.gemm_full(a.reshape(M, K), b.reshape(K, N), c.reshape(M, N), alpha, beta)

    def launch():
        dc.upload(c)
        px.compute(fn, 32, [(da.ptr, (M, K)), (db.ptr, (K, N)), (dc.ptr, (M, N))],
                   [(3, 4, px.f32_bits(alpha)), (4, 4, px.f32_bits(beta))],
                   (M // 128, N // 128, 1), (256, 1, 1), stream)  # the reference's geometry

    def check():
        got = dc.download(np.float32, M * N).reshape(M, N)
        rel = np.abs(got - want) / np.maximum(np.abs(want), 1e-2 * np.sqrt(np.mean(want ** 2)))
        assert rel.max() < 1e-4, rel.max()

    return launch, check, (da, db, dc)


def _run_checked(px, stream, launch, check, ws=None):
    """Warm launch (a first launch loads the code object, which allocates),
    then a launch bracketed by hipMemGetInfo.  With ws (a DeviceBuffer bound
    as the workspace) filled with the sentinel, returns whether the launch
    wrote into it."""
    launch()
    stream.synchronize()
    if ws is not None:
        px.check(px.lib().phx_memset_async(ws.ptr, SENTINEL, ws.nbytes, None))
        px.synchronize()
    with _NoGc():
        before = _free_bytes()
        launch()
        stream.synchronize()
        after = _free_bytes()
    assert after == before, f"the launch changed free device memory by {before - after} B"
    check()
    if ws is not None:
        w = ws.download(np.uint8, ws.nbytes)
        return bool((w != SENTINEL).any())
    return False


@pytest.fixture()
def bare_stream(px_gpu):
    s = px_gpu.Stream()
    yield s
    s.destroy()


def test_reference_flash_launch_splits_inside_the_bound_workspace(px_gpu, bare_stream):
    px, s = px_gpu, bare_stream
    sp, need = px.split_plan(px.FLASH_FP16, [4096, 4096, 64])
    assert sp > 1 and need > 0
    ws = px.DeviceBuffer(need)
    px.set_workspace(s, ws.ptr, need)
    assert px.get_workspace(s) == (ws.ptr, need)
    launch, check, _ = _one_head_flash(px, s)
    assert _run_checked(px, s, launch, check, ws), "the split did not use the bound workspace"
    px.set_workspace(s, 0, 0)
    assert px.get_workspace(s) == (0, 0)


def test_unbound_stream_runs_without_a_split_and_allocates_nothing(px_gpu, bare_stream):
    # the flash launch runs unsplit; the gemm_fp32 launch (whose built-in
    # plan splits 16 ways) runs its 64 x 64 tiling, which needs no workspace
    px, s = px_gpu, bare_stream
    assert px.get_workspace(s) == (0, 0)
    launch, check, _ = _one_head_flash(px, s, seed=15)
    _run_checked(px, s, launch, check)
    glaunch, gcheck, _ = _gemm_fp32_compute(px, s, seed=21)
    _run_checked(px, s, glaunch, gcheck)
    # one 256 x 256 tile would take about 1.8 ms; the 64 x 64 tiling about 0.15
    e0, e1 = px.Event(), px.Event()
    e0.record(s)
    for _ in range(3):
        glaunch()
    e1.record(s)
    e1.synchronize()
    assert e0.elapsed_ms(e1) / 3 < 0.8


def test_gemm_compute_splits_inside_the_bound_workspace(px_gpu, bare_stream):
    px, s = px_gpu, bare_stream
    sp, need = px.split_plan(px.GEMM_FP32, [256, 256, 8192])
    assert sp == 16 and need == sp * 256 * 256 * 4
    ws = px.DeviceBuffer(need)
    px.set_workspace(s, ws.ptr, need)
    launch, check, _ = _gemm_fp32_compute(px, s)
    assert _run_checked(px, s, launch, check, ws)
    # a workspace that holds three chunks: the launch takes at most three
    small = 3 * 256 * 256 * 4
    px.set_workspace(s, ws.ptr, small)
    px.check(px.lib().phx_memset_async(ws.ptr, SENTINEL, need, None))
    px.synchronize()
    launch()
    s.synchronize()
    check()
    w = ws.download(np.uint8, need)
    assert (w[:small] != SENTINEL).any() and (w[small:] == SENTINEL).all()
    # 512^3 runs the 64 x 64 tiling unsplit: nothing allocated either
    assert px.split_plan(px.GEMM_FP32, [512, 512, 512]) == (1, 0)
    launch2, check2, _ = _gemm_fp32_compute(px, s, 512, 512, 512, seed=61)
    _run_checked(px, s, launch2, check2)
    px.set_workspace(s, 0, 0)


def test_misaligned_workspace_is_refused(px_gpu, bare_stream):
    px = px_gpu
    with pytest.raises(px.PhxError, match="256-byte"):
        px.set_workspace(bare_stream, 0x1000 + 16, 1 << 20)


def test_pod_split_compute_takes_an_arena_slab(px_gpu, tmp_path):
    # A 256 x 256 x 8192 gemm_fp32 COMPUTE (split 16 ways by the built-in
    # rule) in a pod: the tiles take 16.25 MiB of the arena and the split's
    # partial sums another 4 MiB slab while the leaf runs.  The COMPUTE runs
    # in a segment of its own, between one that ALLOCs and LOADs its tiles
    # and one that STOREs and FREEs them (tiles stay resident across
    # segments), so free device memory can be read around it alone (LOAD and
    # STORE stage through pinned host chunks the pod allocates as it needs
    # them).  With an arena too small for the slab the leaf runs unsplit, to
    # the same bound.
    from phobos_amd import cluster as cl
    px = px_gpu
    M, N, K = 256, 256, 8192
    alpha, beta = 0.125, 1.5
    sp, need = px.split_plan(px.GEMM_FP32, [M, N, K])
    assert sp > 1
    a, b, c = (oracle.lcg_f32(31 + i, n) for i, n in enumerate((M * K, K * N, M * N)))
    want = oracle.gemm_full(a.reshape(M, K), b.reshape(K, N), c.reshape(M, N), alpha, beta)
    paths = [str(tmp_path / f) for f in ("a.bin", "b.bin", "c.bin", "out.bin")]
    for p, t in zip(paths, (a, b, c, c)):
        t.tofile(p)
    load = "\n".join([
        f"1 - ALLOC 1 {M}x{K} f32", f"2 - ALLOC 2 {K}x{N} f32", f"3 - ALLOC 3 {M}x{N} f32",
        f"4 1 LOAD 1 0 0,0 {M},{K}", f"5 2 LOAD 2 1 0,0 {K},{N}", f"6 3 LOAD 3 2 0,0 {M},{N}"]) + "\n"
    compute = (f"1 - COMPUTE 1 1:r,2:r,3:rmw 3:f32:0x{px.f32_bits(alpha):08x},"
               f"4:f32:0x{px.f32_bits(beta):08x} 4,4,1 256,1,1\n")
    store = "\n".join([f"1 - STORE 3 3 0,0 {M},{N}", "2 1 FREE 1 0", "3 1 FREE 2 0",
                       "4 1 FREE 3 0"]) + "\n"
    tiles = 4 * (M * K + K * N + M * N)
    for arena, split in ((tiles + need + (1 << 20), True), (tiles + (1 << 20), False)):
        pod = cl.Pod(arena, 2)
        for t, (p, shape) in enumerate(zip(paths, ((M, K), (K, N), (M, N), (M, N)))):
            pod.set_tensor(t, "file://" + p, shape)
        pod.set_kernel(1, px.GEMM_FP32)
        pod.run(load)
        # warm both pod streams: the code objects load on first use, and a
        # kernel that spills registers makes HIP grow the launch queue's
        # scratch area on its first launch there (gemm_fp32's 256 x 256
        # kernels spill outside their K loop)
        pod.run(compute)
        pod.run(compute)
        pod.run(store)
        pod.run(load)
        with _NoGc():
            before = _free_bytes()
            st = pod.run(compute)
            assert _free_bytes() == before
        assert st["compute"] == 1
        bump = pod.arena_stats()[1]
        assert (bump >= tiles + need) == split, (bump, tiles, need)
        pod.run(store)
        got = np.fromfile(paths[3], np.float32).reshape(M, N)
        rel = np.abs(got - want) / np.maximum(np.abs(want), 1e-2 * np.sqrt(np.mean(want ** 2)))
        assert rel.max() < 1e-4, (split, rel.max())
        pod.close()


def test_two_streams_with_their_own_workspaces(px_gpu):
    # split launches on two streams at once, each stream with its own bound
    # workspace: ten interleaved rounds, every result equal to the first
    px = px_gpu
    s1, s2 = px.Stream(), px.Stream()
    try:
        sp, need = px.split_plan(px.FLASH_FP16, [4096, 4096, 64])
        assert sp > 1
        w1, w2 = px.DeviceBuffer(need), px.DeviceBuffer(need)
        px.set_workspace(s1, w1.ptr, need)
        px.set_workspace(s2, w2.ptr, need)
        l1, c1, k1 = _one_head_flash(px, s1, seed=101)
        l2, c2, k2 = _one_head_flash(px, s2, seed=201)
        l1()
        l2()
        s1.synchronize()
        s2.synchronize()
        first1, first2 = c1(), c2()
        for _ in range(10):
            l1()
            l2()
        s1.synchronize()
        s2.synchronize()
        assert np.array_equal(c1(), first1) and np.array_equal(c2(), first2)
    finally:
        s1.destroy()
        s2.destroy()


@pytest.mark.parametrize("slabs", [6, 2])
def test_pod_concurrent_split_computes_each_take_a_slab(px_gpu, tmp_path, slabs):
    # six independent split gemm_fp32 COMPUTEs (256 x 256 x 8192, one C tile
    # each) on a pod's four streams: each leaf binds its own arena slab to its
    # stream for its launch.  With room for all six slabs every leaf splits;
    # with room for two, the others find the arena full and run unsplit on
    # the 256 x 256 tiling.  Every C matches the oracle either way.
    from phobos_amd import cluster as cl
    px = px_gpu
    M, N, K, n = 256, 256, 8192, 6
    alpha, beta = 0.5, -1.0
    sp, need = px.split_plan(px.GEMM_FP32, [M, N, K])
    assert sp > 1
    a = oracle.lcg_f32(71, M * K)
    b = oracle.lcg_f32(72, K * N)
    cs = [oracle.lcg_f32(80 + i, M * N) for i in range(n)]
    paths = [str(tmp_path / "a.bin"), str(tmp_path / "b.bin")] + \
        [str(tmp_path / f"c{i}.bin") for i in range(n)]
    a.tofile(paths[0])
    b.tofile(paths[1])
    for i in range(n):
        cs[i].tofile(paths[2 + i])
    lines = [f"1 - ALLOC 1 {M}x{K} f32", f"2 - ALLOC 2 {K}x{N} f32",
             f"3 1 LOAD 1 0 0,0 {M},{K}", f"4 2 LOAD 2 1 0,0 {K},{N}"]
    sc = f"3:f32:0x{px.f32_bits(alpha):08x},4:f32:0x{px.f32_bits(beta):08x}"
    iid = 5
    frees = []
    for i in range(n):
        t = 10 + i
        lines += [f"{iid} - ALLOC {t} {M}x{N} f32", f"{iid + 1} {iid} LOAD {t} {2 + i} 0,0 {M},{N}",
                  f"{iid + 2} 3,4,{iid + 1} COMPUTE 1 1:r,2:r,{t}:rmw {sc} 1,1,1 256,1,1",
                  f"{iid + 3} {iid + 2} STORE {t} {2 + i} 0,0 {M},{N}",
                  f"{iid + 4} {iid + 3} FREE {t} 0"]
        frees.append(str(iid + 2))
        iid += 5
    lines += [f"{iid} {','.join(frees)} FREE 1 0", f"{iid + 1} {','.join(frees)} FREE 2 0"]
    tiles = 4 * (M * K + K * N + n * M * N)
    pod = cl.Pod(tiles + slabs * need + (1 << 20), 4)
    for t, (p, shape) in enumerate(zip(paths, [(M, K), (K, N)] + [(M, N)] * n)):
        pod.set_tensor(t, "file://" + p, shape)
    pod.set_kernel(1, px.GEMM_FP32)
    st = pod.run("\n".join(lines) + "\n")
    assert st["compute"] == n
    A, B = a.reshape(M, K), b.reshape(K, N)
    for i in range(n):
        got = np.fromfile(paths[2 + i], np.float32).reshape(M, N)
        want = oracle.gemm_full(A, B, cs[i].reshape(M, N), alpha, beta)
        rel = np.abs(got - want) / np.maximum(np.abs(want), 1e-2 * np.sqrt(np.mean(want ** 2)))
        assert rel.max() < 1e-4, (slabs, i, rel.max())
    pod.close()
