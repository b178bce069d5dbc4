"""The matmul_cluster config on one pod: ALLOC/LOAD/COMPUTE/STORE/FREE with
async copies, file:// tensors, checked against the f64 oracle.

Tolerance: relative error <= 1e-4 (the reference checks 1e-3,
cluster_correctness.rs:344-375; the north star tightens it).  Lcg inputs are
all in [-1, 0], so 0.125*A@B + 1.5*C does not cancel at these sizes."""
import os

import numpy as np
import pytest

import oracle
from phobos_amd import cluster as cl

pytestmark = pytest.mark.gpu


def test_small_job_full_check(px_gpu, tmp_path):
    M = N = K = 1024
    stats, paths, ins = cl.run_matmul_job(str(tmp_path), M, N, K, 256, 512, 256, 0.125, 1.5)
    c = cl.count_ops(ins)
    assert stats["alloc"] == c["ALLOC"] and stats["load"] == c["LOAD"]
    assert stats["compute"] == c["COMPUTE"] and stats["store"] == c["STORE"]
    assert stats["free"] == c["FREE"]
    A = oracle.lcg_f32(1, M * K).reshape(M, K)
    B = oracle.lcg_f32(2, K * N).reshape(K, N)
    C = oracle.lcg_f32(3, M * N).reshape(M, N)
    got = np.fromfile(paths[cl.C], np.float32).reshape(M, N)
    want = oracle.gemm_full(A, B, C, 0.125, 1.5)
    rel = np.abs(got - want) / np.abs(want)
    assert rel.max() < 1e-4, rel.max()
    # inputs are untouched
    assert np.array_equal(np.fromfile(paths[cl.A], np.float32), A.ravel())


def test_chain_matches_leaf_replay(px_gpu, tmp_path):
    # init C = fl(1.5*C), then C = fl(fl(0.125*acc_k) + C) per K supertile
    M, N, K, TM, TN, TK = 256, 256, 512, 256, 256, 128
    stats, paths, _ = cl.run_matmul_job(str(tmp_path), M, N, K, TM, TN, TK, 0.125, 1.5)
    A = oracle.lcg_f32(1, M * K).reshape(M, K)
    B = oracle.lcg_f32(2, K * N).reshape(K, N)
    want = oracle.matmul_init(1.5, oracle.lcg_f32(3, M * N).reshape(M, N))
    for k0 in range(0, K, TK):
        acc = oracle.gemm_full(A[:, k0:k0 + TK], B[k0:k0 + TK], None, 1.0, 0.0).astype(np.float32)
        want = oracle.matmul_step_epilogue(0.125, acc, want)
    got = np.fromfile(paths[cl.C], np.float32).reshape(M, N)
    assert (np.abs(got - want) / np.abs(want)).max() < 1e-5


def test_arena_exhausted_is_reported(px_gpu, tmp_path):
    import phobos_amd as px
    with pytest.raises(cl.PhxError) as e:
        cl.run_matmul_job(str(tmp_path), 512, 512, 512, 256, 256, 256, 0.125, 1.5,
                          arena_bytes=1 << 16)
    assert e.value.code == px.PHX_E_EXHAUSTED


def test_malformed_segment_rejected(px_gpu):
    import phobos_amd as px
    pod = cl.Pod(1 << 20, 2)
    with pytest.raises(cl.PhxError) as e:
        pod.run("1 - ALLOC 0x1 16x16 f32\n2 7 FREE 0x1 0\n")
    assert e.value.code == 1006
    with pytest.raises(cl.PhxError):
        pod.run("1 - BOGUS 0x1\n")
    pod.close()


def test_baseline_job_16384(px_gpu, tmp_path):
    # matmul_cluster config: 16384^3 f32, supertiles 4096/8192/4096,
    # alpha 0.125, beta 1.5, A/B/C from Lcg seeds 1/2/3 in 1 GiB files.
    M = N = K = 16384
    print(f"[cluster] writing inputs to {tmp_path}", flush=True)
    stats, paths, ins = cl.run_matmul_job(str(tmp_path), M, N, K, 4096, 8192, 4096, 0.125, 1.5)
    print(f"[cluster] stats {stats}", flush=True)
    assert (stats["alloc"], stats["load"], stats["compute"], stats["store"], stats["free"]) == \
        (32, 32, 40, 8, 32)
    A = np.memmap(paths[cl.A], np.float32, "r", shape=(M, K))
    B = np.memmap(paths[cl.B], np.float32, "r", shape=(K, N))
    Cin = oracle.lcg_f32(3, M * N)
    got = np.memmap(paths[cl.C], np.float32, "r", shape=(M, N))
    r, c = oracle.sample_points(M, N, 12)
    for i, j in zip(r.astype(int), c.astype(int)):
        want = 0.125 * np.dot(A[i].astype(np.float64), B[:, j].astype(np.float64)) + \
            1.5 * float(Cin[i * N + j])
        assert abs(got[i, j] - want) / abs(want) < 1e-4, (i, j, got[i, j], want)
    tflops = 2 * M * N * K / (stats["compute_ns"] * 1e-9) / 1e12
    print(f"[cluster] compute {tflops:.1f} TFLOP/s, wall {stats['wall_ns'] / 1e9:.2f} s", flush=True)


def test_wire_format_job_matches_text_job(px_gpu, tmp_path):
    # The same one-pod job fed as the scheduler's messages: a JobManifest
    # (tensors by index, leaves bound by entry name, server.rs:189-225) and an
    # encoded Segment (server.rs:239-248).  The result file must equal the
    # text-path run bit for bit.
    M, N, K, TM, TN, TK = 512, 1024, 512, 256, 512, 256
    text_dir, pb_dir = tmp_path / "text", tmp_path / "pb"
    text_dir.mkdir()
    pb_dir.mkdir()
    _, paths_t, ins = cl.run_matmul_job(str(text_dir), M, N, K, TM, TN, TK, 0.125, 1.5)
    shapes = {cl.A: (M, K), cl.B: (K, N), cl.C: (M, N)}
    paths = {t: os.path.join(str(pb_dir), f"{n}.tensor") for t, n in ((cl.A, "a"), (cl.B, "b"), (cl.C, "c"))}
    for t, seed in ((cl.A, 1), (cl.B, 2), (cl.C, 3)):
        cl.init_tensor(paths[t], shapes[t], "random", seed)
    manifest = cl.manifest_pb([(t, "file://" + paths[t], shapes[t]) for t in (cl.A, cl.B, cl.C)],
                              [(cl.STEP_LEAF, "0" * 64, "matmul"), (cl.INIT_LEAF, "1" * 64, "matmul_init")])
    pod = cl.Pod(4 * (M * K + K * N + M * N) + (1 << 20), 4)
    try:
        pod.set_manifest_pb(manifest)
        stats = pod.run_pb(cl.segment_pb(ins, 1))
    finally:
        pod.close()
    assert stats["compute"] == cl.count_ops(ins)["COMPUTE"]
    got = np.fromfile(paths[cl.C], np.float32)
    assert np.array_equal(got.view(np.uint32), np.fromfile(paths_t[cl.C], np.float32).view(np.uint32))


def test_manifest_unknown_kernel_name_is_reported(px_gpu):
    pod = cl.Pod(1 << 20, 1)
    try:
        with pytest.raises(px_gpu.PhxError) as e:
            pod.set_manifest_pb(cl.manifest_pb([], [(0, "0" * 64, "gemm")]))
        assert e.value.code == 1003 and "phx_pod_set_kernel" in str(e.value)
    finally:
        pod.close()


def test_job_file_runs_on_one_pod(px_gpu, tmp_path):
    # A matmul_cluster job file (phobos-sched job format) seeded with the
    # phobos-tensor tool, run through phobos_amd.job, checked against the
    # oracle at the xorshift sample points.
    from phobos_amd import job as jb
    from phobos_amd import tensor as tn
    M, N, K = 512, 1024, 256
    for name, shape, seed in (("a", f"{M}x{K}", 1), ("b", f"{K}x{N}", 2), ("c", f"{M}x{N}", 3)):
        assert tn.main(["init", "--uri", f"file://{tmp_path}/{name}.tensor", "--shape", shape,
                        "--fill", "random", "--seed", str(seed)]) == 0
    p = tmp_path / "job.txt"
    p.write_text(f"source = x\ndim M = {M}\ndim N = {N}\ndim K = {K}\n"
                 f"tensor A = read f32 {M}x{K} file://{tmp_path}/a.tensor\n"
                 f"tensor B = read f32 {K}x{N} file://{tmp_path}/b.tensor\n"
                 f"tensor C = rmw f32 {M}x{N} file://{tmp_path}/c.tensor\n"
                 "scalar alpha = f32 0.125\nscalar beta = f32 1.5\n")
    stats = jb.run_job(jb.parse_job(str(p), read_source=False), tiles=(256, 512, 128))
    assert stats["compute"] == 2 * 2 * (1 + 2)
    A = oracle.lcg_f32(1, M * K).reshape(M, K)
    B = oracle.lcg_f32(2, K * N).reshape(K, N)
    C = oracle.lcg_f32(3, M * N).reshape(M, N)
    got = np.fromfile(f"{tmp_path}/c.tensor", np.float32).reshape(M, N)
    r, c = oracle.sample_points(M, N, 64)
    want = oracle.gemm_points(r, c, A, B, C, 0.125, 1.5)
    assert (np.abs(got[r, c] - want) / np.abs(want)).max() < 1e-4


def test_loopback_add_from_a_caller_code_object(px_gpu, tmp_path):
    # The loopback job's second half (phobos-pod/examples/loopback.rs:116-156):
    # c = a + b over 1024 Lcg draws (seeds 3 and 4), checked bit for bit.  The
    # `add` leaf is not built in: its code object is loaded from bytes and
    # bound to the segment's kernel id, as a SetKernels reply binds PTX, and
    # the COMPUTE runs with its own grid and cta (here the reference-style
    # 64 x 64 threads).
    px = px_gpu
    n = 1024
    x, y = oracle.lcg_f32(3, n), oracle.lcg_f32(4, n)
    paths = [str(tmp_path / f) for f in ("a.bin", "b.bin", "c.bin")]
    x.tofile(paths[0])
    y.tofile(paths[1])
    np.zeros(n, np.float32).tofile(paths[2])
    with open(os.path.join(px.LIB_DIR, "ew_add_fp32.hsaco"), "rb") as f:
        mod = px.module_load_data(f.read())
    pod = cl.Pod(64 << 20, nstreams=2)
    for t, p in enumerate(paths):
        pod.set_tensor(t, "file://" + p, (n,))
    seg = "\n".join([
        "1 - ALLOC 101 1024 f32", "2 - ALLOC 102 1024 f32", "3 - ALLOC 103 1024 f32",
        "4 1 LOAD 101 0 0 1024", "5 2 LOAD 102 1 0 1024",
        "6 3,4,5 COMPUTE 9 101:r,102:r,103:w - 64,1,1 64,1,1",
        "7 6 STORE 103 2 0 1024",
        "8 7 FREE 101 0", "9 7 FREE 102 0", "10 7 FREE 103 0",
    ])
    probe = cl.Pod(64 << 20, nstreams=1)
    for t, p in enumerate(paths):
        probe.set_tensor(t, "file://" + p, (n,))
    with pytest.raises(px.PhxError, match="not bound"):  # kernel id 9 not bound there
        probe.run(seg)
    probe.close()
    pod.set_kernel_function(9, px.module_get_function(mod, "add"), 32)
    stats = pod.run(seg)
    assert stats["compute"] == 1 and stats["load"] == 2 and stats["store"] == 1
    got = np.fromfile(paths[2], np.float32)
    assert np.array_equal(got.view(np.uint32), (x + y).view(np.uint32))
    pod.close()
    px.module_unload(mod)


def _job_files(workdir, M, N, K):
    paths = {t: os.path.join(workdir, f"{n}.tensor") for t, n in ((cl.A, "a"), (cl.B, "b"), (cl.C, "c"))}
    shapes = {cl.A: (M, K), cl.B: (K, N), cl.C: (M, N)}
    for t, seed in ((cl.A, 1), (cl.B, 2), (cl.C, 3)):
        cl.init_tensor(paths[t], shapes[t], "random", seed)
    return paths, shapes


def _pod_for(paths, shapes, arena_bytes):
    pod = cl.Pod(arena_bytes, 2)
    for t in (cl.A, cl.B, cl.C):
        pod.set_tensor(t, "file://" + paths[t], shapes[t])
    pod.set_kernel(cl.STEP_LEAF, cl.MATMUL)
    pod.set_kernel(cl.INIT_LEAF, cl.MATMUL_INIT)
    return pod


def _check_c(paths, M, N, K):
    A = oracle.lcg_f32(1, M * K).reshape(M, K)
    B = oracle.lcg_f32(2, K * N).reshape(K, N)
    C = oracle.lcg_f32(3, M * N).reshape(M, N)
    got = np.fromfile(paths[cl.C], np.float32).reshape(M, N)
    want = oracle.gemm_full(A, B, C, 0.125, 1.5)
    rel = np.abs(got - want) / np.abs(want)
    assert rel.max() < 1e-4, rel.max()


def test_several_pods_own_c_supertiles(px_gpu, tmp_path):
    # cluster_correctness.rs:432-482 runs N in-process nodes on one GPU; here
    # three pods, each owning the C supertiles (pm*gn + pn) % 3 == rank (the
    # planner's block-cyclic owner-computes), run concurrently and write
    # disjoint regions of the same C file.
    import threading
    M = N = K = 768
    TM, TN, TK = 256, 256, 256
    paths, shapes = _job_files(str(tmp_path), M, N, K)
    gn = N // TN
    errors, stats = [], [None] * 3

    def node(rank):
        try:
            ins = cl.lower_matmul(M, N, K, TM, TN, TK, 0.125, 1.5,
                                  owns=lambda pm, pn: (pm * gn + pn) % 3 == rank)
            pod = _pod_for(paths, shapes, 64 << 20)
            try:
                stats[rank] = (pod.run(cl.segment_text(ins)), cl.count_ops(ins))
            finally:
                pod.close()
        except Exception as e:  # reported below
            errors.append((rank, e))

    threads = [threading.Thread(target=node, args=(r,)) for r in range(3)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    assert sum(st["compute"] for st, _ in stats) == (M // TM) * (N // TN) * (1 + K // TK)
    for st, c in stats:
        assert st["store"] == c["STORE"] == 3 and st["compute"] == c["COMPUTE"]
    _check_c(paths, M, N, K)


def test_job_split_into_segments_under_a_small_arena(px_gpu, tmp_path):
    # budgeted.rs:53-137: a job larger than the pod's memory budget runs as
    # more than one segment.  The arena holds one C row of supertiles with
    # its A panel and all of B (24 of the job's 48 supertiles), so the 4 x 4
    # supertile job runs as 4 segments, one per C supertile row, in turn,
    # each reusing the memory the previous one freed.
    M = N = K = 1024
    TM, TN, TK = 256, 256, 256
    paths, shapes = _job_files(str(tmp_path), M, N, K)
    st_bytes = 4 * TM * TK
    arena = st_bytes * (4 + 16 + 4) + (1 << 20)   # A row panel + all of B + a C row
    full = 4 * (M * K + K * N + M * N)
    assert arena < full
    pod = _pod_for(paths, shapes, arena)
    try:
        total = 0
        for row in range(M // TM):
            ins = cl.lower_matmul(M, N, K, TM, TN, TK, 0.125, 1.5, owns=lambda pm, pn: pm == row)
            total += pod.run(cl.segment_text(ins))["compute"]
        assert total == (M // TM) * (N // TN) * (1 + K // TK)
    finally:
        pod.close()
    _check_c(paths, M, N, K)


def test_io_errors_return_promptly_and_release_the_segment(px_gpu, tmp_path):
    # Eight LOADs of a file that does not exist finish on the I/O pool at
    # about the same time.  The segment fails with PHX_E_IO without waiting
    # on them forever, and gives back its tiles and staging: the same pod
    # then runs a good segment that reuses the tile ids.
    import time
    px = px_gpu
    n = 1024
    good = str(tmp_path / "good.bin")
    out = str(tmp_path / "out.bin")
    x = oracle.lcg_f32(7, n)
    x.tofile(good)
    np.zeros(n, np.float32).tofile(out)
    pod = cl.Pod(64 << 20, nstreams=2)
    pod.set_tensor(0, "file://" + str(tmp_path / "missing.bin"), (n,))
    pod.set_tensor(1, "file://" + good, (n,))
    pod.set_tensor(2, "file://" + out, (n,))
    bad = [f"{i} - ALLOC {100 + i} {n} f32" for i in range(1, 9)]
    bad += [f"{10 + i} {i} LOAD {100 + i} 0 0 {n}" for i in range(1, 9)]
    t0 = time.monotonic()
    with pytest.raises(cl.PhxError) as e:
        pod.run("\n".join(bad) + "\n")
    assert time.monotonic() - t0 < 10
    assert e.value.code == 1005 and "missing.bin" in str(e.value)
    seg = "\n".join(["1 - ALLOC 101 1024 f32", "2 1 LOAD 101 1 0 1024",
                     "3 2 STORE 101 2 0 1024", "4 3 FREE 101 0"]) + "\n"
    stats = pod.run(seg)
    assert stats["load"] == 1 and stats["store"] == 1
    assert np.array_equal(np.fromfile(out, np.float32).view(np.uint32), x.view(np.uint32))
    pod.close()


def test_flat_region_over_a_2d_tensor(px_gpu, tmp_path):
    # A rank-1 region over a rank-2 tensor is a flat element range
    # (storage.rs:22-79 byte_spans): 0..R*C covers the whole tensor, and an
    # offset of half the elements the second half.
    R, C = 32, 32
    src, dst = str(tmp_path / "src.bin"), str(tmp_path / "dst.bin")
    x = oracle.lcg_f32(8, R * C)
    x.tofile(src)
    np.zeros(R * C, np.float32).tofile(dst)
    pod = cl.Pod(16 << 20, nstreams=1)
    pod.set_tensor(0, "file://" + src, (R, C))
    pod.set_tensor(1, "file://" + dst, (R, C))
    half = R * C // 2
    seg = "\n".join([
        f"1 - ALLOC 201 {R * C} f32", f"2 - ALLOC 202 {half} f32",
        f"3 1 LOAD 201 0 0 {R * C}", f"4 2 LOAD 202 0 {half} {half}",
        f"5 3 STORE 201 1 0 {R * C}", f"6 4,5 STORE 202 1 0 {half}",
        "7 6 FREE 201 0", "8 6 FREE 202 0"]) + "\n"
    pod.run(seg)
    got = np.fromfile(dst, np.float32)
    want = np.concatenate([x[half:], x[half:]])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    pod.close()


@pytest.mark.gpu
def test_multi_chunk_transfers(px_gpu, tmp_path):
    # Tiles larger than one staging chunk (8 MiB) move chunk by chunk: a
    # 2900 x 2400 region (27.8 MB, rows of 9600 bytes straddling chunk
    # boundaries) and a flat 2500001-element region (two chunks and a ragged
    # tail) go file -> device -> file unchanged.  The pod runs the segment
    # twice, then a segment whose LOAD fails, then the good one again, so
    # staging buffers come back after success and after failure alike.
    R, C = 3000, 2500
    src, dst, fsrc, fdst = (str(tmp_path / n) for n in ("s.bin", "d.bin", "fs.bin", "fd.bin"))
    x = oracle.lcg_f32(9, R * C)
    x.tofile(src)
    x.tofile(fsrc)
    pod = cl.Pod(64 << 20, nstreams=2)
    pod.set_tensor(0, "file://" + src, (R, C))
    pod.set_tensor(1, "file://" + dst, (R, C))
    pod.set_tensor(2, "file://" + fsrc, (R * C,))
    pod.set_tensor(3, "file://" + fdst, (R * C,))
    pod.set_tensor(4, "file://" + str(tmp_path / "missing.bin"), (R, C))
    n = 2500001
    seg = "\n".join([
        "1 - ALLOC 301 2900x2400 f32", f"2 - ALLOC 302 {n} f32",
        "3 1 LOAD 301 0 7,13 2900,2400", f"4 2 LOAD 302 2 123 {n}",
        "5 3 STORE 301 1 50,61 2900,2400", f"6 4 STORE 302 3 1000 {n}",
        "7 5 FREE 301 0", "8 6 FREE 302 0"]) + "\n"
    bad = seg.replace("LOAD 301 0 7,13", "LOAD 301 4 7,13")
    xm = x.reshape(R, C)
    for run in ("good", "good", "bad", "good"):
        np.zeros(R * C, np.float32).tofile(dst)
        np.zeros(R * C, np.float32).tofile(fdst)
        if run == "bad":
            with pytest.raises(cl.PhxError):
                pod.run(bad)
            continue
        st = pod.run(seg)
        assert st["load"] == 2 and st["store"] == 2
        got = np.fromfile(dst, np.float32).reshape(R, C)
        want = np.zeros((R, C), np.float32)
        want[50:2950, 61:2461] = xm[7:2907, 13:2413]
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        gf = np.fromfile(fdst, np.float32)
        wf = np.zeros(R * C, np.float32)
        wf[1000:1000 + n] = x[123:123 + n]
        assert np.array_equal(gf.view(np.uint32), wf.view(np.uint32))
    pod.close()
