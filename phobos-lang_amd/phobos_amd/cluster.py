"""One-pod segment for the matmul_cluster job, and a Pod wrapper.

`lower_matmul` produces the instruction list a phobos scheduler hands to a
single pod for examples/matmul_cluster_fp32.ph, following the planner's rules
(phobos-sched/src/lib.rs):
  * supertile grid points in row-major order, last axis fastest
    (`advance`, lib.rs:287-296);
  * per point: the init leaf on C(pm,pn), then one step leaf per K supertile
    (clustergen.rs:1292-1399; leaf 0 = step "matmul", leaf 1 = "matmul_init");
  * lowering per compute (lib.rs:640-800): ALLOC a supertile on first use,
    LOAD it if it is read or read-modify-written, COMPUTE with deps on each
    argument's last writer, then STORE+FREE an output (or FREE an input after
    its consumers) at its last use;
  * TileId = tensor<<52 | version<<36 | linear supertile coord (tile.rs:5-30);
  * leaf grid = supertile / first @autotune choice (32), cta 256
    (lib.rs:380-429).

The text form of a segment is one instruction per line:
  <iid> <deps|-> ALLOC   <tile> <d0xd1> f32
  <iid> <deps>   LOAD    <tile> <tensor> <off0,off1> <s0,s1>
  <iid> <deps>   COMPUTE <kernel> <tile:r|w|rmw,...> <pos:f32:0xBITS,...|-> <gx,gy,gz> <cx,cy,cz>
  <iid> <deps>   STORE   <tile> <tensor> <off0,off1> <s0,s1>
  <iid> <deps>   FREE    <tile> <expected_serves>
"""
import ctypes
import os

import numpy as np

from . import (MATMUL, MATMUL_INIT, PhxError, check, f32_bits, lib)

A, B, C = 0, 1, 2
STEP_LEAF, INIT_LEAF = 0, 1
LEAF_DEVICE_TILE = 32    # first @autotune choice of TILE_M / TILE_N
LEAF_CTA = (256, 1, 1)


def tile_id(tensor, version, coord):
    assert tensor < (1 << 12) and coord < (1 << 36)
    return (tensor << 52) | (version << 36) | coord


def lower_matmul(M, N, K, TM, TN, TK, alpha, beta, c_rmw=True, version=0, owns=None):
    """Instruction list (list of dicts) of the single-node plan.

    c_rmw=True is the alpha/beta GEMM (C read-modify-write, init leaf
    C = beta*C); c_rmw=False is a plain `C = acc` kernel (C write-only, no
    LOAD of C, zero-init leaf), the form the planner's own tests pin.
    owns(pm, pn) -> bool keeps only the C supertiles a node owns (the
    planner's owner-computes split, phobos-sched/src/lib.rs:217, 238); the
    A and B supertiles they read are loaded by that node's segment."""
    assert M % TM == 0 and N % TN == 0 and K % TK == 0
    gm, gn, gk = M // TM, N // TN, K // TK
    super_shape = {A: (TM, TK), B: (TK, TN), C: (TM, TN)}
    super_grid = {A: (gm, gk), B: (gk, gn), C: (gm, gn)}
    mode_of = {A: "r", B: "r", C: "rmw" if c_rmw else "w"}

    def lin(t, coords):
        v = 0
        for c, g in zip(coords, super_grid[t]):
            v = v * g + c
        return v

    computes = []
    for pm in range(gm):
        for pn in range(gn):
            if owns is not None and not owns(pm, pn):
                continue
            scal = [(1, beta)] if c_rmw else []
            computes.append((INIT_LEAF, [(C, (pm, pn), "rmw" if c_rmw else "w")], scal))
            for k in range(gk):
                computes.append((STEP_LEAF, [(A, (pm, k), "r"), (B, (k, pn), "r"),
                                             (C, (pm, pn), "rmw")],
                                 [(3, alpha), (4, beta)]))
    last_use = {}
    for pos, (_, args, _) in enumerate(computes):
        for (t, co, _) in args:
            last_use[(t, lin(t, co))] = pos

    grid = (TM // LEAF_DEVICE_TILE, TN // LEAF_DEVICE_TILE, 1)
    out = []
    iid = [0]

    def nxt():
        iid[0] += 1
        return iid[0]

    slots = {}
    for pos, (leaf, args, scal) in enumerate(computes):
        deps = []
        for (t, co, mode) in args:
            key = (t, lin(t, co))
            if key not in slots:
                tid = tile_id(t, version, key[1])
                a = nxt()
                out.append({"iid": a, "deps": [], "op": "ALLOC", "tile": tid,
                            "shape": super_shape[t]})
                last_write = None
                if mode_of[t] in ("r", "rmw"):
                    ld = nxt()
                    out.append({"iid": ld, "deps": [a], "op": "LOAD", "tile": tid, "tensor": t,
                                "offset": tuple(c * s for c, s in zip(co, super_shape[t])),
                                "shape": super_shape[t]})
                    last_write = ld
                slots[key] = {"tile": tid, "alloc": a, "last_write": last_write, "consumers": []}
            s = slots[key]
            if mode in ("r", "rmw"):
                assert s["last_write"] is not None, "read before produced"
                deps.append(s["last_write"])
            else:
                deps.append(s["alloc"])
        deps = sorted(set(deps))
        ci = nxt()
        out.append({"iid": ci, "deps": deps, "op": "COMPUTE", "kernel": leaf,
                    "args": [(slots[(t, lin(t, co))]["tile"], m) for (t, co, m) in args],
                    "scalars": scal, "grid": grid, "cta": LEAF_CTA})
        for (t, co, mode) in args:
            s = slots[(t, lin(t, co))]
            if mode in ("w", "rmw"):
                s["last_write"] = ci
            else:
                s["consumers"].append(ci)
        for (t, co, _) in args:
            key = (t, lin(t, co))
            if last_use[key] != pos:
                continue
            s = slots[key]
            if mode_of[t] in ("w", "rmw"):
                st = nxt()
                out.append({"iid": st, "deps": [s["last_write"]], "op": "STORE",
                            "tile": s["tile"], "tensor": t,
                            "offset": tuple(c * sz for c, sz in zip(co, super_shape[t])),
                            "shape": super_shape[t]})
                out.append({"iid": nxt(), "deps": [st], "op": "FREE", "tile": s["tile"],
                            "serves": 0})
            else:
                out.append({"iid": nxt(), "deps": list(s["consumers"]), "op": "FREE",
                            "tile": s["tile"], "serves": 0})
    return out


def segment_text(instrs):
    """Renders an instruction list in the executor's text form."""
    lines = []
    for i in instrs:
        deps = ",".join(str(d) for d in i["deps"]) or "-"
        head = f"{i['iid']} {deps} {i['op']}"
        if i["op"] == "ALLOC":
            lines.append(f"{head} {i['tile']:#x} {'x'.join(map(str, i['shape']))} f32")
        elif i["op"] in ("LOAD", "STORE"):
            lines.append(f"{head} {i['tile']:#x} {i['tensor']} "
                         f"{','.join(map(str, i['offset']))} {','.join(map(str, i['shape']))}")
        elif i["op"] == "COMPUTE":
            args = ",".join(f"{t:#x}:{m}" for t, m in i["args"])
            sc = ",".join(f"{p}:f32:{f32_bits(v):#x}" for p, v in i["scalars"]) or "-"
            g = ",".join(map(str, i["grid"]))
            c = ",".join(map(str, i["cta"]))
            lines.append(f"{head} {i['kernel']} {args} {sc} {g} {c}")
        else:
            lines.append(f"{head} {i['tile']:#x} {i['serves']}")
    return "\n".join(lines) + "\n"


# ------------------------------------------------------------ wire format
# proto3 encoding of phobos.v1.Segment and JobManifest
# (phobos-cluster/proto/v1/phobos_v1_isa.proto, phobos_v1_scheduler.proto):
# fields in field-number order, repeated scalars packed, default values
# omitted -- the canonical form protobuf libraries write.
def _varint(v):
    v &= (1 << 64) - 1
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        out.append(b | (0x80 if v else 0))
        if not v:
            return bytes(out)


def _key(field, wt):
    return _varint((field << 3) | wt)


def _u(field, v):
    return _key(field, 0) + _varint(v) if v else b""


def _msg(field, body, keep_empty=False):
    if not body and not keep_empty:
        return b""
    return _key(field, 2) + _varint(len(body)) + body


def _packed(field, vals):
    return _msg(field, b"".join(_varint(v) for v in vals))


_AM = {"r": 1, "w": 2, "rmw": 3}
_OPS = {"ALLOC": 1, "LOAD": 2, "COMPUTE": 4, "STORE": 5, "FREE": 6}


def _region(offset, shape):
    return _packed(1, offset) + _packed(2, shape)


def _operation(i):
    op = i["op"]
    if op == "ALLOC":
        body = _u(1, i["tile"]) + _packed(2, i["shape"]) + _u(3, 2)        # DATA_TYPE_F32
    elif op in ("LOAD", "STORE"):
        ref = _u(1, i["tensor"]) + _msg(2, _region(i["offset"], i["shape"]), True)
        body = _u(1, i["tile"]) + _msg(2, ref, True)
    elif op == "COMPUTE":
        body = _u(1, i["kernel"])
        for t, m in i["args"]:
            body += _msg(2, _u(1, t) + _u(2, _AM[m]), True)
        dim = lambda d: _u(1, d[0]) + _u(2, d[1]) + _u(3, d[2])
        body += _msg(3, dim(i["grid"]), True) + _msg(4, dim(i["cta"]), True)
        for pos, val in i["scalars"]:
            sv = _key(1, 5) + int(f32_bits(val)).to_bytes(4, "little")   # ScalarValue.f32
            body += _msg(5, _u(1, pos) + _msg(2, sv, True), True)
    else:  # FREE
        body = _u(1, i["tile"]) + _u(2, i.get("serves", 0))
    return _msg(_OPS[op], body, True)


def segment_pb(instrs, segment_id=0):
    """Encodes an instruction list as a phobos.v1.Segment."""
    out = _u(1, segment_id)
    for i in instrs:
        out += _msg(2, _u(1, i["iid"]) + _packed(2, i["deps"]) + _msg(3, _operation(i), True),
                    True)
    return out


def manifest_pb(tensors, kernels):
    """Encodes a phobos.v1.JobManifest: tensors [(index, uri, shape)] (f32),
    kernels [(index, hash, name)]."""
    out = b""
    for idx, uri, shape in tensors:
        out += _msg(1, _u(1, idx) + _msg(2, uri.encode()) + _u(3, 2) + _packed(4, shape), True)
    for idx, h, name in kernels:
        out += _msg(2, _u(1, idx) + _msg(2, h.encode()) + _msg(3, name.encode()), True)
    return out


def count_ops(instrs):
    out = {}
    for i in instrs:
        out[i["op"]] = out.get(i["op"], 0) + 1
    return out


# ------------------------------------------------------------------ tensors
def init_tensor(path, shape, fill="random", seed=1, value=0.0):
    """phobos-tensor `init` (phobos-cluster/src/bin/phobos-tensor.rs:41-83):
    raw little-endian f32, filled with zeros, Lcg(seed) uniforms, a constant or
    iota, written chunk by chunk."""
    from .tensor import init
    init("file://" + os.path.abspath(path), list(shape), fill, value, seed)


def read_region(path, tensor_shape, offset, shape):
    """storage::load_f32 (phobos-cluster/src/storage.rs:48-60) in numpy."""
    mm = np.memmap(path, np.float32, "r", shape=tuple(tensor_shape))
    sl = tuple(slice(o, o + s) for o, s in zip(offset, shape))
    return np.array(mm[sl])


# ------------------------------------------------------------------ pod
STATS = ("alloc", "load", "compute", "store", "free", "compute_ns", "wall_ns", "io_ns")


class Pod:
    """A one-GPU pod (phx_pod_*): arena + streams + async LOAD/STORE."""

    def __init__(self, arena_bytes, nstreams=4):
        h = ctypes.c_void_p()
        check(lib().phx_pod_create(ctypes.byref(h), arena_bytes, nstreams))
        self.h = h.value

    def set_tensor(self, tensor, uri, shape):
        arr = (ctypes.c_uint64 * len(shape))(*shape)
        check(lib().phx_pod_set_tensor(self.h, tensor, uri.encode(), arr, len(shape)))

    def set_kernel(self, kernel_id, builtin):
        check(lib().phx_pod_set_kernel(self.h, kernel_id, builtin))

    def set_kernel_function(self, kernel_id, function, index_bits=32):
        """Binds a kernel id to a loaded function (module_load_data /
        module_get_function); its COMPUTEs use their own grid and cta."""
        check(lib().phx_pod_set_kernel_function(self.h, kernel_id, function, index_bits))

    def run(self, text):
        st = (ctypes.c_uint64 * 8)()
        check(lib().phx_pod_run_segment(self.h, text.encode(), st))
        return dict(zip(STATS, list(st)))

    def arena_stats(self):
        """(capacity, bump offset, base address) of the pod's device arena."""
        a = ctypes.c_void_p()
        check(lib().phx_pod_get_arena(self.h, ctypes.byref(a)))
        cap, bump, base = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_uint64()
        check(lib().phx_arena_stats(a, ctypes.byref(cap), ctypes.byref(bump), ctypes.byref(base)))
        return cap.value, bump.value, base.value

    def set_manifest_pb(self, data):
        """Applies an encoded phobos.v1.JobManifest (tensors, kernels)."""
        check(lib().phx_pod_set_manifest_pb(self.h, data, len(data)))

    def run_pb(self, data):
        """Runs an encoded phobos.v1.Segment."""
        st = (ctypes.c_uint64 * 8)()
        check(lib().phx_pod_run_segment_pb(self.h, data, len(data), st))
        return dict(zip(STATS, list(st)))

    def close(self):
        if self.h:
            lib().phx_pod_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def run_matmul_job(workdir, M, N, K, TM, TN, TK, alpha, beta, arena_bytes=None, nstreams=4,
                   make_inputs=True):
    """Seeds A, B, C (Lcg seeds 1, 2, 3) as file:// tensors in workdir, runs
    the one-pod segment and returns (stats, paths, instrs)."""
    paths = {t: os.path.join(workdir, f"{n}.tensor") for t, n in ((A, "a"), (B, "b"), (C, "c"))}
    shapes = {A: (M, K), B: (K, N), C: (M, N)}
    if make_inputs:
        for t, seed in ((A, 1), (B, 2), (C, 3)):
            init_tensor(paths[t], shapes[t], "random", seed)
    instrs = lower_matmul(M, N, K, TM, TN, TK, alpha, beta)
    if arena_bytes is None:  # every supertile resident at once
        arena_bytes = 4 * (M * K + K * N + M * N) + (1 << 20)
    pod = Pod(arena_bytes, nstreams)
    try:
        for t in (A, B, C):
            pod.set_tensor(t, "file://" + paths[t], shapes[t])
        pod.set_kernel(STEP_LEAF, MATMUL)
        pod.set_kernel(INIT_LEAF, MATMUL_INIT)
        stats = pod.run(segment_text(instrs))
    finally:
        pod.close()
    return stats, paths, instrs
