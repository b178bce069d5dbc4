"""Python host mirror of the phobos leaf-kernel launch interface on MI355X.

This is a thin ctypes layer over libphobos_hip.so (the C ABI in
include/phobos_hip.h).  It mirrors the reference's host-side launch helpers:

  launch_saxpy  -- phobos-bench/src/main.rs:1227-1239 (the saxpy launch! call)
  launch_gemm   -- phobos-bench/src/main.rs:290-327
  launch_flash  -- phobos-bench/src/main.rs:334-371
  compute       -- phobos-pod/src/engine.rs:582-647 (exploded-memref marshalling)

Every call goes to the gfx950 code objects through hipModuleLaunchKernel.
There is no CPU fallback: if the library or a code object is missing, or no
GPU is present, the call raises.
"""
import ctypes
import os
import re

import numpy as np

_PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(_PKG)  # phobos-lang_amd/
LIB_DIR = os.path.join(ROOT, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libphobos_hip.so")
HEADER = os.path.join(os.path.dirname(ROOT), "include", "phobos_hip.h")

# phx_kernel ids (include/phobos_hip.h)
SAXPY_FP32 = 0
GEMM_FP32 = 1
GEMM_FP16TC_FP32ACC = 2
GEMM_FP16 = 3
FLASH_FP32 = 4
FLASH_FP16 = 5
MATMUL = 6
MATMUL_INIT = 7
FLASH_FP32_BH = 8
FLASH_FP16_BH = 9
NUM_KERNELS = 10

KERNEL_NAMES = {
    SAXPY_FP32: "saxpy_fp32", GEMM_FP32: "gemm_fp32",
    GEMM_FP16TC_FP32ACC: "gemm_fp16tc_fp32acc", GEMM_FP16: "gemm_fp16",
    FLASH_FP32: "flash_fp32", FLASH_FP16: "flash_fp16", MATMUL: "matmul",
    MATMUL_INIT: "matmul_init", FLASH_FP32_BH: "flash_fp32_bh", FLASH_FP16_BH: "flash_fp16_bh",
}

CODE_OBJECTS = ["saxpy_fp32.hsaco", "gemm_fp32.hsaco", "gemm_fp16tc_fp32acc.hsaco",
                "gemm_fp16.hsaco", "flash_attention_fp32.hsaco", "flash_attention_fp16.hsaco",
                "matmul_cluster_fp32.hsaco"]

PHX_E_INVALID = 1001
PHX_E_NOT_INIT = 1002
PHX_E_NOT_FOUND = 1003
PHX_E_EXHAUSTED = 1004


class PhxError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"phx error {code}: {msg}")
        self.code = code


class TileArg(ctypes.Structure):
    _fields_ = [("addr", ctypes.c_uint64), ("rank", ctypes.c_uint32),
                ("shape", ctypes.c_uint64 * 3)]


class ScalarArg(ctypes.Structure):
    _fields_ = [("pos", ctypes.c_uint32), ("bytes", ctypes.c_uint32), ("bits", ctypes.c_uint64)]


_LIB = None
_INIT = False

_u64 = ctypes.c_uint64
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_u32a3 = ctypes.c_uint32 * 3


def header_symbols():
    """Every phx_* function declared in include/phobos_hip.h."""
    with open(HEADER) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(phx_[a-z0-9_]+)\s*\(", text)))


def lib():
    """Load libphobos_hip.so (raises if it has not been built)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build the backend first "
                           "(python -c 'import __graft_entry__ as g; g.build()')")
    L = ctypes.CDLL(LIB_PATH)
    L.phx_last_error.restype = ctypes.c_char_p
    L.phx_init.argtypes = [ctypes.c_int, ctypes.c_char_p]
    L.phx_device_info.argtypes = [ctypes.c_char_p, _sz, ctypes.POINTER(ctypes.c_int),
                                  ctypes.POINTER(ctypes.c_int), ctypes.POINTER(_sz),
                                  ctypes.POINTER(ctypes.c_int)]
    L.phx_malloc.argtypes = [ctypes.POINTER(_u64), _sz]
    L.phx_free.argtypes = [_u64]
    L.phx_host_alloc.argtypes = [ctypes.POINTER(_vp), _sz]
    L.phx_host_free.argtypes = [_vp]
    L.phx_memcpy_h2d.argtypes = [_u64, _vp, _sz]
    L.phx_memcpy_d2h.argtypes = [_vp, _u64, _sz]
    L.phx_kernel_by_name.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_char_p, ctypes.c_char_p]
    L.phx_launch_by_name.argtypes = [ctypes.c_char_p, ctypes.c_char_p, _vp, _vp, _vp,
                                     ctypes.POINTER(ctypes.c_void_p)]
    L.phx_memcpy_d2d.argtypes = [_u64, _u64, _sz]
    L.phx_memcpy_h2d_async.argtypes = [_u64, _vp, _sz, _vp]
    L.phx_memcpy_d2h_async.argtypes = [_vp, _u64, _sz, _vp]
    L.phx_memset_async.argtypes = [_u64, ctypes.c_int, _sz, _vp]
    L.phx_stream_create.argtypes = [ctypes.POINTER(_vp)]
    L.phx_stream_destroy.argtypes = [_vp]
    L.phx_stream_synchronize.argtypes = [_vp]
    L.phx_stream_set_workspace.argtypes = [_vp, _u64, _sz]
    L.phx_stream_get_workspace.argtypes = [_vp, ctypes.POINTER(_u64), ctypes.POINTER(_sz)]
    L.phx_event_create.argtypes = [ctypes.POINTER(_vp)]
    L.phx_event_destroy.argtypes = [_vp]
    L.phx_event_record.argtypes = [_vp, _vp]
    L.phx_event_query.argtypes = [_vp]
    L.phx_event_synchronize.argtypes = [_vp]
    L.phx_event_elapsed_ms.argtypes = [ctypes.POINTER(ctypes.c_float), _vp, _vp]
    L.phx_module_load_data.argtypes = [ctypes.POINTER(_vp), ctypes.c_char_p, _sz]
    L.phx_module_load_file.argtypes = [ctypes.POINTER(_vp), ctypes.c_char_p]
    L.phx_module_unload.argtypes = [_vp]
    L.phx_module_get_function.argtypes = [ctypes.POINTER(_vp), _vp, ctypes.c_char_p]
    L.phx_builtin_function.argtypes = [ctypes.POINTER(_vp), ctypes.c_int]
    L.phx_kernel_abi.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_int), _u32a3]
    L.phx_launch.argtypes = [_vp, _u32a3, _u32a3, ctypes.c_uint32, _vp, ctypes.POINTER(_vp)]
    L.phx_grid_for.argtypes = [ctypes.c_int, ctypes.POINTER(_i64), ctypes.c_int, _u32a3, _u32a3]
    L.phx_check_shape.argtypes = [ctypes.c_int, ctypes.POINTER(_i64), ctypes.c_int]
    L.phx_split_plan.argtypes = [ctypes.c_int, ctypes.POINTER(_i64), ctypes.c_int,
                                 ctypes.POINTER(ctypes.c_int), ctypes.POINTER(_sz)]
    L.phx_plan_get.argtypes = [ctypes.c_int, ctypes.POINTER(_i64), ctypes.c_int,
                               ctypes.POINTER(Plan)]
    L.phx_plan_pin.argtypes = [ctypes.c_int, ctypes.POINTER(_i64), ctypes.c_int,
                               ctypes.POINTER(Plan)]
    L.phx_compute.argtypes = [_vp, ctypes.c_int, ctypes.POINTER(TileArg), ctypes.c_uint32,
                              ctypes.POINTER(ScalarArg), ctypes.c_uint32, _u32a3, _u32a3, _vp]
    L.phx_saxpy.argtypes = [_vp, _u64, _u64, _u64, _i64, ctypes.c_float]
    L.phx_gemm.argtypes = [_vp, ctypes.c_int, _u64, _u64, _u64, _i64, _i64, _i64,
                           ctypes.c_float, ctypes.c_float]
    L.phx_matmul_init.argtypes = [_vp, _u64, _i64, _i64, ctypes.c_float]
    L.phx_flash_attention.argtypes = [_vp, ctypes.c_int, _u64, _u64, _u64, _u64, _i64, _i64,
                                      _i64, ctypes.c_float]
    L.phx_flash_attention_bh.argtypes = [_vp, ctypes.c_int, _u64, _u64, _u64, _u64, _i64, _i64,
                                         _i64, _i64, ctypes.c_float]
    L.phx_flash_attention_bh_noalloc.argtypes = L.phx_flash_attention_bh.argtypes
    L.phx_size_class.argtypes = [_sz]
    L.phx_size_class.restype = _sz
    L.phx_arena_create.argtypes = [ctypes.POINTER(_vp), _sz]
    L.phx_arena_destroy.argtypes = [_vp]
    L.phx_arena_alloc.argtypes = [_vp, _sz, ctypes.POINTER(_u64), ctypes.POINTER(_sz)]
    L.phx_arena_free.argtypes = [_vp, _u64, _sz]
    L.phx_arena_can_alloc.argtypes = [_vp, _sz]
    L.phx_arena_stats.argtypes = [_vp, ctypes.POINTER(_sz), ctypes.POINTER(_sz),
                                  ctypes.POINTER(_u64)]
    L.phx_lcg_fill_f32.argtypes = [_u64, _sz, ctypes.POINTER(ctypes.c_float)]
    L.phx_normal_fill_f32.argtypes = [_u64, _sz, ctypes.c_double, ctypes.POINTER(ctypes.c_float)]
    L.phx_f32_to_f16.argtypes = [_sz, ctypes.POINTER(ctypes.c_float),
                                 ctypes.POINTER(ctypes.c_uint16)]
    L.phx_f16_to_f32.argtypes = [_sz, ctypes.POINTER(ctypes.c_uint16),
                                 ctypes.POINTER(ctypes.c_float)]
    L.phx_pod_create.argtypes = [ctypes.POINTER(_vp), _sz, ctypes.c_int]
    L.phx_pod_destroy.argtypes = [_vp]
    L.phx_pod_get_arena.argtypes = [_vp, ctypes.POINTER(_vp)]
    L.phx_pod_set_tensor.argtypes = [_vp, ctypes.c_uint32, ctypes.c_char_p,
                                     ctypes.POINTER(_u64), ctypes.c_uint32]
    L.phx_pod_set_kernel.argtypes = [_vp, ctypes.c_uint32, ctypes.c_int]
    L.phx_pod_set_kernel_function.argtypes = [_vp, ctypes.c_uint32, _vp, ctypes.c_int]
    L.phx_pod_run_segment.argtypes = [_vp, ctypes.c_char_p, ctypes.POINTER(_u64)]
    L.phx_lcg_fill_f32_stream.argtypes = [ctypes.POINTER(_u64), ctypes.c_size_t, _vp]
    L.phx_pod_set_manifest_pb.argtypes = [_vp, ctypes.c_char_p, ctypes.c_size_t]
    L.phx_pod_run_segment_pb.argtypes = [_vp, ctypes.c_char_p, ctypes.c_size_t,
                                         ctypes.POINTER(_u64)]
    L.phx_segment_pb_to_text.argtypes = [ctypes.c_char_p, ctypes.c_size_t, ctypes.c_char_p,
                                         ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]
    _LIB = L
    return L


def check(rc):
    if rc != 0:
        raise PhxError(rc, lib().phx_last_error().decode(errors="replace"))


def init(device=0):
    """cust::quick_init (main.rs:169): select the device and load code objects lazily."""
    global _INIT
    if not _INIT:
        code_dir = os.environ.get("PHX_CODE_OBJECT_DIR") or LIB_DIR
        check(lib().phx_init(device, code_dir.encode()))
        _INIT = True


def device_info():
    name = ctypes.create_string_buffer(256)
    cus, clk, lds = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    hbm = _sz()
    check(lib().phx_device_info(name, 256, ctypes.byref(cus), ctypes.byref(clk),
                                ctypes.byref(hbm), ctypes.byref(lds)))
    return {"name": name.value.decode(), "cus": cus.value, "clock_khz": clk.value,
            "hbm_bytes": hbm.value, "lds_bytes_per_cu": lds.value}


def synchronize():
    check(lib().phx_device_synchronize())


# ------------------------------------------------------------------- memory
class DeviceBuffer:
    """A hipMalloc'd buffer (the reference's DeviceBuffer / as_dbuf)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = _u64()
        check(lib().phx_malloc(ctypes.byref(p), self.nbytes))
        self.ptr = p.value

    @classmethod
    def from_array(cls, arr):
        arr = np.ascontiguousarray(arr)
        b = cls(arr.nbytes)
        b.upload(arr)
        return b

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        check(lib().phx_memcpy_h2d(self.ptr, arr.ctypes.data, arr.nbytes))

    def download(self, dtype, shape):
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        check(lib().phx_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def zero(self, stream=None):
        check(lib().phx_memset_async(self.ptr, 0, self.nbytes, _sh(stream)))

    def free(self):
        if self.ptr:
            check(lib().phx_free(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            if self.ptr and _LIB is not None:
                _LIB.phx_free(self.ptr)
                self.ptr = 0
        except Exception:
            pass


class Stream:
    """A non-blocking HIP stream at default priority (main.rs:170)."""

    def __init__(self):
        h = _vp()
        check(lib().phx_stream_create(ctypes.byref(h)))
        self.handle = h.value

    def synchronize(self):
        check(lib().phx_stream_synchronize(self.handle))

    def destroy(self):
        if self.handle:
            check(lib().phx_stream_destroy(self.handle))
            buf = _WORKSPACES.pop(self.handle, None)
            if buf is not None:
                buf.free()  # the stream was drained by its destroy
            self.handle = None


class Event:
    def __init__(self):
        h = _vp()
        check(lib().phx_event_create(ctypes.byref(h)))
        self.handle = h.value

    def record(self, stream):
        check(lib().phx_event_record(self.handle, stream.handle if stream else None))

    def synchronize(self):
        check(lib().phx_event_synchronize(self.handle))

    def query(self):
        rc = lib().phx_event_query(self.handle)
        if rc not in (0, 1):
            check(rc)
        return rc == 0

    def elapsed_ms(self, later):
        ms = ctypes.c_float()
        check(lib().phx_event_elapsed_ms(ctypes.byref(ms), self.handle, later.handle))
        return ms.value

    def destroy(self):
        if self.handle:
            check(lib().phx_event_destroy(self.handle))
            self.handle = None


def _sh(stream):
    return stream.handle if isinstance(stream, Stream) else stream


# Workspaces bound by bind_workspace, kept alive while bound: stream handle -> buffer
_WORKSPACES = {}


def set_workspace(stream, addr, nbytes):
    """phx_stream_set_workspace: bind caller-owned device memory (256-byte
    aligned) as the split workspace of launches on stream (None: the legacy
    default stream); addr 0 unbinds.  The caller keeps the memory alive."""
    check(lib().phx_stream_set_workspace(_sh(stream), int(addr), int(nbytes)))


def get_workspace(stream):
    """(address, bytes) of the workspace bound to stream, (0, 0) for none."""
    a, n = _u64(), _sz()
    check(lib().phx_stream_get_workspace(_sh(stream), ctypes.byref(a), ctypes.byref(n)))
    return a.value, n.value


def bind_workspace(stream, nbytes):
    """Allocates a workspace of nbytes (hipMalloc, 256-byte aligned) and binds
    it to stream, replacing (and freeing) one an earlier call bound; nbytes 0
    unbinds.  Split launches on the stream then use it; the launches
    themselves never allocate."""
    key = _sh(stream)
    set_workspace(stream, 0, 0)
    old = _WORKSPACES.pop(key, None)
    if old is not None:
        synchronize()  # launches in flight may still use it
        old.free()
    if nbytes:
        buf = DeviceBuffer(nbytes)
        set_workspace(stream, buf.ptr, nbytes)
        _WORKSPACES[key] = buf


# ------------------------------------------------------------------- launches
def _addr(buf, nbytes, what):
    """Device address of `buf` (a DeviceBuffer or a raw address).  For a
    DeviceBuffer the size is checked against the bytes the kernel touches, so
    a wrong buffer raises on the host instead of faulting the GPU."""
    if isinstance(buf, DeviceBuffer):
        if buf.nbytes < nbytes:
            raise PhxError(PHX_E_INVALID, f"{what}: buffer holds {buf.nbytes} B, kernel "
                                          f"accesses {nbytes} B")
        return buf.ptr
    return int(buf)


# gemm_fp32's tilings by launch-plan variant (TILE_M, TILE_N, TILE_K), as
# include/phobos_hip.h lists them; variant 0 is the built-in tiling.
GEMM_FP32_TILINGS = [(256, 256, 16), (256, 128, 16), (128, 256, 16), (128, 128, 16),
                     (128, 128, 32), (128, 128, 8), (256, 256, 8), (64, 64, 16)]

_GEMM_ESZ = {GEMM_FP32: 4, GEMM_FP16TC_FP32ACC: 4, GEMM_FP16: 2, MATMUL: 4}


def launch_saxpy(stream, x, y, out, n, alpha):
    """saxpy_fp32.ph: out = alpha*x + y (main.rs:1227-1239)."""
    check(lib().phx_saxpy(_sh(stream), _addr(x, 4 * n, "x"), _addr(y, 4 * n, "y"),
                          _addr(out, 4 * n, "out"), n, alpha))


def launch_gemm(stream, kernel, a, b, c, M, N, K, alpha, beta):
    """C = alpha*A@B + beta*C for the gemm-family kernel ids (main.rs:290-327)."""
    e = _GEMM_ESZ.get(kernel, 4)
    check(lib().phx_gemm(_sh(stream), kernel, _addr(a, e * M * K, "A"), _addr(b, e * K * N, "B"),
                         _addr(c, e * M * N, "C"), M, N, K, alpha, beta))


def launch_matmul_init(stream, c, M, N, beta):
    check(lib().phx_matmul_init(_sh(stream), _addr(c, 4 * M * N, "C"), M, N, beta))


def launch_flash(stream, kernel, q, k, v, o, Nq, Nk, D, scale):
    """One-head flash attention (main.rs:334-371)."""
    e = 2 if kernel == FLASH_FP16 else 4
    check(lib().phx_flash_attention(_sh(stream), kernel, _addr(q, e * Nq * D, "Q"),
                                    _addr(k, e * Nk * D, "K"), _addr(v, e * Nk * D, "V"),
                                    _addr(o, e * Nq * D, "O"), Nq, Nk, D, scale))


def launch_flash_bh(stream, kernel, q, k, v, o, BH, Nq, Nk, D, scale):
    e = 2 if kernel == FLASH_FP16_BH else 4
    check(lib().phx_flash_attention_bh(_sh(stream), kernel, _addr(q, e * BH * Nq * D, "Q"),
                                       _addr(k, e * BH * Nk * D, "K"),
                                       _addr(v, e * BH * Nk * D, "V"),
                                       _addr(o, e * BH * Nq * D, "O"), BH, Nq, Nk, D, scale))


def grid_for(kernel, dims):
    d = (_i64 * len(dims))(*dims)
    g, b = _u32a3(), _u32a3()
    check(lib().phx_grid_for(kernel, d, len(dims), g, b))
    return tuple(g), tuple(b)


def kernel_by_name(ph_file, entry):
    """Built-in kernel id for the reference's .ph file stem and entry name."""
    k = ctypes.c_int()
    check(lib().phx_kernel_by_name(ctypes.byref(k), ph_file.encode(), entry.encode()))
    return k.value


def check_shape(kernel, dims):
    d = (_i64 * len(dims))(*dims)
    return lib().phx_check_shape(kernel, d, len(dims))


def split_plan(kernel, dims):
    """(splits, workspace bytes) of a launch of kernel over dims (phx_split_plan)."""
    d = (_i64 * len(dims))(*dims)
    sp, ws = ctypes.c_int(), _sz()
    check(lib().phx_split_plan(kernel, d, len(dims), ctypes.byref(sp), ctypes.byref(ws)))
    return sp.value, ws.value


class Plan(ctypes.Structure):
    """phx_plan: K or key chunks (1 = unsplit) and kernel variant."""
    _fields_ = [("splits", ctypes.c_int32), ("variant", ctypes.c_int32)]


def plan_get(kernel, dims):
    """(splits, variant) a launch of kernel over dims uses now (phx_plan_get)."""
    d = (_i64 * len(dims))(*dims)
    p = Plan()
    check(lib().phx_plan_get(kernel, d, len(dims), ctypes.byref(p)))
    return p.splits, p.variant


def plan_pin(kernel, dims, splits=None, variant=0):
    """Pins (splits, variant) for kernel at dims; splits None removes the pin."""
    d = (_i64 * len(dims))(*dims)
    p = None if splits is None else ctypes.byref(Plan(splits, variant))
    check(lib().phx_plan_pin(kernel, d, len(dims), p))


def plan_unpin_all():
    check(lib().phx_plan_unpin_all())


def kernel_abi(kernel):
    bits = ctypes.c_int()
    b = _u32a3()
    check(lib().phx_kernel_abi(kernel, ctypes.byref(bits), b))
    return bits.value, tuple(b)


def builtin_function(kernel):
    f = _vp()
    check(lib().phx_builtin_function(ctypes.byref(f), kernel))
    return f.value


def module_load_data(image):
    """PtxCache::insert with a gfx950 code object in place of PTX
    (phobos-pod/src/ptx_cache.rs:12-82): returns a module handle."""
    m = _vp()
    check(lib().phx_module_load_data(ctypes.byref(m), image, len(image)))
    return m.value


def module_get_function(module, name):
    f = _vp()
    check(lib().phx_module_get_function(ctypes.byref(f), module, name.encode()))
    return f.value


def module_unload(module):
    check(lib().phx_module_unload(module))


def compute(func, index_bits, tiles, scalars, grid, cta, stream=None):
    """Pod COMPUTE marshalling (engine.rs:582-647).

    tiles: [(addr, shape_tuple)], scalars: [(pos, bytes, bits)]."""
    ta = (TileArg * max(1, len(tiles)))()
    for i, (addr, shape) in enumerate(tiles):
        ta[i].addr = addr
        ta[i].rank = len(shape)
        for j, s in enumerate(shape):
            ta[i].shape[j] = s
    sa = (ScalarArg * max(1, len(scalars)))()
    for i, (pos, nbytes, bits) in enumerate(scalars):
        sa[i].pos, sa[i].bytes, sa[i].bits = pos, nbytes, bits
    check(lib().phx_compute(func, index_bits, ta, len(tiles), sa, len(scalars), _u32a3(*grid),
                            _u32a3(*cta), _sh(stream)))


def f32_bits(x):
    """ScalarValue::F32(x).to_bits() (phobos-cluster/src/tile.rs:75-84)."""
    return int(np.array([x], np.float32).view(np.uint32)[0])


# ------------------------------------------------------------------- inputs
def lcg_f32(seed, n):
    """Lcg::unit_f32s (phobos-base/src/rng.rs:9-25), generated by the library."""
    out = np.empty(n, np.float32)
    check(lib().phx_lcg_fill_f32(seed, n, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
    return out


def normal_f32(seed, n, scale=1.0):
    out = np.empty(n, np.float32)
    check(lib().phx_normal_fill_f32(seed, n, scale,
                                    out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
    return out


def to_f16_bits(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    check(lib().phx_f32_to_f16(x.size, x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                               out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))))
    return out


def from_f16_bits(bits):
    bits = np.ascontiguousarray(bits, np.uint16)
    out = np.empty(bits.shape, np.float32)
    check(lib().phx_f16_to_f32(bits.size, bits.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
                               out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
    return out


def segment_pb_to_text(data):
    """Decodes an encoded phobos.v1.Segment into the pod's text form
    (phx_segment_pb_to_text; no device needed)."""
    need = ctypes.c_size_t()
    check(lib().phx_segment_pb_to_text(data, len(data), None, 0, ctypes.byref(need)))
    buf = ctypes.create_string_buffer(need.value)
    check(lib().phx_segment_pb_to_text(data, len(data), buf, need.value, ctypes.byref(need)))
    return buf.value.decode()
