"""CPU oracle for the phobos leaf kernels -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker (or the timed CPU baseline).  The product
path (libphobos_hip.so and the gfx950 code objects) never calls it.

The C restatement lives in oracle.c (built into liboracle.so by the Makefile
beside it); this module is a thin ctypes/numpy wrapper.  Each function names the
reference file:line it restates.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_sz = ctypes.c_size_t


def build():
    """Compile liboracle.so in place (gcc; no GPU needed)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        L.orc_lcg_fill_f32.argtypes = [ctypes.c_uint64, _sz, _f32p]
        L.orc_lcg_u64.argtypes = [ctypes.c_uint64, _sz, _u64p]
        L.orc_normal_fill_f32.argtypes = [ctypes.c_uint64, _sz, ctypes.c_double, _f32p]
        L.orc_f32_to_f16_bits.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16_bits.restype = ctypes.c_uint16
        L.orc_f16_round.argtypes = [ctypes.c_float]
        L.orc_f16_round.restype = ctypes.c_float
        L.orc_f16_round_array.argtypes = [_sz, _f32p, _f32p]
        L.orc_f32_to_f16_array.argtypes = [_sz, _f32p, _u16p]
        L.orc_f16_to_f32_array.argtypes = [_sz, _u16p, _f32p]
        L.orc_saxpy.argtypes = [_sz, ctypes.c_float, _f32p, _f32p, _f32p]
        L.orc_saxpy_mt.argtypes = [_sz, ctypes.c_float, _f32p, _f32p, _f32p]
        L.orc_sample_points.argtypes = [_sz, _sz, _sz, _u64p, _u64p]
        L.orc_gemm_points_f64.argtypes = [_sz, _u64p, _u64p, _sz, _f32p, _sz, _f32p, _sz,
                                          _f32p, _sz, ctypes.c_double, ctypes.c_double,
                                          ctypes.c_int, _f64p]
        L.orc_gemm_full_f64.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _f32p, ctypes.c_double,
                                        ctypes.c_double, ctypes.c_int, _f64p]
        L.orc_gemm_fp16acc_point.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _sz, _f32p,
                                             ctypes.c_float, ctypes.c_float]
        L.orc_gemm_fp16acc_point.restype = ctypes.c_float
        L.orc_flash_rows_f64.argtypes = [_sz, _u64p, _sz, _sz, _f32p, _f32p, _f32p,
                                         ctypes.c_double, _f64p]
        L.orc_flash_heads_f64.argtypes = [_sz, _sz, _sz, _sz, _f32p, _f32p, _f32p,
                                          ctypes.c_double, _f64p]
        L.orc_matmul_init.argtypes = [_sz, ctypes.c_float, _f32p]
        L.orc_matmul_step_epilogue.argtypes = [_sz, ctypes.c_float, _f32p, _f32p]
        L.orc_sgemm_f32.argtypes = [_sz, _sz, _sz, ctypes.c_float, _f32p, _f32p,
                                    ctypes.c_float, _f32p]
        L.orc_flash_f32.argtypes = [_sz, _sz, _sz, _sz, _f32p, _f32p, _f32p, ctypes.c_float,
                                    _f32p]
        L.orc_num_threads.restype = ctypes.c_int
        _LIB = L
    return _LIB


def _p(a, t):
    return a.ctypes.data_as(t)


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- inputs
def lcg_f32(seed, n):
    """Lcg::unit_f32s (phobos-base/src/rng.rs:9-25)."""
    out = np.empty(n, np.float32)
    lib().orc_lcg_fill_f32(seed, n, _p(out, _f32p))
    return out


def lcg_u64(seed, n):
    out = np.empty(n, np.uint64)
    lib().orc_lcg_u64(seed, n, _p(out, _u64p))
    return out


def normal_f32(seed, n, scale=1.0):
    """Box-Muller over Lcg draws (this build's convention, see oracle.c)."""
    out = np.empty(n, np.float32)
    lib().orc_normal_fill_f32(seed, n, scale, _p(out, _f32p))
    return out


def f16_bits(x):
    """f32 -> IEEE f16 bit patterns, RNE (main.rs:447-449, half::f16::from_f32)."""
    x = _c32(x).ravel()
    out = np.empty(x.size, np.uint16)
    lib().orc_f32_to_f16_array(x.size, _p(x, _f32p), _p(out, _u16p))
    return out


def f16_to_f32(bits):
    bits = np.ascontiguousarray(bits, dtype=np.uint16).ravel()
    out = np.empty(bits.size, np.float32)
    lib().orc_f16_to_f32_array(bits.size, _p(bits, _u16p), _p(out, _f32p))
    return out


def f16_round(x):
    x = _c32(x)
    out = np.empty_like(x)
    lib().orc_f16_round_array(x.size, _p(x, _f32p), _p(out, _f32p))
    return out


# ---------------------------------------------------------------- kernels
def saxpy(alpha, x, y):
    """out = fl(fl(alpha*x) + y) (saxpy_fp32.ph:1-5, main.rs:1176-1188)."""
    x, y = _c32(x), _c32(y)
    out = np.empty_like(x)
    lib().orc_saxpy(x.size, alpha, _p(x, _f32p), _p(y, _f32p), _p(out, _f32p))
    return out


def saxpy_mt(alpha, x, y):
    """saxpy over the host cores (OpenMP); the same bits as saxpy()."""
    x, y = _c32(x), _c32(y)
    out = np.empty_like(x)
    lib().orc_saxpy_mt(x.size, alpha, _p(x, _f32p), _p(y, _f32p), _p(out, _f32p))
    return out


def sample_points(M, N, count=64):
    """xorshift64 sampler of main.rs:399-410."""
    r = np.empty(count, np.uint64)
    c = np.empty(count, np.uint64)
    lib().orc_sample_points(M, N, count, _p(r, _u64p), _p(c, _u64p))
    return r, c


def gemm_points(rows, cols, A, B, Cin, alpha, beta, round16=False):
    """f64 alpha*A@B + beta*Cin at given points (main.rs:411-436)."""
    A, B = _c32(A), _c32(B)
    M, K = A.shape
    N = B.shape[1]
    rows = np.ascontiguousarray(rows, np.uint64)
    cols = np.ascontiguousarray(cols, np.uint64)
    out = np.empty(rows.size, np.float64)
    cp = None
    if Cin is not None:
        Cin = _c32(Cin)
        cp = _p(Cin, _f32p)
    lib().orc_gemm_points_f64(rows.size, _p(rows, _u64p), _p(cols, _u64p), K, _p(A, _f32p), K,
                              _p(B, _f32p), N, cp, N, alpha, beta, int(round16),
                              _p(out, _f64p))
    return out


def gemm_full(A, B, Cin, alpha, beta, round16=False):
    """Full f64 alpha*A@B + beta*Cin (same arithmetic as gemm_points)."""
    A, B = _c32(A), _c32(B)
    M, K = A.shape
    N = B.shape[1]
    out = np.empty((M, N), np.float64)
    cp = None
    if Cin is not None:
        Cin = _c32(Cin)
        cp = _p(Cin, _f32p)
    lib().orc_gemm_full_f64(M, N, K, _p(A, _f32p), _p(B, _f32p), cp, alpha, beta,
                            int(round16), _p(out, _f64p))
    return out


def gemm_fp16acc_point(i, j, A, B, Cin, alpha, beta):
    """Reference's sequential f16-accumulate model (main.rs:659-672)."""
    A, B = _c32(A), _c32(B)
    K = A.shape[1]
    N = B.shape[1]
    cp = None
    if Cin is not None:
        Cin = _c32(Cin)
        cp = _p(Cin, _f32p)
    return lib().orc_gemm_fp16acc_point(i, j, K, _p(A, _f32p), _p(B, _f32p), N, cp, alpha, beta)


def flash_rows(rows, q, k, v, scale):
    """f64 online-softmax replay (main.rs:894-911) for the given rows of one head."""
    q, k, v = _c32(q), _c32(k), _c32(v)
    Nk, D = k.shape
    rows = np.ascontiguousarray(rows, np.uint64)
    out = np.empty((rows.size, D), np.float64)
    lib().orc_flash_rows_f64(rows.size, _p(rows, _u64p), Nk, D, _p(q, _f32p), _p(k, _f32p),
                             _p(v, _f32p), scale, _p(out, _f64p))
    return out


def flash_heads(q, k, v, scale):
    """f64 online softmax for all rows of [heads, N, D] tensors."""
    q, k, v = _c32(q), _c32(k), _c32(v)
    H, Nq, D = q.shape
    Nk = k.shape[1]
    out = np.empty((H, Nq, D), np.float64)
    lib().orc_flash_heads_f64(H, Nq, Nk, D, _p(q, _f32p), _p(k, _f32p), _p(v, _f32p), scale,
                              _p(out, _f64p))
    return out


def matmul_init(beta, c):
    """matmul_init leaf: C = fl(beta*C) (clustergen.rs:1292-1360)."""
    c = _c32(c).copy()
    lib().orc_matmul_init(c.size, beta, _p(c, _f32p))
    return c


def matmul_step_epilogue(alpha, acc, c):
    """matmul step leaf store: C = fl(fl(alpha*acc) + C) (clustergen.rs:1369-1399)."""
    acc, c = _c32(acc), _c32(c).copy()
    lib().orc_matmul_step_epilogue(c.size, alpha, _p(acc, _f32p), _p(c, _f32p))
    return c


# ------------------------------------------------------------ CPU baselines
def sgemm_f32(alpha, A, B, beta, C):
    A, B = _c32(A), _c32(B)
    C = _c32(C).copy()
    M, K = A.shape
    N = B.shape[1]
    lib().orc_sgemm_f32(M, N, K, alpha, _p(A, _f32p), _p(B, _f32p), beta, _p(C, _f32p))
    return C


def flash_f32(q, k, v, scale):
    q, k, v = _c32(q), _c32(k), _c32(v)
    H, Nq, D = q.shape
    Nk = k.shape[1]
    o = np.empty_like(q)
    lib().orc_flash_f32(H, Nq, Nk, D, _p(q, _f32p), _p(k, _f32p), _p(v, _f32p), scale,
                        _p(o, _f32p))
    return o


def num_threads():
    return lib().orc_num_threads()
