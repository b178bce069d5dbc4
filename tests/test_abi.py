"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, and its host-only logic agrees with the oracle / reference
rules.  No GPU calls."""
import ctypes
import os

import numpy as np
import pytest

import oracle
import phobos_amd as px


def test_library_exports_every_header_symbol():
    L = px.lib()
    syms = px.header_symbols()
    assert len(syms) > 40
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing


def test_code_objects_built():
    for name in px.CODE_OBJECTS:
        p = os.path.join(px.LIB_DIR, name)
        assert os.path.exists(p), p
        with open(p, "rb") as f:
            head = f.read(24)
        assert head.startswith(b"__CLANG_OFFLOAD_BUNDLE__") or head.startswith(b"\x7fELF")


def test_lcg_and_normal_match_oracle():
    for seed in (1, 2, 3, 1001):
        assert np.array_equal(px.lcg_f32(seed, 10000).view(np.uint32),
                              oracle.lcg_f32(seed, 10000).view(np.uint32))
    assert np.array_equal(px.normal_f32(5, 4097, 1 / 64).view(np.uint32),
                          oracle.normal_f32(5, 4097, 1 / 64).view(np.uint32))


def test_f16_conversion_matches_oracle():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(100000) * 10.0 ** rng.integers(-9, 6, 100000)).astype(np.float32)
    x = np.concatenate([x, np.array([0.0, -0.0, 65520.0, 65519.0, np.inf, -np.inf], np.float32)])
    assert np.array_equal(px.to_f16_bits(x), oracle.f16_bits(x))
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    fin = bits[np.isfinite(bits.view(np.float16))]
    assert np.array_equal(px.from_f16_bits(fin), oracle.f16_to_f32(fin))


def test_size_class_rules():
    # tile_store.rs:228-242
    sc = px.lib().phx_size_class
    tile = 10240 * 10240 * 4
    assert sc(tile) == tile
    assert 3 * sc(tile) <= 1200 << 20
    assert sc(257) == 512
    assert sc(256) == 256
    assert sc(1) == 256
    assert sc(0) == 256


def test_grid_for_and_shape_checks():
    g, b = px.grid_for(px.SAXPY_FP32, [1 << 24])
    assert b == (256, 1, 1) and g == ((1 << 24) // 4096, 1, 1)
    g, b = px.grid_for(px.GEMM_FP16TC_FP32ACC, [4096, 4096, 4096])
    assert g == (256, 1, 1) and b == (256, 1, 1)
    g, b = px.grid_for(px.GEMM_FP32, [4096, 4096, 4096])
    assert g == (256, 1, 1)
    g, b = px.grid_for(px.GEMM_FP32, [384, 640, 32])  # the 64 x 64 tiling at this size
    assert g == (6 * 10, 1, 1)
    g, b = px.grid_for(px.GEMM_FP16, [384, 640, 32])  # 256-wide tiles, the last ones partial
    assert g == (6, 1, 1)
    g, b = px.grid_for(px.FLASH_FP16_BH, [64, 4096, 4096, 64])
    assert g == (16, 64, 1) and b == (512, 1, 1)  # f16: 8 waves x 32 queries
    g, b = px.grid_for(px.FLASH_FP32_BH, [64, 4096, 4096, 64])
    assert g == (32, 64, 1) and b == (256, 1, 1)
    g, b = px.grid_for(px.FLASH_FP16, [384, 1024, 64])  # 256-row workgroups, last one half full
    assert g == (2, 1, 1)
    g, b = px.grid_for(px.MATMUL, [4096, 8192, 4096])
    assert g == (16 * 32, 1, 1)
    assert px.check_shape(px.GEMM_FP16, [4096, 4096, 4096]) == 0
    assert px.check_shape(px.GEMM_FP16, [4096, 100, 4096]) == px.PHX_E_INVALID
    assert px.check_shape(px.FLASH_FP32, [4096, 4096, 128]) == px.PHX_E_INVALID
    assert px.check_shape(px.GEMM_FP32, [1 << 16, 1 << 16, 128]) == px.PHX_E_INVALID  # i32 idx
    assert px.check_shape(px.SAXPY_FP32, [1 << 31]) == px.PHX_E_INVALID


def test_ragged_shape_rules():
    # The reference's autotuner accepts M, N multiples of its smallest tile
    # (32) and K of its K tile (16 for f16, 4 for f32); these kernels accept
    # every such shape and more: M any, N and K whole 16-byte chunks (K % 8
    # for gemm_fp16tc), flash any Nq and Nk.
    ok = px.check_shape
    for M, N, K in [(96, 100, 64), (1, 4, 4), (257, 516, 1000), (32, 32, 16)]:
        assert ok(px.GEMM_FP32, [M, N, K]) == 0, (M, N, K)
        assert ok(px.MATMUL, [M, N, K]) == 0
    assert ok(px.GEMM_FP16TC_FP32ACC, [96, 100, 64]) == 0
    assert ok(px.GEMM_FP16TC_FP32ACC, [96, 100, 60]) == px.PHX_E_INVALID  # K % 8
    assert ok(px.GEMM_FP16, [96, 104, 64]) == 0
    assert ok(px.GEMM_FP16, [96, 100, 64]) == px.PHX_E_INVALID             # N % 8
    assert ok(px.GEMM_FP32, [96, 102, 64]) == px.PHX_E_INVALID             # N % 4
    assert "N%4==0" in px.lib().phx_last_error().decode()
    assert ok(px.GEMM_FP32, [0, 4, 4]) == px.PHX_E_INVALID
    g, _ = px.grid_for(px.GEMM_FP16, [300, 264, 40])    # 2 x 2 tiles of 256
    assert g == (4, 1, 1)
    g, _ = px.grid_for(px.GEMM_FP16TC_FP32ACC, [1, 4, 8])
    assert g == (1, 1, 1)
    for k in (px.FLASH_FP32, px.FLASH_FP16):
        for Nq, Nk in [(1, 1), (100, 37), (300, 200)]:
            assert ok(k, [Nq, Nk, 64]) == 0, (k, Nq, Nk)
        assert ok(k, [0, 64, 64]) == px.PHX_E_INVALID
        assert ok(k, [64, 0, 64]) == px.PHX_E_INVALID
    assert px.grid_for(px.FLASH_FP32, [300, 37, 64])[0] == (3, 1, 1)   # 128-row workgroups
    assert px.grid_for(px.FLASH_FP16_BH, [5, 300, 37, 64])[0] == (2, 5, 1)


def test_kernel_by_reference_names():
    # (.ph file stem, entry) -> kernel id; three files export "gemm"
    want = {("saxpy_fp32", "saxpy"): px.SAXPY_FP32, ("gemm_fp32", "gemm"): px.GEMM_FP32,
            ("gemm_fp16tc_fp32acc", "gemm"): px.GEMM_FP16TC_FP32ACC,
            ("gemm_fp16", "gemm"): px.GEMM_FP16,
            ("flash_attention_fp32", "flash_attention"): px.FLASH_FP32,
            ("flash_attention_fp16", "flash_attention"): px.FLASH_FP16,
            ("flash_attention_fp32", "flash_attention_bh"): px.FLASH_FP32_BH,
            ("flash_attention_fp16", "flash_attention_bh"): px.FLASH_FP16_BH,
            ("matmul_cluster_fp32", "matmul"): px.MATMUL,
            ("matmul_cluster_fp32", "matmul_init"): px.MATMUL_INIT}
    for (f, e), k in want.items():
        assert px.kernel_by_name(f, e) == k, (f, e)
    for f, e in [("gemm", "gemm"), ("gemm_fp16tc", "gemm"), ("saxpy_fp32", "gemm")]:
        with pytest.raises(px.PhxError):
            px.kernel_by_name(f, e)


def test_kernel_abi_index_widths():
    # requires_wide_index: @tensorcore kernels use i64 descriptors (lib.rs:47-49)
    assert px.kernel_abi(px.SAXPY_FP32)[0] == 32
    assert px.kernel_abi(px.GEMM_FP32)[0] == 32
    assert px.kernel_abi(px.GEMM_FP16TC_FP32ACC)[0] == 64
    assert px.kernel_abi(px.GEMM_FP16)[0] == 64
    assert px.kernel_abi(px.FLASH_FP32)[0] == 64
    assert px.kernel_abi(px.FLASH_FP16)[0] == 64
    assert px.kernel_abi(px.MATMUL)[0] == 32          # pod leaves: default Context
    assert px.kernel_abi(px.MATMUL_INIT)[0] == 32


def test_calls_before_init_fail_loudly():
    f = ctypes.c_void_p()
    if px._INIT:
        pytest.skip("already initialised in this process")
    rc = px.lib().phx_builtin_function(ctypes.byref(f), px.GEMM_FP16)
    assert rc == px.PHX_E_NOT_INIT


def test_rust_ffi_stub_matches_header():
    # The integration notes' phobos-hip-sys block (the binding the reference's
    # Rust side would add) declares every function of include/phobos_hip.h
    # with the same number of parameters.
    import re
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    h = re.sub(r"/\*.*?\*/", "", open(os.path.join(root, "include", "phobos_hip.h")).read(), flags=re.S)
    decls = {n: 0 if p.strip() in ("", "void") else p.count(",") + 1
             for n, p in re.findall(r"^(?:int|const char \*|size_t|void)\s*(phx_\w+)\s*\(([^;]*?)\)\s*;",
                                    h, flags=re.M)}
    md = open(os.path.join(root, "INTEGRATION.md")).read()
    block = md[md.index('#[link(name = "phobos_hip")]'):]
    block = block[:block.index("}\n```")]
    rs = {n: 0 if not p.strip() else p.count(",") + 1
          for n, p in re.findall(r"pub fn (phx_\w+)\(([^)]*)\)", block)}
    assert len(decls) >= 60
    assert rs == decls


def test_stream_workspace_binding_is_host_logic():
    # phx_stream_set_workspace / _get_workspace keep a per-stream table and
    # touch no device: bind, rebind, unbind, per-stream isolation and the
    # alignment check, with stream handles that are only keys here
    s1, s2 = 0x1000, 0x2000
    px.set_workspace(s1, 1 << 20, 4096)
    px.set_workspace(s2, 2 << 20, 8192)
    assert px.get_workspace(s1) == (1 << 20, 4096)
    assert px.get_workspace(s2) == (2 << 20, 8192)
    px.set_workspace(s1, 3 << 20, 256)
    assert px.get_workspace(s1) == (3 << 20, 256)
    px.set_workspace(s1, 0, 0)
    assert px.get_workspace(s1) == (0, 0) and px.get_workspace(s2) == (2 << 20, 8192)
    px.set_workspace(s2, 2 << 20, 0)  # zero bytes unbinds too
    assert px.get_workspace(s2) == (0, 0)
    with pytest.raises(px.PhxError, match="256-byte aligned"):
        px.set_workspace(s1, (1 << 20) + 128, 4096)
    assert px.get_workspace(s1) == (0, 0)
