"""The launch-plan rules and pins of the C ABI (phx_split_plan, phx_plan_get,
phx_plan_pin) on the CPU: they are host logic, so no device is needed.  The
split rule is restated here independently (phx_geometry.h's constants:
256 x 256 output tiles, 32-deep K steps, at least 128 tiles or 256 of 512
flash slots before anything splits, at most 16 chunks, aiming at 256
workgroups with at least 1 K step per chunk for gemm_fp32 and at 128 with at
least 8 (32 from 64 tiles up) for the f16 GEMMs; flash aiming at 256
workgroups with at least 5 (f16) or 2 (f32) key blocks per chunk; no empty
chunk; gemm_fp32 takes its 64 x 64 x 16 tiling instead of a
split below 256 tiles of 256 x 256 when that gives at least 128 tiles, or 16
with K <= 4096) and compared over a grid of shapes."""
import itertools

import pytest

import phobos_amd as px


@pytest.fixture(autouse=True)
def _unpin():
    px.plan_unpin_all()
    yield
    px.plan_unpin_all()


def _rounded(units, sp):
    sp = min(sp, units)
    if sp < 2:
        return 1
    per = -(-units // sp)
    return -(-units // per)


def _s32_tiling(M, N, K):
    """gemm_fp32's built-in tiling variant: 0 (256 x 256 x 16) or 7 (64 x 64 x 16)."""
    if -(-M // 256) * -(-N // 256) >= 256:
        return 0
    small = -(-M // 64) * -(-N // 64)
    return 7 if small >= 128 or (small >= 16 and K <= 4096) else 0


def _gemm_rule(kern, M, N, K):
    tiles = -(-M // 256) * -(-N // 256)
    steps = -(-K // 32)
    if kern == px.GEMM_FP32 and _s32_tiling(M, N, K):
        return 1
    if tiles >= 128:
        return 1
    if kern == px.GEMM_FP32:
        target, min_steps = 256, 1
    else:
        target, min_steps = 128, (32 if tiles >= 64 else 8)
    sp = min(target // tiles, steps // min_steps, 16)
    return _rounded(steps, sp)


def _flash_rule(f16, BH, Nq, Nk):
    items = -(-Nq // (256 if f16 else 128)) * BH
    nkb = -(-Nk // 64)
    if 2 * items >= 512:
        return 1
    return _rounded(nkb, min(256 // items, nkb // (5 if f16 else 2), 16))


GEMMS = ["GEMM_FP32", "GEMM_FP16TC_FP32ACC", "GEMM_FP16"]


@pytest.mark.parametrize("name", GEMMS)
def test_gemm_split_rule(name):
    kern = getattr(px, name)
    for M, N, K in itertools.product((64, 256, 300, 1024, 2048, 4096), (256, 512, 4096),
                                     (64, 512, 1000, 4096, 16384)):
        if kern != px.GEMM_FP32 and K % 8:
            continue
        want = _gemm_rule(kern, M, N, K)
        sp, ws = px.split_plan(kern, [M, N, K])
        assert sp == want, (M, N, K, sp, want)
        assert ws == (sp * M * N * 4 if sp > 1 else 0)
        assert px.plan_get(kern, [M, N, K])[0] == want
        if kern == px.GEMM_FP32:
            v = _s32_tiling(M, N, K)
            assert px.plan_get(kern, [M, N, K]) == (want, v)
            tm, tn, _ = px.GEMM_FP32_TILINGS[v]
            assert px.grid_for(kern, [M, N, K])[0] == (-(-M // tm) * -(-N // tn), 1, 1)


def test_gemm_fp32_small_tiling_is_64x64():
    assert px.GEMM_FP32_TILINGS[7] == (64, 64, 16)
    assert px.plan_get(px.GEMM_FP32, [3072, 3072, 1024]) == (1, 7)
    assert px.plan_get(px.GEMM_FP32, [4096, 4096, 4096]) == (1, 0)
    assert px.plan_get(px.GEMM_FP32, [512, 512, 16384])[1] == 0  # long K, few tiles: split
    assert px.plan_get(px.GEMM_FP32, [512, 512, 16384])[0] > 1


@pytest.mark.parametrize("f16", [True, False])
def test_flash_split_rule(f16):
    one, bh = (px.FLASH_FP16, px.FLASH_FP16_BH) if f16 else (px.FLASH_FP32, px.FLASH_FP32_BH)
    for BH, Nq, Nk in itertools.product((1, 2, 16, 64), (64, 300, 4096), (64, 700, 4096, 16384)):
        want = _flash_rule(f16, BH, Nq, Nk)
        sp, ws = px.split_plan(bh, [BH, Nq, Nk, 64])
        assert sp == want, (BH, Nq, Nk, sp, want)
        assert ws == (sp * BH * Nq * 66 * 4 if sp > 1 else 0)
        if BH == 1:
            assert px.split_plan(one, [Nq, Nk, 64])[0] == want


def test_pins_override_the_rule_and_come_off():
    dims = [512, 512, 8192]
    rule = px.plan_get(px.GEMM_FP32, dims)
    px.plan_pin(px.GEMM_FP32, dims, 3)
    assert px.plan_get(px.GEMM_FP32, dims) == (3, 0)
    assert px.split_plan(px.GEMM_FP32, dims) == (3, 3 * 512 * 512 * 4)
    assert px.plan_get(px.GEMM_FP32, [512, 512, 4096]) == (1, 7)  # pins are per shape
    with pytest.raises(px.PhxError, match="outside 1..16"):
        px.plan_pin(px.GEMM_FP32, dims, 500)
    assert px.plan_get(px.GEMM_FP32, dims) == (3, 0)  # a refused pin leaves the old one
    px.plan_pin(px.GEMM_FP32, dims, None)
    assert px.plan_get(px.GEMM_FP32, dims) == rule


def test_pin_validation():
    dims = [512, 512, 4096]
    for sp, var in ((0, 0), (17, 0), (1, 8), (1, -1), (2, 1)):
        with pytest.raises(px.PhxError):
            px.plan_pin(px.GEMM_FP32, dims, sp, var)
    for sp, var in ((1, 1), (1, 7)):  # gemm_fp16 has no tilings to choose from
        with pytest.raises(px.PhxError):
            px.plan_pin(px.GEMM_FP16, dims, sp, var)
    # gemm_fp32's tilings: pinned unsplit, and the grid follows the tile
    px.plan_pin(px.GEMM_FP32, dims, 1, 3)  # 128 x 128 x 16
    assert px.plan_get(px.GEMM_FP32, dims) == (1, 3)
    assert px.split_plan(px.GEMM_FP32, dims) == (1, 0)
    assert px.grid_for(px.GEMM_FP32, dims)[0] == (16, 1, 1)
    px.plan_pin(px.GEMM_FP32, dims, 1, 7)  # 64 x 64 x 16
    assert px.grid_for(px.GEMM_FP32, dims)[0] == (64, 1, 1)
    px.plan_pin(px.GEMM_FP32, dims, 1, 0)  # 256 x 256 x 16
    assert px.grid_for(px.GEMM_FP32, dims)[0] == (4, 1, 1)
    px.plan_pin(px.GEMM_FP32, dims, None)  # the built-in plan here: 64 x 64 x 16
    assert px.plan_get(px.GEMM_FP32, dims) == (1, 7)
    px.plan_pin(px.GEMM_FP16TC_FP32ACC, dims, 1, 1)
    assert px.plan_get(px.GEMM_FP16TC_FP32ACC, dims) == (1, 1)
    # a pinned count is rounded like a requested one (whole steps, no empty chunk)
    px.plan_pin(px.GEMM_FP32, [512, 512, 96], 16)
    assert px.plan_get(px.GEMM_FP32, [512, 512, 96])[0] == 3
    # one-head and batched flash share a pin; other heads counts do not
    px.plan_pin(px.FLASH_FP16, [4096, 4096, 64], 4)
    assert px.plan_get(px.FLASH_FP16_BH, [1, 4096, 4096, 64]) == (4, 0)
    assert px.plan_get(px.FLASH_FP16_BH, [2, 4096, 4096, 64])[0] == _flash_rule(True, 2, 4096, 4096)
    assert px.plan_get(px.FLASH_FP32, [4096, 4096, 64])[0] == _flash_rule(False, 1, 4096, 4096)
    px.plan_pin(px.FLASH_FP16, [4096, 4096, 64], None)
    assert px.plan_get(px.FLASH_FP16, [4096, 4096, 64])[0] == _flash_rule(True, 1, 4096, 4096)
