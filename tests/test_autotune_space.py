"""The autotuner's search space (phobos_amd.autotune), on the CPU: the split
counts it tries are exactly the distinct counts the runtime can run (whole
32-deep K steps or 64-key blocks per chunk, no empty chunk), as
phx_runtime.cpp's gemm_split / flash_split round a requested count."""
import itertools

from phobos_amd import GEMM_FP16, GEMM_FP16TC_FP32ACC, GEMM_FP32, autotune


def _runtime_round(units, sp):
    # a brute-force restatement of the rounding: the chunk count of the
    # smallest chunk length that covers units in at most sp chunks
    sp = min(sp, units)
    if sp < 2:
        return 1
    for per in itertools.count(1):
        if per * sp >= units:
            return len(range(0, units, per))


def test_effective_matches_brute_force():
    for units in range(1, 200):
        for sp in range(1, 20):
            assert autotune._effective(units, sp) == _runtime_round(units, sp), (units, sp)


def test_gemm_space():
    s = autotune.gemm_space(GEMM_FP32, 512, 512, 4096)  # 128 steps, then the other tilings
    assert s == [(1, 0), (2, 0), (3, 0), (4, 0), (6, 0), (8, 0), (12, 0), (16, 0)] + \
        [(1, v) for v in range(1, 8)]
    s = autotune.gemm_space(GEMM_FP16, 512, 512, 96)  # 3 steps: 1, 2, 3 chunks
    assert s == [(1, 0), (2, 0), (3, 0)]
    s = autotune.gemm_space(GEMM_FP16TC_FP32ACC, 4096, 4096, 4096)
    assert (1, 1) in s and s.count((1, 1)) == 1
    assert (1, 1) in autotune.gemm_space(GEMM_FP16TC_FP32ACC, 4000, 4096, 4104)
    # the workspace cap drops large splits of large outputs
    assert max(sp for sp, _ in autotune.gemm_space(GEMM_FP32, 16384, 16384, 4096)) == 4


def test_gemm_fp32_tile_space_covers_the_reference_ranges():
    # gemm_fp32.ph's @autotune: TILE_M, TILE_N in [32, 256], TILE_K in [4, 32]
    # (examples/gemm_fp32.ph:1); the built-in tiling is variant 0
    from phobos_amd import GEMM_FP32_TILINGS
    assert GEMM_FP32_TILINGS[0] == (256, 256, 16)
    assert len(set(GEMM_FP32_TILINGS)) == len(GEMM_FP32_TILINGS) == 8
    for tm, tn, tk in GEMM_FP32_TILINGS:
        assert 32 <= tm <= 256 and 32 <= tn <= 256 and 4 <= tk <= 32
    assert {t[2] for t in GEMM_FP32_TILINGS} == {8, 16, 32}
    assert {t[0] for t in GEMM_FP32_TILINGS} == {64, 128, 256}
    # the names the pins and the logs use
    assert autotune.plan_from_pins(GEMM_FP32, {"TILE_M": 128, "TILE_N": 128, "TILE_K": 32}) == (1, 4)
    assert autotune.plan_from_pins(GEMM_FP32, {"TILE_N": 128}) == (1, 1)  # 256 x 128 x 16
    assert autotune.plan_from_pins(GEMM_FP32, {"splits": 4}) == (4, 0)
    assert autotune.plan_name(GEMM_FP32, (1, 7)) == "TILE_M=64 TILE_N=64 TILE_K=16 splits=1"
    import pytest
    from phobos_amd import PhxError
    with pytest.raises(PhxError, match="no gemm_fp32 tiling"):
        autotune.plan_from_pins(GEMM_FP32, {"TILE_M": 32})
    assert "TILE_M" in autotune.search_dims(GEMM_FP32)
    assert "TILE_M" not in autotune.search_dims(GEMM_FP16)


def test_flash_space():
    assert autotune.flash_space(1, 4096, 4096) == [(1, 0), (2, 0), (3, 0), (4, 0), (6, 0),
                                                   (8, 0), (11, 0), (16, 0)]
    assert autotune.flash_space(1, 64, 100) == [(1, 0), (2, 0)]  # two key blocks
