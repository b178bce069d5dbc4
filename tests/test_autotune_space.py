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
    s = autotune.gemm_space(GEMM_FP32, 512, 512, 4096)  # 128 steps
    assert s == [(1, 0), (2, 0), (3, 0), (4, 0), (6, 0), (8, 0), (12, 0), (16, 0)]
    s = autotune.gemm_space(GEMM_FP16, 512, 512, 96)  # 3 steps: 1, 2, 3 chunks
    assert s == [(1, 0), (2, 0), (3, 0)]
    s = autotune.gemm_space(GEMM_FP16TC_FP32ACC, 4096, 4096, 4096)
    assert (1, 1) in s and s.count((1, 1)) == 1
    assert (1, 1) not in autotune.gemm_space(GEMM_FP16TC_FP32ACC, 4000, 4096, 4096)
    # the workspace cap drops large splits of large outputs
    assert max(sp for sp, _ in autotune.gemm_space(GEMM_FP32, 16384, 16384, 4096)) == 4


def test_flash_space():
    assert autotune.flash_space(1, 4096, 4096) == [(1, 0), (2, 0), (3, 0), (4, 0), (6, 0),
                                                   (8, 0), (11, 0), (16, 0)]
    assert autotune.flash_space(1, 64, 100) == [(1, 0), (2, 0)]  # two key blocks
