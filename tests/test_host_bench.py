"""The native phobos-bench host (phobos-lang_amd/host/phobos_bench.cpp): a C++
program over the C ABI alone, the counterpart of phobos-bench/src/main.rs.
Its command-line checks run on the CPU (they come before any device call, as
Options::parse comes before cust::quick_init in main.rs:164-168); the runs
are GPU tests, each passing the reference's own result checks (sampled f64
GEMM and flash replays, saxpy bit-exact) inside the program."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "phobos-lang_amd", "lib", "phobos-bench")


def _run(*args, timeout=300):
    assert os.path.exists(EXE), "phobos-bench is not built (make -C phobos-lang_amd)"
    return subprocess.run([EXE, *args], capture_output=True, text=True, timeout=timeout)


@pytest.mark.parametrize("args,msg", [
    (["--bench", "gemm_fp8"], "unknown --bench 'gemm_fp8'; available: saxpy_fp32, gemm_fp32"),
    (["--autotune", "splits=2"], "--autotune pins are kernel-specific; pass --bench to pick one"),
    (["--bench", "gemm_fp32", "--autotune", "splits"], "bad autotune pin 'splits', expected NAME=VALUE"),
    (["--bench", "gemm_fp32", "--autotune", "splits=two"], "autotune pin 'splits' has a non-integer value 'two'"),
    (["--peak-fp32", "-3"], "--peak-fp32 value must be positive"),
    (["--peak-fp16tc", "abc"], "--peak-fp16tc value 'abc' is not a number"),
    (["--bench"], "--bench needs a benchmark name"),
    (["--frobnicate"], "unknown argument '--frobnicate' (try --help)"),
])
def test_command_line_errors(args, msg):
    r = _run(*args, timeout=30)
    assert r.returncode == 2 and msg in r.stderr, (r.returncode, r.stderr)


def test_help():
    r = _run("--help", timeout=30)
    assert r.returncode == 0 and "usage: phobos-bench" in r.stdout and "--csv [PATH]" in r.stdout


@pytest.mark.gpu
def test_pinned_gemm_run_passes_its_checks(tmp_path):
    csv = tmp_path / "r.csv"
    r = _run("--bench", "gemm_fp32", "--autotune", "splits=1 variant=0", "--csv", str(csv))
    assert r.returncode == 0, r.stderr
    assert "autotune: 1 configs" in r.stdout and "check: 16777216 elements sampled at 64 points, correct" in r.stdout
    rows = csv.read_text().splitlines()
    assert rows[0] == "benchmark,impl,precision,gflops,peak_gflops,pct_of_peak"
    name, impl, prec, gflops, peak, pct = rows[1].split(",")
    assert (name, impl, prec) == ("gemm_fp32", "phobos", "f32") and float(gflops) > 1e4


@pytest.mark.gpu
@pytest.mark.parametrize("bench", ["saxpy_fp32", "gemm_fp16", "flash_fp16", "flash_fp32"])
def test_searched_runs_pass_their_checks(bench):
    r = _run("--bench", bench)
    assert r.returncode == 0, r.stderr
    assert "correct" in r.stdout
    if bench != "saxpy_fp32":
        assert "autotune winner: splits=" in r.stdout


@pytest.mark.gpu
def test_unknown_pin_dim_is_refused():
    r = _run("--bench", "gemm_fp16", "--autotune", "TILE_M=256")
    assert r.returncode == 1
    assert "autotune pin 'TILE_M' is not a search dim of this kernel (dims: splits, variant)" in r.stderr


@pytest.mark.gpu
def test_gemm_fp32_tile_pin_by_reference_dim_names():
    # gemm_fp32.ph's @autotune dims (examples/gemm_fp32.ph:1) as pins: the
    # 128 x 128 x 32 tiling runs and passes the reference's 64-point check
    r = _run("--bench", "gemm_fp32", "--autotune", "TILE_M=128 TILE_N=128 TILE_K=32")
    assert r.returncode == 0, r.stderr
    assert "TILE_M=128 TILE_N=128 TILE_K=32" in r.stdout and "correct" in r.stdout
    r = _run("--bench", "gemm_fp32", "--autotune", "TILE_M=96")
    assert r.returncode == 1 and "no gemm_fp32 tiling TILE_M=96" in r.stderr
