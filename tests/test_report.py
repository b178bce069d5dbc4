"""Results CSV and peaks (phobos-bench/src/report.rs) and the plot script."""
import os
import subprocess
import sys

import pytest

from phobos_amd import report

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_csv_rows_match_the_reference_format():
    # the reference's own results.csv rows (results/results.csv:2,7) rebuilt
    # from their gflops and peak: one decimal, pct = 100 * gflops / peak
    res = report.Results()
    res.push("saxpy_fp32", "phobos", "f32", 72.0)
    res.push("gemm_fp16", "phobos", "f16-tc", 49691.2)
    peaks = report.Peaks(fp32_tflops=11.2, fp16tc_tflops=89.2)
    lines = res.to_csv(peaks).splitlines()
    assert lines[0] == "benchmark,impl,precision,gflops,peak_gflops,pct_of_peak"
    assert lines[1] == "saxpy_fp32,phobos,f32,72.0,11200.0,0.6"
    assert lines[2] == "gemm_fp16,phobos,f16-tc,49691.2,89200.0,55.7"


def test_mi355x_peaks_and_overrides():
    p = report.Peaks()
    assert p.peak("f32") == 157300.0
    assert p.peak("f16-tc") == p.peak("f16-tc-f32-acc") == 2516600.0
    q = report.Peaks(fp16tcf32acc_tflops=1000.0)
    assert q.peak("f16-tc-f32-acc") == 1e6 and q.peak("f16-tc") == 2516600.0
    assert "(override)" in q.describe()
    with pytest.raises(ValueError):
        report.Results().push("x", "phobos", "bf16", 1.0)


def test_write_read_and_plot(tmp_path):
    res = report.Results()
    res.push("gemm_fp32", "phobos", "f32", 144200.0)
    res.push("gemm_fp32", "rocBLAS", "f32", 148000.0)
    res.push("flash_fp16tc_fp32acc", "phobos", "f16-tc-f32-acc", 954220.0)
    path = tmp_path / "r.csv"
    assert res.write_csv(path, report.Peaks()) == 3
    rows = report.read_csv(path)
    assert [r["impl"] for r in rows] == ["phobos", "rocBLAS", "phobos"]
    assert rows[2]["pct"] == pytest.approx(37.9)
    pytest.importorskip("matplotlib")
    png = tmp_path / "r.png"
    subprocess.run([sys.executable, os.path.join(ROOT, "phobos-lang_amd", "plot.py"), str(path),
                    "-o", str(png)], check=True, capture_output=True, timeout=120)
    assert png.stat().st_size > 1000


def test_bench_cli_mirrors_phobos_bench_flags():
    # --bench NAME takes phobos-bench's names (main.rs:26-33, 62-67) and
    # rejects others; --autotune pins have no search to pin here.
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    run = lambda *a: subprocess.run([sys.executable, os.path.join(root, "bench.py"), *a],
                                    capture_output=True, text=True, timeout=120)
    r = run("--bench", "gemm_fp8")
    assert r.returncode == 2 and "available: saxpy_fp32, gemm_fp32" in r.stderr
    r = run("--bench", "gemm_fp16", "--autotune", "TILE_M=256")
    assert r.returncode == 2 and "'TILE_M' is not a search dim" in r.stderr
    r = run("--autotune", "splits=2")
    assert r.returncode == 2 and "pass --bench to pick one" in r.stderr
    r = run("--bench", "gemm_fp16", "--autotune", "splits=two")
    assert r.returncode == 2 and "non-integer value 'two'" in r.stderr
    for bad in ("gemm_fp32=1", "saxpy_fp32=1,0", "gemm_fp8=1,0", "flash_fp16=a,0"):
        r = run("--pin", bad)  # --pin NAME=SPLITS,VARIANT, kernels with plans only
        assert r.returncode == 2 and f"bad --pin '{bad}'" in r.stderr
    r = run("--help")
    assert r.returncode == 0 and "--bench NAME" in r.stdout and "--csv" in r.stdout
    assert "--pin NAME=SPLITS,VARIANT" in r.stdout
