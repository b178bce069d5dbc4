"""Benchmark results as the reference's CSV, against MI355X peaks.

Mirrors phobos-bench/src/report.rs: a Results list of (benchmark, impl,
precision, GFLOP/s) rows (`Results::push`, report.rs:55-68) written as the CSV
`benchmark,impl,precision,gflops,peak_gflops,pct_of_peak` with one decimal
(`to_csv`, report.rs:70-88), each row normalised by the peak of its precision
(`Precision::peak_gflops`, report.rs:27-34).  The precision labels are the
reference's (report.rs:17-24).

`Peaks` replaces report.rs:113-185, which derives NVIDIA peaks from SM
count, clock and compute capability: here the peaks are MI355X's published
dense rates (256 CUs at 2.4 GHz).  AMD matrix cores always accumulate f16
products in f32, so "f16-tc" and "f16-tc-f32-acc" share the dense f16 MFMA
rate; "f32" is the f32 rate, which the vector ALUs and the f32 matrix cores
share on MI355X.  The overrides are TFLOP/s, as the reference's
--peak-fp32 / --peak-fp16tc / --peak-fp16tcf32acc flags (main.rs:82-90).
"""
import os

PRECISIONS = ("f32", "f16-tc", "f16-tc-f32-acc")

# MI355X published dense peaks, GFLOP/s
MI355X_FP32_GFLOPS = 157_300.0
MI355X_FP16_MFMA_GFLOPS = 2_516_600.0

HEADER = "benchmark,impl,precision,gflops,peak_gflops,pct_of_peak"


class Peaks:
    """Theoretical peaks (GFLOP/s) per precision label."""

    def __init__(self, fp32_tflops=None, fp16tc_tflops=None, fp16tcf32acc_tflops=None):
        self.gflops = {
            "f32": MI355X_FP32_GFLOPS if fp32_tflops is None else fp32_tflops * 1e3,
            "f16-tc": MI355X_FP16_MFMA_GFLOPS if fp16tc_tflops is None else fp16tc_tflops * 1e3,
            "f16-tc-f32-acc": (MI355X_FP16_MFMA_GFLOPS if fp16tcf32acc_tflops is None
                               else fp16tcf32acc_tflops * 1e3),
        }
        self.overridden = {"f32": fp32_tflops is not None, "f16-tc": fp16tc_tflops is not None,
                           "f16-tc-f32-acc": fp16tcf32acc_tflops is not None}

    def peak(self, precision):
        return self.gflops[precision]

    def describe(self):
        return ", ".join(f"{p} {self.gflops[p] / 1e3:.1f} TFLOP/s"
                         + (" (override)" if self.overridden[p] else "") for p in PRECISIONS)


class Results:
    """Rows collected over a run (report.rs:45-68)."""

    def __init__(self):
        self.records = []

    def push(self, benchmark, impl, precision, gflops):
        if precision not in PRECISIONS:
            raise ValueError(f"unknown precision {precision!r}; one of {PRECISIONS}")
        self.records.append((benchmark, impl, precision, float(gflops)))

    def to_csv(self, peaks):
        lines = [HEADER]
        for bench, impl, prec, gflops in self.records:
            peak = peaks.peak(prec)
            lines.append(f"{bench},{impl},{prec},{gflops:.1f},{peak:.1f},{100.0 * gflops / peak:.1f}")
        return "\n".join(lines) + "\n"

    def write_csv(self, path, peaks):
        with open(path, "w") as f:
            f.write(self.to_csv(peaks))
        return len(self.records)


def read_csv(path):
    """Rows of a results CSV as dicts with float gflops / peak / pct."""
    import csv
    rows = []
    with open(path, newline="", encoding="utf-8-sig") as f:
        for r in csv.DictReader(f):
            if not r.get("peak_gflops"):
                continue
            rows.append({"benchmark": r["benchmark"], "impl": r["impl"],
                         "precision": r["precision"], "gflops": float(r["gflops"]),
                         "peak": float(r["peak_gflops"]), "pct": float(r["pct_of_peak"])})
    return rows


DEFAULT_CSV = "phobos-bench.csv"  # main.rs:48-49
