#!/usr/bin/env python3
"""Bar chart of a results CSV written by `python bench.py --csv`.

Counterpart of the reference's phobos-bench/plot.py: for each benchmark (in
CSV order) one bar per implementation with its achieved GFLOP/s, drawn over a
grey bar at the theoretical peak of the benchmark's precision, each labelled
with its percent of peak.  Rows without a peak are skipped.

    python3 phobos-lang_amd/plot.py phobos-bench.csv -o bench.png --title "MI355X"
"""
import argparse
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from phobos_amd.report import read_csv  # noqa: E402


def draw(rows, out, title):
    import matplotlib
    if out:
        matplotlib.use("Agg")
    import matplotlib.pyplot as plt

    benches, impls = [], []
    for r in rows:
        if r["benchmark"] not in benches:
            benches.append(r["benchmark"])
        if r["impl"] not in impls:
            impls.append(r["impl"])
    cell = {(r["benchmark"], r["impl"]): r for r in rows}
    colors = plt.rcParams["axes.prop_cycle"].by_key()["color"]
    width = 0.8
    bar = width / len(impls)
    fig, ax = plt.subplots(figsize=(max(7.0, 1.6 * len(benches)), 5.0))
    for x, bench in enumerate(benches):
        peak = max(r["peak"] for r in rows if r["benchmark"] == bench)
        ax.bar(x, peak, width=width, color="0.85", zorder=0,
               label="theoretical peak" if x == 0 else None)
        for j, impl in enumerate(impls):
            r = cell.get((bench, impl))
            if r is None:
                continue
            xi = x - width / 2 + bar * (j + 0.5)
            ax.bar(xi, r["gflops"], width=0.92 * bar, color=colors[j % len(colors)], zorder=2,
                   label=impl if (bench, impl) == next((b, impl) for b in benches
                                                       if (b, impl) in cell) else None)
            ax.text(xi, r["gflops"], f"{r['pct']:.0f}%", ha="center", va="bottom", fontsize=8,
                    zorder=3)
    ax.set_xticks(range(len(benches)))
    ax.set_xticklabels(benches, rotation=15)
    ax.set_ylabel("GFLOP/s")
    ax.set_title(title)
    ax.legend(loc="upper right", framealpha=0.9)
    ax.margins(y=0.12)
    fig.tight_layout()
    if out:
        fig.savefig(out, dpi=150)
        print(f"wrote {out}")
    else:
        plt.show()


def main():
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("csv", help="results CSV from `python bench.py --csv`")
    ap.add_argument("-o", "--out", help="output image (default: show interactively)")
    ap.add_argument("--title", default="phobos leaf kernels on MI355X: achieved vs peak")
    args = ap.parse_args()
    rows = read_csv(args.csv)
    if not rows:
        sys.exit(f"no rows with a peak in {args.csv}")
    draw(rows, args.out, args.title)


if __name__ == "__main__":
    main()
