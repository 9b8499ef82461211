"""
Figures of the N_input sweep (bench_perceiver_ni.py rows, experiment
"perceiver_ni"), the set of experiments/plot_perceiver.py in the reference:

  perceiver_latency_vs_ni.png    latency vs N_input, log-log, with the N_input
                                 where a batch element's K/V outgrow the
                                 XCD's L2 and the Infinity Cache;
  perceiver_speedup_vs_warp.png  speedup of every implementation over the
                                 baseline one (warp by default) where both ran;
  perceiver_gflops_vs_ni.png     achieved GFLOP/s vs N_input (linear y);
  perceiver_pct_peak_vs_ni.png   % of the peak each row is measured against
                                 (fp32 MFMA for fp32 rows, the 16-bit MFMA
                                 peak for fp16/bf16 rows);
  perceiver_roofline.png         achieved GFLOP/s vs arithmetic intensity under
                                 the device's fp32 and bf16 MFMA ceilings and
                                 its HBM slope.

    python experiments/plot_perceiver.py [--csv results/perceiver_ni.csv] [--outdir results]
"""

import argparse
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import plotting as pl  # noqa: E402


def subtitle(meta, baseline=None):
    s = f"{meta.get('gpu', '?')}  ·  B={meta.get('B', '?')}  ·  N_latent={meta.get('N_latent', '?')}"
    return s + (f"  ·  baseline = {baseline}" if baseline else "")


def plot_latency(by_impl, nis, meta, outdir):
    fig, ax = pl.axes("Cross-attention latency vs input length", subtitle(meta))
    for impl, rows in by_impl.items():
        xs, ys = pl.series(rows, nis, "latency_ms_mean")
        if xs:
            pl.draw(ax, impl, xs, ys)
        limited = [n for n in nis if rows.get(n, {}).get("status") == "design-limited"]
        if limited and xs:
            ax.annotate(f"{impl}: design-limited\nfrom N_input={limited[0]}",
                        xy=(xs[-1], ys[-1]), xytext=(12, -28), textcoords="offset points",
                        fontsize=8.5, color=pl.style(impl)[0],
                        arrowprops=dict(arrowstyle="->", color=pl.style(impl)[0]))
    ax.set_yscale("log")
    pl.log_x(ax, nis, [pl.square_label(n) for n in nis])
    pl.cache_markers(ax, meta.get("gpu"), 2 * 768 * 4)
    ax.set_xlabel("N_input (image side²)")
    ax.set_ylabel("latency per call (ms, log)")
    ax.legend(frameon=True)
    return pl.save(fig, outdir, "perceiver_latency_vs_ni.png")


def plot_speedup(by_impl, nis, meta, outdir, baseline):
    base = by_impl.get(baseline, {})
    fig, ax = pl.axes(f"Speedup over {baseline}", subtitle(meta, baseline))
    drew = False
    for impl, rows in by_impl.items():
        if impl == baseline:
            continue
        pts = [(n, pl.value(base.get(n), "latency_ms_mean"), pl.value(rows.get(n),
                                                                      "latency_ms_mean"))
               for n in nis]
        pts = [(n, b / t) for n, b, t in pts if b and t]
        if not pts:
            continue
        xs, ys = zip(*pts)
        pl.draw(ax, impl, xs, ys)
        for x, y in pts:
            ax.annotate(f"{y:.1f}×", (x, y), textcoords="offset points", xytext=(0, 7),
                        ha="center", fontsize=8, color=pl.style(impl)[0])
        drew = True
    if not drew:
        pl.plt.close(fig)
        return None
    ax.axhline(1.0, color="gray", ls=":")
    ax.set_yscale("log")
    pl.log_x(ax, nis, [pl.square_label(n) for n in nis])
    ax.set_xlabel("N_input (where the baseline ran)")
    ax.set_ylabel(f"speedup vs {baseline} (×, log)")
    ax.legend(frameon=True)
    return pl.save(fig, outdir, "perceiver_speedup_vs_warp.png")


def plot_gflops(by_impl, nis, meta, outdir):
    fig, ax = pl.axes("Throughput vs input length", subtitle(meta))
    for impl, rows in by_impl.items():
        xs, ys = pl.series(rows, nis, "achieved_gflops")
        if xs:
            pl.draw(ax, impl, xs, ys)
    pl.log_x(ax, nis, [pl.square_label(n) for n in nis])
    ax.set_ylim(bottom=0)
    pl.cache_markers(ax, meta.get("gpu"), 2 * 768 * 4)
    ax.set_xlabel("N_input (image side²)")
    ax.set_ylabel("achieved GFLOP/s")
    ax.legend(frameon=True)
    return pl.save(fig, outdir, "perceiver_gflops_vs_ni.png")


def plot_pct_peak(by_impl, nis, meta, outdir):
    fig, ax = pl.axes("Fraction of the MFMA peak", subtitle(meta))
    drew = False
    for impl, rows in by_impl.items():
        xs, ys = pl.series(rows, nis, "pct_peak_compute")
        if xs and any(ys):
            pl.draw(ax, impl, xs, ys)
            drew = True
    if not drew:
        pl.plt.close(fig)
        return None
    pl.log_x(ax, nis, [pl.square_label(n) for n in nis])
    ax.set_ylim(0, 100)
    ax.set_xlabel("N_input (image side²)")
    ax.set_ylabel("% of the row's precision peak")
    ax.legend(frameon=True)
    return pl.save(fig, outdir, "perceiver_pct_peak_vs_ni.png")


def plot_roofline(by_impl, nis, meta, outdir):
    from gpu_specs import GPU_SPECS
    spec = GPU_SPECS.get(meta.get("gpu"))
    fig, ax = pl.axes("Roofline", subtitle(meta))
    pts_all = []
    for impl, rows in by_impl.items():
        pts = [(pl.value(rows.get(n), "arithmetic_intensity"),
                pl.value(rows.get(n), "achieved_gflops")) for n in nis]
        pts = sorted((a, g) for a, g in pts if a and g)
        if pts:
            xs, ys = zip(*pts)
            pl.draw(ax, impl, xs, ys)
            pts_all += pts
    if spec:
        bw = spec["peak_bw_bytes"]
        lo = min([a for a, _ in pts_all] + [1.0]) / 2
        hi = max([a for a, _ in pts_all] + [2048.0]) * 2
        for key, colour, name in (("peak_fp32_flops", "0.25", "fp32 MFMA"),
                                  ("peak_bf16_tc_flops", "#bcbd22", "bf16/fp16 MFMA")):
            peak = spec[key]
            ridge = peak / bw
            ax.plot([lo, ridge, hi], [bw * lo / 1e9, peak / 1e9, peak / 1e9], color=colour,
                    lw=1.6, ls="--", label=f"{name} {peak / 1e12:.0f} TFLOP/s, ridge {ridge:.0f}")
    ax.set_xscale("log")
    ax.set_yscale("log")
    ax.set_xlabel("arithmetic intensity (FLOP / HBM byte)")
    ax.set_ylabel("achieved GFLOP/s (log)")
    ax.legend(frameon=True, fontsize=8, loc="lower right")
    return pl.save(fig, outdir, "perceiver_roofline.png")


def main(argv=None):
    ap = argparse.ArgumentParser(description="Plot the Perceiver N_input sweep")
    ap.add_argument("--csv", default="results/perceiver_ni.csv")
    ap.add_argument("--outdir", default="results")
    ap.add_argument("--impls", nargs="+", default=None, help="plot only these implementations")
    ap.add_argument("--baseline", default="warp", help="implementation speedups are relative to")
    args = ap.parse_args(argv)
    if not os.path.exists(args.csv):
        print(f"No log at {args.csv}; run bench_perceiver_ni.py first.")
        return 1
    by_impl, meta = pl.load(args.csv, "perceiver_ni", "N_input")
    if args.impls:
        by_impl = {k: v for k, v in by_impl.items() if k in args.impls}
    if not by_impl:
        print("No perceiver_ni rows in the log.")
        return 1
    nis = sorted({n for rows in by_impl.values() for n in rows})
    made = [plot_latency(by_impl, nis, meta, args.outdir),
            plot_speedup(by_impl, nis, meta, args.outdir, args.baseline),
            plot_gflops(by_impl, nis, meta, args.outdir),
            plot_pct_peak(by_impl, nis, meta, args.outdir),
            plot_roofline(by_impl, nis, meta, args.outdir)]
    for p in made:
        if p:
            print(p)
    return 0


if __name__ == "__main__":
    sys.exit(main())
