"""
This library's kernels against PyTorch-ROCm's SDPA backends, the figures of
experiments/plot_pytorch_compare.py in the reference, from N_input-sweep rows
that include sdpa_* implementations (bench_perceiver_ni.py --impls splitk
vectorized sdpa_math sdpa_efficient ...):

  pytorch_latency_vs_ni.png     latency vs N_input, log-log, head to head;
  pytorch_bar_anchor.png        latencies at one N_input (--anchor, default
                                4096), fastest first, with this library's
                                best row set against SDPA-math and the
                                fastest fused SDPA backend;
  pytorch_slowdown_vs_math.png  each implementation's latency over fp32
                                SDPA-math's at the same N_input.

    python experiments/plot_pytorch_compare.py --csv results/perceiver_ni.csv --anchor 4096
"""

import argparse
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import plotting as pl  # noqa: E402

MATH = "sdpa_math"


def subtitle(meta):
    return (f"{meta.get('gpu', '?')}  ·  B={meta.get('B', '?')}  ·  "
            f"N_latent={meta.get('N_latent', '?')}  ·  single head, head_dim 768")


def lat(rows, n):
    return pl.value(rows.get(n), "latency_ms_mean")


def plot_latency(by_impl, nis, meta, outdir):
    fig, ax = pl.axes("Fused MFMA kernels vs PyTorch SDPA", subtitle(meta))
    for impl, rows in by_impl.items():
        xs, ys = pl.series(rows, nis, "latency_ms_mean")
        if xs:
            pl.draw(ax, impl, xs, ys)
    ax.set_yscale("log")
    pl.log_x(ax, nis, [pl.square_label(n) for n in nis])
    ax.set_xlabel("N_input (image side²)")
    ax.set_ylabel("latency per call (ms, log)")
    ax.legend(frameon=True, fontsize=8.5)
    return pl.save(fig, outdir, "pytorch_latency_vs_ni.png")


def plot_bar(by_impl, anchor, meta, outdir):
    items = sorted(((impl, lat(rows, anchor)) for impl, rows in by_impl.items()),
                   key=lambda t: (t[1] is None, t[1] or 0.0))
    items = [(i, v) for i, v in items if v is not None]
    if not items:
        return None
    fig, ax = pl.axes(f"Latency at N_input = {anchor}", subtitle(meta))
    fig.set_size_inches(max(8.0, 1.05 * len(items)), 5.2)
    bars = ax.bar(range(len(items)), [v for _, v in items],
                  color=[pl.style(i)[0] for i, _ in items], edgecolor="black", linewidth=0.5)
    for b, (_, v) in zip(bars, items):
        ax.text(b.get_x() + b.get_width() / 2, v, f"{v:.3f}", ha="center", va="bottom",
                fontsize=8.5)
    ax.set_xticks(range(len(items)))
    ax.set_xticklabels([i for i, _ in items], rotation=30, ha="right", fontsize=9)
    ax.set_ylabel("latency per call (ms)")
    d = dict(items)
    ours = [(v, i) for i, v in items if i in pl.OURS]
    fused = [(v, i) for i, v in items if i.startswith("sdpa_") and not i.startswith(MATH)]
    notes = []
    if ours and MATH in d:
        v, i = min(ours)
        notes.append(f"{i}: {d[MATH] / v:.1f}× SDPA-math fp32 speed")
    if ours and fused:
        v, i = min(ours)
        fv, fi = min(fused)
        notes.append(f"{i}: {fv / v:.1f}× the fastest fused SDPA ({fi})")
    if notes:
        ax.text(0.02, 0.97, "\n".join(notes), transform=ax.transAxes, va="top", fontsize=9.5,
                bbox=dict(boxstyle="round", fc="#f4f4f4", ec="0.7"))
    return pl.save(fig, outdir, "pytorch_bar_anchor.png")


def plot_slowdown(by_impl, nis, meta, outdir):
    math_rows = by_impl.get(MATH, {})
    fig, ax = pl.axes("Latency relative to fp32 SDPA-math", subtitle(meta))
    drew = False
    for impl, rows in by_impl.items():
        if impl == MATH:
            continue
        pts = [(n, lat(rows, n), lat(math_rows, n)) for n in nis]
        pts = [(n, t / m) for n, t, m in pts if t and m]
        if pts:
            xs, ys = zip(*pts)
            pl.draw(ax, impl, xs, ys)
            drew = True
    if not drew:
        pl.plt.close(fig)
        return None
    ax.axhline(1.0, color="gray", ls=":")
    ax.set_yscale("log")
    pl.log_x(ax, nis, [pl.square_label(n) for n in nis])
    ax.set_xlabel("N_input (image side²)")
    ax.set_ylabel("latency / SDPA-math latency (log; < 1 is faster)")
    ax.legend(frameon=True, fontsize=8.5)
    return pl.save(fig, outdir, "pytorch_slowdown_vs_math.png")


def main(argv=None):
    ap = argparse.ArgumentParser(description="Plot this library against PyTorch SDPA")
    ap.add_argument("--csv", default="results/perceiver_ni.csv")
    ap.add_argument("--outdir", default="results")
    ap.add_argument("--anchor", type=int, default=4096)
    ap.add_argument("--impls", nargs="+", default=None, help="plot only these implementations")
    args = ap.parse_args(argv)
    if not os.path.exists(args.csv):
        print(f"No log at {args.csv}; run bench_perceiver_ni.py with sdpa_* impls first.")
        return 1
    by_impl, meta = pl.load(args.csv, "perceiver_ni", "N_input")
    if args.impls:
        by_impl = {k: v for k, v in by_impl.items() if k in args.impls}
    if not by_impl:
        print("No perceiver_ni rows in the log.")
        return 1
    nis = sorted({n for rows in by_impl.values() for n in rows})
    for p in (plot_latency(by_impl, nis, meta, args.outdir),
              plot_bar(by_impl, args.anchor, meta, args.outdir),
              plot_slowdown(by_impl, nis, meta, args.outdir)):
        if p:
            print(p)
    return 0


if __name__ == "__main__":
    sys.exit(main())
