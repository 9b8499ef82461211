"""
Figures of the N_latent (occupancy) sweep (bench_perceiver_nl.py rows,
experiment "perceiver_nl"), the set of experiments/plot_perceiver_nl.py in
the reference:

  perceiver_nl_gflops.png     achieved GFLOP/s vs N_latent;
  perceiver_nl_latency.png    latency vs N_latent, log-log;
  perceiver_nl_occupancy.png  workgroups each implementation launched
                              (the "blocks=" note of each row, which counts
                              this library's internal key splits) against the
                              device's compute units.

    python experiments/plot_perceiver_nl.py [--csv results/perceiver_nl.csv] [--outdir results]
"""

import argparse
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import plotting as pl  # noqa: E402


def subtitle(meta):
    return (f"{meta.get('gpu', '?')}  ·  B={meta.get('B', '?')}  ·  "
            f"N_input={meta.get('N_input', '?')}")


def workgroups(row):
    """Workgroups of a row from its note ('blocks=N;act_cu=M;...'), or None."""
    for part in (row or {}).get("note", "").split(";"):
        k, _, v = part.partition("=")
        if k.strip() == "blocks":
            try:
                return int(v)
            except ValueError:
                return None
    return None


def cu_count(gpu):
    from gpu_specs import GPU_SPECS
    return GPU_SPECS.get(gpu, {}).get("sm_count")


def _lines(ax, by_impl, nls, field):
    for impl, rows in by_impl.items():
        xs, ys = pl.series(rows, nls, field)
        if xs:
            pl.draw(ax, impl, xs, ys)


def plot_gflops(by_impl, nls, meta, outdir):
    fig, ax = pl.axes("Throughput vs number of latents", subtitle(meta))
    _lines(ax, by_impl, nls, "achieved_gflops")
    ax.set_xscale("log", base=2)
    ax.set_xticks(nls)
    ax.set_xticklabels([str(n) for n in nls])
    ax.minorticks_off()
    ax.set_ylim(bottom=0)
    ax.set_xlabel("N_latent")
    ax.set_ylabel("achieved GFLOP/s")
    ax.legend(frameon=True)
    return pl.save(fig, outdir, "perceiver_nl_gflops.png")


def plot_latency(by_impl, nls, meta, outdir):
    fig, ax = pl.axes("Latency vs number of latents", subtitle(meta))
    _lines(ax, by_impl, nls, "latency_ms_mean")
    ax.set_xscale("log", base=2)
    ax.set_yscale("log")
    ax.set_xticks(nls)
    ax.set_xticklabels([str(n) for n in nls])
    ax.minorticks_off()
    ax.set_xlabel("N_latent")
    ax.set_ylabel("latency per call (ms, log)")
    ax.legend(frameon=True)
    return pl.save(fig, outdir, "perceiver_nl_latency.png")


def plot_occupancy(by_impl, nls, meta, outdir):
    fig, ax = pl.axes("Workgroups launched vs compute units", subtitle(meta))
    drew = False
    for impl, rows in by_impl.items():
        pts = [(n, workgroups(rows.get(n))) for n in nls]
        pts = [(n, w) for n, w in pts if w]
        if pts:
            xs, ys = zip(*pts)
            pl.draw(ax, impl, xs, ys)
            drew = True
    if not drew:
        pl.plt.close(fig)
        return None
    cu = cu_count(meta.get("gpu"))
    if cu:
        ax.axhline(cu, color="#d62728", ls="--", lw=1.6, label=f"{cu} CUs (one round)")
    ax.set_xscale("log", base=2)
    ax.set_yscale("log")
    ax.set_xticks(nls)
    ax.set_xticklabels([str(n) for n in nls])
    ax.minorticks_off()
    ax.set_xlabel("N_latent")
    ax.set_ylabel("workgroups per call (log)")
    ax.legend(frameon=True, fontsize=8.5)
    return pl.save(fig, outdir, "perceiver_nl_occupancy.png")


def main(argv=None):
    ap = argparse.ArgumentParser(description="Plot the Perceiver N_latent sweep")
    ap.add_argument("--csv", default="results/perceiver_nl.csv")
    ap.add_argument("--outdir", default="results")
    args = ap.parse_args(argv)
    if not os.path.exists(args.csv):
        print(f"No log at {args.csv}; run bench_perceiver_nl.py first.")
        return 1
    by_impl, meta = pl.load(args.csv, "perceiver_nl", "N_latent")
    if not by_impl:
        print("No perceiver_nl rows in the log.")
        return 1
    nls = sorted({n for rows in by_impl.values() for n in rows})
    for p in (plot_gflops(by_impl, nls, meta, args.outdir),
              plot_latency(by_impl, nls, meta, args.outdir),
              plot_occupancy(by_impl, nls, meta, args.outdir)):
        if p:
            print(p)
    return 0


if __name__ == "__main__":
    sys.exit(main())
