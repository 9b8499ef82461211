"""
Shared pieces of the sweep figures (plot_perceiver.py, plot_perceiver_nl.py,
plot_pytorch_compare.py): reading the measurement log written by csvlog.py,
one colour / marker / label per implementation, axes set-up, and the MI355X
cache-capacity markers.  Pure matplotlib on the Agg backend: no GPU and no
kernels.so are needed to draw.
"""

import csv
import os

import matplotlib

matplotlib.use("Agg")
import matplotlib.pyplot as plt  # noqa: E402

RC = {
    "figure.figsize": (8, 5.2), "figure.dpi": 150, "savefig.dpi": 150,
    "savefig.bbox": "tight", "font.size": 12, "axes.titlesize": 14,
    "axes.titleweight": "bold", "axes.labelsize": 12, "legend.fontsize": 10,
    "axes.grid": True, "grid.linestyle": "--", "grid.alpha": 0.4,
    "axes.axisbelow": True, "figure.facecolor": "white",
}

# impl -> (colour, marker, legend label).  This library's kernels are the
# reference's implementation names (cuda_wrappers.LAUNCHERS and the split-K /
# WMMA drivers) rebuilt for gfx950; sdpa_* are PyTorch-ROCm's backends.
STYLE = {
    "naive": ("#d62728", "o", "Naive"),
    "warp": ("#1f77b4", "s", "Warp parallel"),
    "tiled": ("#2ca02c", "^", "Tiled"),
    "vectorized": ("#7a2fbf", "D", "fp32 MFMA (vectorized entry)"),
    "splitk": ("#000000", "*", "fp32 MFMA split-K"),
    "wmma": ("#ff7f0e", "P", "fp16 MFMA"),
    "wmma_bf16": ("#bcbd22", "P", "bf16 MFMA"),
    "wmma_splitk": ("#e377c2", "X", "fp16 MFMA split-K"),
    "wmma_splitk_bf16": ("#f7b6d2", "X", "bf16 MFMA split-K"),
    "sdpa_math": ("#8c564b", "v", "PyTorch SDPA-math (materialized)"),
    "bmm_fp16": ("#c49c94", "v", "torch bmm/softmax/bmm fp16 (materialized)"),
    "bmm_bf16": ("#dbb9a9", "v", "torch bmm/softmax/bmm bf16 (materialized)"),
    "sdpa_efficient": ("#17becf", "<", "PyTorch SDPA-efficient (fused)"),
    "sdpa_efficient_fp16": ("#9edae5", "<", "PyTorch SDPA-efficient fp16"),
    "sdpa_efficient_bf16": ("#6fc3cf", "<", "PyTorch SDPA-efficient bf16"),
    "sdpa_flash_fp16": ("#393b79", ">", "PyTorch SDPA-flash fp16"),
    "sdpa_flash_bf16": ("#6b6ecf", ">", "PyTorch SDPA-flash bf16"),
}
OURS = ("naive", "warp", "tiled", "vectorized", "splitk", "wmma", "wmma_bf16", "wmma_splitk",
        "wmma_splitk_bf16")

# Capacities a batch element's K and V cross as N_input grows (bytes): the L2
# of the XCD its workgroups run on (the library deals one batch element's row
# blocks to one XCD) and the device-wide Infinity Cache (MALL).
CACHES = {
    "MI355X": [("L2 / XCD 4 MB", 4 << 20), ("Infinity Cache 256 MB", 256 << 20)],
    "MI350X": [("L2 / XCD 4 MB", 4 << 20), ("Infinity Cache 256 MB", 256 << 20)],
}
OK = ("ok", "ACCURACY?")


def style(impl):
    return STYLE.get(impl, ("#7f7f7f", "o", impl))


def load(csv_path, experiment, key):
    """{impl: {key value: row}} of the log's rows of ``experiment``, plus the
    first row's gpu / shape / precision as a dict."""
    by_impl, meta = {}, {}
    with open(csv_path, newline="") as f:
        for r in csv.DictReader(f):
            if r.get("experiment") != experiment:
                continue
            try:
                x = int(r[key])
            except (KeyError, ValueError, TypeError):
                continue
            by_impl.setdefault(r.get("impl", "?"), {})[x] = r
            for field in ("gpu", "B", "N_latent", "N_input", "precision"):
                meta.setdefault(field, r.get(field, "?"))
    return by_impl, meta


def value(row, field):
    """A numeric field of a measured row; None for missing, refused or failed rows."""
    if not row or row.get("status") not in OK:
        return None
    try:
        return float(row.get(field, ""))
    except (TypeError, ValueError):
        return None


def series(rows, xs, field):
    """(x, y) lists of the points of one implementation that have ``field``."""
    pts = [(x, value(rows.get(x), field)) for x in xs]
    pts = [(x, y) for x, y in pts if y is not None]
    return [x for x, _ in pts], [y for _, y in pts]


def axes(title, subtitle):
    with plt.rc_context(RC):
        fig, ax = plt.subplots()
    ax.set_title(title, pad=22)
    ax.text(0.5, 1.015, subtitle, transform=ax.transAxes, ha="center", va="bottom",
            fontsize=9.5, color="0.35")
    return fig, ax


def draw(ax, impl, xs, ys, **kw):
    c, m, lab = style(impl)
    ax.plot(xs, ys, marker=m, color=c, label=lab,
            lw=2.4 if impl in OURS else 1.8, ms=8, **kw)


def log_x(ax, ticks, labels=None):
    ax.set_xscale("log")
    ax.set_xticks(ticks)
    ax.set_xticklabels(labels or [str(t) for t in ticks], fontsize=9)
    ax.minorticks_off()


def cache_markers(ax, gpu, bytes_per_key):
    """Vertical lines at the N_input where one batch element's K and V
    (bytes_per_key each key) outgrow each cache level of ``gpu``."""
    lo, hi = ax.get_xlim()
    for label, cap in CACHES.get(gpu, []):
        n = cap / bytes_per_key
        if lo <= n <= hi:
            ax.axvline(n, color="gray", ls=":", lw=1.3)
            ax.text(n, ax.get_ylim()[1], f" {label}", color="gray", fontsize=8, va="top",
                    ha="left", rotation=90)


def save(fig, outdir, name):
    os.makedirs(outdir, exist_ok=True)
    path = os.path.join(outdir, name)
    with plt.rc_context(RC):
        fig.savefig(path)
    plt.close(fig)
    return path


def square_label(n):
    """'50176\\n(224^2)' for perfect squares (image side), else the number."""
    r = int(round(n ** 0.5))
    return f"{n}\n({r}²)" if r * r == n else str(n)
