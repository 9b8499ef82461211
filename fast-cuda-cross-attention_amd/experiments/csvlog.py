"""
Measurement log: one CSV row per measured (experiment, impl, shape) point.

The column set is the reference's (experiments/csvlog.py:12-25), so rows
written here and rows from the reference's runs on other hardware load into
one table.  Fields a row does not set stay empty; extra keys are ignored.
The header is written only when the file is new or empty, so several runs
append to one file.
"""

import csv
import os

FIELDS = [
    "experiment",            # which sweep produced the row
    "gpu",                   # gpu_specs key (e.g. MI355X) or the raw device name
    "impl",                  # naive|warp|tiled|vectorized|splitk|wmma|wmma_splitk|..._bf16|sdpa_*
    "precision",             # fp32|fp16|bf16
    "B", "N_latent", "N_input", "D",
    "latency_ms_mean", "latency_ms_std",
    "achieved_gflops", "achieved_gbs",
    "pct_peak_compute", "pct_peak_bw",
    "arithmetic_intensity", "ridge_point", "bound",
    "max_abs_err", "rel_err",
    "status",                # ok | error | unsupported | design-limited | ACCURACY?
    "note",
]


def writer(path):
    """Open ``path`` for appending; returns (file, csv.DictWriter).  The
    header goes in first when the file does not exist yet or is empty."""
    fresh = not os.path.exists(path) or os.path.getsize(path) == 0
    fh = open(path, "a", newline="")
    w = csv.DictWriter(fh, fieldnames=FIELDS, extrasaction="ignore")
    if fresh:
        w.writeheader()
    return fh, w


def write_row(path, **fields):
    """Append one row (missing fields empty)."""
    fh, w = writer(path)
    try:
        w.writerow(fields)
    finally:
        fh.close()


def read_rows(path):
    """All rows of a log as dicts (strings, as written)."""
    with open(path, newline="") as fh:
        return list(csv.DictReader(fh))
