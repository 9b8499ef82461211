"""The sweep figures and the comparison table drawn from a synthetic log
(no GPU): every figure is written as a PNG, refused and failed rows are left
out, and the table is sorted, highlighted and normalised to SDPA-math."""

import os
import sys

import pytest

from conftest import PKG

EXP = os.path.join(PKG, "experiments")
if EXP not in sys.path:
    sys.path.insert(0, EXP)

import comparison_table  # noqa: E402
import csvlog  # noqa: E402
import plot_perceiver  # noqa: E402
import plot_perceiver_nl  # noqa: E402
import plot_pytorch_compare  # noqa: E402
import plotting  # noqa: E402
import roofline  # noqa: E402

PNG = b"\x89PNG\r\n\x1a\n"
NIS = [784, 3136, 4096, 12544, 50176]
# synthetic latency model per impl: ms = a + b * NI
MODEL = {"warp": (0.2, 4e-4), "tiled": (0.1, 2e-4), "vectorized": (0.01, 2e-5),
         "splitk": (0.01, 6e-6), "wmma_bf16": (0.005, 2e-6), "sdpa_math": (0.02, 8e-6),
         "sdpa_efficient": (0.05, 3e-5)}


def _row(experiment, impl, b, nl, ni, ms, **kw):
    prec = "bf16" if impl.endswith("bf16") else "fp32"
    r = roofline.roofline_row(b, nl, ni, 768, ms / 1e3, "MI355X", precision=prec,
                              materialized=impl == "sdpa_math")
    row = dict(experiment=experiment, gpu="MI355X", impl=impl, precision=prec, B=b,
               N_latent=nl, N_input=ni, D=768, latency_ms_mean=f"{ms:.6f}",
               latency_ms_std="0.0", status="ok", **r)
    row.update(kw)
    return row


@pytest.fixture(scope="module")
def log(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("log") / "runs.csv")
    fh, w = csvlog.writer(path)
    for impl, (a, b) in MODEL.items():
        for ni in NIS:
            if impl == "warp" and ni > 3136:
                w.writerow(dict(experiment="perceiver_ni", gpu="MI355X", impl=impl, B=1,
                                N_latent=256, N_input=ni, D=768, status="design-limited",
                                note="score row exceeds LDS"))
                continue
            w.writerow(_row("perceiver_ni", impl, 1, 256, ni, a + b * ni))
    for nl in (64, 128, 256, 512, 1024):
        for impl in ("warp", "tiled", "vectorized"):
            w.writerow(_row("perceiver_nl", impl, 1, nl, 3136, 0.01 + nl * 1e-4,
                            note=f"blocks={nl // 4};act_cu={min(nl // 4, 256)}"))
    for impl, ms in (("sdpa_math", 0.05), ("splitk", 0.047), ("sdpa_efficient_fp16", 0.2),
                     ("wmma_bf16", 0.02)):
        w.writerow(_row("anchor", impl, 1, 256, 4096, ms))
    # a failed row carries no latency and must not appear anywhere
    w.writerow(dict(experiment="anchor", gpu="MI355X", impl="sdpa_flash_fp16", B=1,
                    N_latent=256, N_input=4096, D=768, status="unsupported"))
    fh.close()
    return path


def _pngs(outdir, names):
    for n in names:
        p = os.path.join(outdir, n)
        assert os.path.exists(p), n
        with open(p, "rb") as f:
            assert f.read(8) == PNG, n


def test_ni_figures(log, tmp_path):
    out = str(tmp_path)
    assert plot_perceiver.main(["--csv", log, "--outdir", out]) == 0
    _pngs(out, ["perceiver_latency_vs_ni.png", "perceiver_speedup_vs_warp.png",
                "perceiver_gflops_vs_ni.png", "perceiver_pct_peak_vs_ni.png",
                "perceiver_roofline.png"])


def test_nl_figures(log, tmp_path):
    out = str(tmp_path)
    assert plot_perceiver_nl.main(["--csv", log, "--outdir", out]) == 0
    _pngs(out, ["perceiver_nl_gflops.png", "perceiver_nl_latency.png",
                "perceiver_nl_occupancy.png"])
    assert plot_perceiver_nl.workgroups({"note": "blocks=37;act_cu=37"}) == 37
    assert plot_perceiver_nl.workgroups({"note": "x=1"}) is None


def test_sdpa_figures(log, tmp_path):
    out = str(tmp_path)
    assert plot_pytorch_compare.main(["--csv", log, "--outdir", out, "--anchor", "4096"]) == 0
    _pngs(out, ["pytorch_latency_vs_ni.png", "pytorch_bar_anchor.png",
                "pytorch_slowdown_vs_math.png"])


def test_missing_log_is_reported(tmp_path):
    missing = str(tmp_path / "none.csv")
    assert plot_perceiver.main(["--csv", missing, "--outdir", str(tmp_path)]) == 1
    assert comparison_table.main(["--csv", missing, "--out", str(tmp_path / "t.tex")]) == 1


def test_series_skips_refused_rows(log):
    by_impl, meta = plotting.load(log, "perceiver_ni", "N_input")
    xs, ys = plotting.series(by_impl["warp"], NIS, "latency_ms_mean")
    assert xs == [784, 3136] and len(ys) == 2
    assert meta["gpu"] == "MI355X" and meta["N_latent"] == "256"


def test_comparison_table(log, tmp_path):
    out = str(tmp_path / "table.tex")
    assert comparison_table.main(["--csv", log, "--out", out]) == 0
    text = open(out).read()
    body = [ln for ln in text.splitlines() if ln.rstrip().endswith(r"\\") and "&" in ln][1:]
    names = [ln.split("&")[0].replace(r"\rowcolor{ours}", "").strip() for ln in body]
    # fastest first; the failed flash row is absent
    assert names == ["wmma\\_bf16", "splitk", "sdpa\\_math", "sdpa\\_efficient\\_fp16"]
    ratios = [ln.split("&")[-1].replace(r"\\", "").strip() for ln in body]
    assert ratios == ["2.50", "1.06", "1.00", "0.25"]  # SDPA-math latency / row latency
    assert sum(r"\rowcolor{ours}" in ln for ln in body) == 2
    assert r"\begin{tabular}" in text and r"\end{document}" in text
    # the same table from the N_input sweep's rows at one shape
    assert comparison_table.main(["--csv", log, "--experiment", "perceiver_ni",
                                  "--n-input", "4096", "--out", out]) == 0
    assert "warp" not in open(out).read()  # design-limited at 4096
