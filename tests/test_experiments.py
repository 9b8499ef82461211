"""The experiment drivers' host side: log schema, device ceilings, roofline
figures, the Perceiver fixture format (no GPU)."""

import csv
import math
import os
import sys

import numpy as np
import pytest

from conftest import PKG

EXP = os.path.join(PKG, "experiments")
if EXP not in sys.path:
    sys.path.insert(0, EXP)

import csvlog  # noqa: E402
import gen_perceiver_refs as gpr  # noqa: E402
import gpu_specs  # noqa: E402
import roofline  # noqa: E402
import sweep  # noqa: E402


def test_csvlog_header_once_and_append(tmp_path):
    path = str(tmp_path / "log.csv")
    csvlog.write_row(path, experiment="e", impl="vectorized", B=1, unknown="dropped")
    fh, w = csvlog.writer(path)
    w.writerow({"experiment": "e", "impl": "splitk", "status": "ok"})
    fh.close()
    with open(path) as f:
        lines = f.read().splitlines()
    assert lines[0].split(",") == csvlog.FIELDS
    assert len(lines) == 3 and "dropped" not in lines[1]
    rows = csvlog.read_rows(path)
    assert [r["impl"] for r in rows] == ["vectorized", "splitk"] and rows[0]["B"] == "1"
    # the column set the reference's plots read
    assert csvlog.FIELDS[:8] == ["experiment", "gpu", "impl", "precision", "B", "N_latent",
                                 "N_input", "D"]
    assert len(csvlog.FIELDS) == 21 and csvlog.FIELDS[-2:] == ["status", "note"]


def test_gpu_keys_and_ridges(monkeypatch):
    assert gpu_specs.gpu_key_for_name("AMD Instinct MI355X") == "MI355X"
    assert gpu_specs.gpu_key_for_name("AMD Instinct MI350X") == "MI350X"
    assert gpu_specs.gpu_key_for_name("AMD Instinct MI300X") is None
    assert gpu_specs.gpu_key_for_name(None) is None
    # ridge = peak / bandwidth: 157.3 TFLOP/s / 8 TB/s and 2516.6 / 8
    assert gpu_specs.ridge_point("MI355X", "fp32") == pytest.approx(19.6625)
    assert gpu_specs.ridge_point("MI355X", "bf16") == pytest.approx(314.575)
    assert gpu_specs.ridge_point("MI355X", "fp16") == gpu_specs.ridge_point("MI355X", "bf16")
    # MI350X is the same chip at 2.2 / 2.4 of the clock
    r = gpu_specs.GPU_SPECS["MI350X"]["peak_fp32_flops"] / gpu_specs.GPU_SPECS["MI355X"][
        "peak_fp32_flops"]
    assert r == pytest.approx(2.2 / 2.4, rel=2e-3)
    monkeypatch.setenv("XATTN_GPU_KEY", "MI355X")
    assert gpu_specs.detect_gpu_name() == "MI355X"
    monkeypatch.setenv("XATTN_GPU_KEY", "nonsense")
    assert gpu_specs.detect_gpu_name() is None


def test_roofline_headline_figures():
    # headline B=32 NL=1024 NI=784 D=768: 78.92 GFLOP, 355.47 MB (fp32, fused)
    assert roofline.flops(32, 1024, 784, 768) == pytest.approx(78.92e9, rel=1e-4)
    assert roofline.bytes_moved(32, 1024, 784, 768) == pytest.approx(355.47e6, rel=1e-4)
    # bf16 inputs with fp32 rows out: 32 * (1024*768*2 + 2*784*768*2 + 1024*768*4)
    assert roofline.bytes_moved(32, 1024, 784, 768, "bf16", out_precision="fp32") == \
        32 * (1024 * 768 * 2 + 2 * 784 * 768 * 2 + 1024 * 768 * 4)
    # the reference's fused 16-bit model writes the output in 16 bits too
    assert roofline.bytes_moved(1, 256, 4096, 768, "fp16") == (2 * 256 + 2 * 4096) * 768 * 2
    # materialized adds a write and a read of the score matrix
    assert (roofline.bytes_moved(2, 3, 5, 768, "fp32", materialized=True)
            - roofline.bytes_moved(2, 3, 5, 768, "fp32")) == 2 * 2 * 3 * 5 * 4
    row = roofline.roofline_row(32, 1024, 784, 768, 1e-3, "MI355X")
    assert row["pct_peak_compute"] == pytest.approx(100 * 78.92e9 / 1e-3 / 157.3e12, rel=1e-4)
    assert row["pct_peak_bw"] == pytest.approx(100 * 355.47e6 / 1e-3 / 8e12, rel=1e-4)
    assert row["bound"] == "compute" and row["arithmetic_intensity"] == pytest.approx(222.0,
                                                                                      rel=1e-3)
    # an unknown card gets no %-peak columns
    assert "pct_peak_compute" not in roofline.roofline_row(1, 4, 4, 768, 1e-3, None)
    # small N_input in 16 bits is on the memory side of the ridge
    assert roofline.roofline_row(1, 16, 16, 768, 1e-3, "MI355X", "bf16")["bound"] == "memory"


def test_perceiver_fixture_format(tmp_path, oracle):
    sub = gpr.write_case(str(tmp_path), 8, 40, seed=42)
    assert sub.endswith(os.path.join("perceiver", "Nl8_Ni40"))
    Q, K, V, ref = gpr.load_case(str(tmp_path), 8, 40)
    assert Q.dtype == K.dtype == V.dtype == ref.dtype == np.float32
    assert Q.shape == (8, 768) and K.shape == V.shape == (40, 768) and ref.shape == (1, 8, 768)
    # RandomState(42): Q, then K, then V, standard normal
    rng = np.random.RandomState(42)
    assert np.array_equal(Q, rng.randn(8, 768).astype(np.float32))
    assert np.array_equal(K, rng.randn(40, 768).astype(np.float32))
    assert np.array_equal(V, rng.randn(40, 768).astype(np.float32))
    assert oracle.max_abs(ref, oracle.attention_f64(Q[None], K[None], V[None])) < 1e-6
    assert gpr.load_case(str(tmp_path), 8, 41) is None


def test_reference_output_known_answers():
    rng = np.random.RandomState(3)
    q, k = rng.randn(5, 768).astype(np.float32), rng.randn(9, 768).astype(np.float32)
    v = np.ones((9, 768), np.float32)
    assert np.allclose(gpr.reference_output(q, k, v), 1.0, atol=1e-6)   # rows of P sum to 1
    v = rng.randn(9, 768).astype(np.float32)
    z = gpr.reference_output(np.zeros_like(q), k, v)                    # uniform weights
    assert np.allclose(z, v.mean(axis=0, keepdims=True), atol=1e-6)
    one = gpr.reference_output(q, k[:1], v[:1])                          # a single key
    assert np.allclose(one, v[:1], atol=1e-6)


def test_impl_precisions_and_backends():
    assert sweep.precision_of("vectorized") == "fp32"
    assert sweep.precision_of("wmma") == sweep.precision_of("wmma_splitk") == "fp16"
    assert sweep.precision_of("wmma_splitk_bf16") == "bf16"
    assert sweep.precision_of("sdpa_math") == "fp32"
    assert sweep.precision_of("sdpa_flash_fp16") == "fp16"
    assert sweep.precision_of("sdpa_efficient_bf16") == "bf16"
    assert sweep.sdpa_backend_of("sdpa_eff") == "efficient"
    assert sweep.sdpa_backend_of("sdpa_math_bf16") == "math"
    with pytest.raises(ValueError):
        sweep.sdpa_backend_of("sdpa_cudnn")


def test_drivers_report_missing_references(tmp_path, monkeypatch, capsys):
    """Without generated data a sweep prints how to make it and logs nothing
    but the header (no GPU is touched)."""
    import bench_perceiver_ni
    import bench_perceiver_nl
    import bench_wmma
    monkeypatch.setenv("XATTN_GPU_KEY", "MI355X")
    monkeypatch.chdir(tmp_path)
    for mod, extra in ((bench_perceiver_ni, ["--n-input", "784"]),
                       (bench_perceiver_nl, ["--n-latent", "16"]),
                       (bench_wmma, ["--n-input", "784"])):
        csv_path = str(tmp_path / f"{mod.__name__}.csv")
        assert mod.main(["--data", str(tmp_path / "none"), "--csv", csv_path] + extra) == 0
        out = capsys.readouterr().out
        assert "gen_perceiver_refs.py" in out, out
        with open(csv_path) as f:
            assert list(csv.reader(f)) == [csvlog.FIELDS]


def test_workgroup_counts(cw):
    import bench_perceiver_nl as nl
    cu = 256
    assert nl.workgroups(cw, "warp", 1, 16, 3136, cu) == 4
    assert nl.workgroups(cw, "naive", 2, 16, 3136, cu) == 2 * 4 * 12
    # small row blocks, split over the keys until the CUs are covered
    lpw, s = cw.f32_plan(1, 64, 3136, cu)
    assert s > 1 and nl.workgroups(cw, "vectorized", 1, 64, 3136, cu) == (64 // lpw) * s
    s = cw.plan_num_splits(1024, 3136, 1, cu)
    lpw = cw.lib.xattn_f32_split_latents(1, 1024, 3136, s, cu)
    assert s > 1 and nl.workgroups(cw, "splitk", 1, 1024, 3136, cu) == (1024 // lpw) * s
    assert math.ceil(1024 / cw.LATENTS_PER_WORKGROUP) == 16


def test_gpu_key_from_arch():
    assert gpu_specs.gpu_key_for_arch("gfx950:sramecc+:xnack-", 2400000) == "MI355X"
    assert gpu_specs.gpu_key_for_arch("gfx950", 2200000) == "MI350X"
    assert gpu_specs.gpu_key_for_arch("gfx942:sramecc+:xnack-", 2100000) is None
    assert gpu_specs.gpu_key_for_arch(None, 0) is None
