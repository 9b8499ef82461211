"""The drop-in harness: data generators (CPU) and end-to-end runs (GPU)."""

import os

import numpy as np
import pytest


def test_generators_match_oracle(tmp_path, oracle):
    import generate_references as gr
    gr.write_single(str(tmp_path), [16])
    sub = tmp_path / "N_latent_16"
    q, k, v, ref = (np.load(sub / f"{n}.npy") for n in
                    ("Q_matrix", "K_matrix", "V_matrix", "output_reference"))
    assert q.shape == (16, 768) and k.shape == (784, 768) and ref.shape == (1, 16, 768)
    oq, ok, ov = oracle.make_inputs_legacy(1, 16, 784, 768, seed=42)
    assert np.array_equal(q, oq[0]) and np.array_equal(k, ok[0]) and np.array_equal(v, ov[0])
    assert oracle.max_abs(ref, oracle.attention_f64(oq, ok, ov)) < 2e-6

    gr.write_batched(str(tmp_path), [3], [8])
    sub = tmp_path / "batches" / "batch_3" / "N_latent_8"
    q, ref = np.load(sub / "Q_matrix.npy"), np.load(sub / "output_reference.npy")
    oq, ok, ov = oracle.make_inputs_legacy(3, 8, 784, 768, seed=42)
    assert np.array_equal(q, oq) and ref.shape == (3, 8, 768)
    assert oracle.max_abs(ref, oracle.attention_f64(oq, ok, ov)) < 2e-6


def test_verify_and_load_helpers(tmp_path, monkeypatch, capsys):
    import benchmark
    ref = np.zeros((1, 2, 3))
    assert benchmark.verify_output(ref + 1e-4, ref, "x", tolerance=1e-3)
    assert not benchmark.verify_output(ref + 1e-2, ref, "x", tolerance=1e-3)
    assert "WARNING" in capsys.readouterr().out
    monkeypatch.setattr(benchmark, "DATA_DIR", str(tmp_path))
    assert benchmark.load_reference_data(64) == (None, None, None, None)


@pytest.mark.gpu
def test_single_batch_harness_end_to_end(tmp_path, monkeypatch, cw):
    import benchmark
    import generate_references as gr
    gr.write_single(str(tmp_path / "data"), [64, 128])
    monkeypatch.chdir(tmp_path)
    monkeypatch.setattr(benchmark, "N_latent_values", [64, 128])
    monkeypatch.setattr(benchmark, "_timed",
                        lambda fn, args, it, wu: (fn(*args), 1.0))  # one call each
    res = benchmark.run_unified_benchmark()
    assert res["N_latent"] == [64, 128]
    for key in ("naive", "parallel", "tiled", "optimized"):
        assert all(t is not None for t in res[key]), key


@pytest.mark.gpu
def test_batched_harness_end_to_end(tmp_path, monkeypatch, cw, capsys):
    import benchmark
    import benchmark_batching
    import generate_references as gr
    gr.write_batched(str(tmp_path / "data"), [4], [64])
    monkeypatch.chdir(tmp_path)
    monkeypatch.setattr(benchmark, "_timed", lambda fn, args, it, wu: (fn(*args), 1.0))
    res = benchmark_batching.run_batch_benchmark([4], [64])
    assert res[4]["N_latent"] == [64]
    out = capsys.readouterr().out
    assert out.count("Verification passed") == 4, out
