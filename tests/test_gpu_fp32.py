"""GPU parity of the fp32 entry points against the float64 oracle.

Gate (written here, from the build's correctness contract): max-abs <= 1e-4
and rel = max-abs / (max|ref| + 1e-6) <= 1e-3 (the rel definition of
experiments/bench_perceiver_ni.py:147-148).  Every case calls the HIP library
through its C ABI (cuda_wrappers -> kernels.so).
"""

import numpy as np
import pytest

from conftest import fp32_gate

pytestmark = pytest.mark.gpu


def _events(cw, impl, q, k, v):
    b, nl, d = q.shape
    out, _, _ = cw.benchmark_kernel_events(impl, q, k, v, b, nl, k.shape[1], d, warmup=1,
                                           iters=1)
    return out


# ---------------------------------------------------------------------------
# MFMA kernel (launch_optimized_kernel, the 'vectorized' impl)
# ---------------------------------------------------------------------------

def test_cfg1_matches_oracle_and_golden(cw, oracle):
    import os
    q, k, v = oracle.make_inputs(1, 64, 784, 768, seed=0)
    out = cw.run_vectorized_kernel(q[0], k[0], v[0], 64, 784, 768)
    fp32_gate(out, oracle.attention_f64(q, k, v))
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "cfg1_seed0.npz"))
    fp32_gate(out, g["out"])


def test_headline_shape_and_determinism(cw, oracle):
    q, k, v = oracle.make_inputs(32, 1024, 784, 768, seed=1)
    out1 = _events(cw, "vectorized", q, k, v)
    fp32_gate(out1, oracle.attention_f64(q, k, v))
    out2 = _events(cw, "vectorized", q, k, v)
    assert np.array_equal(out1, out2), "two launches differ bitwise"


@pytest.mark.parametrize("b,nl,ni", [(1, 1, 1), (1, 15, 17), (2, 17, 15), (1, 63, 16),
                                     (3, 65, 33), (1, 100, 785), (2, 129, 1000),
                                     (5, 64, 784), (1, 1024, 3)])
def test_edge_shapes(cw, oracle, b, nl, ni):
    q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=b * 1000 + nl + ni)
    fp32_gate(_events(cw, "vectorized", q, k, v), oracle.attention_f64(q, k, v))


@pytest.mark.parametrize("lpw", [64, 32, 16])
@pytest.mark.parametrize("s", [1, 3, 7])
def test_every_plan_form(cw, oracle, lpw, s):
    """Each workgroup size the planner may pick (64, 32 or 16 latents),
    unsplit and split, through launch_optimized_plan_kernel on a ragged
    shape (latents past the last full block, a partial last key tile)."""
    b, nl, ni = 2, 80, 200
    q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=43)
    res, _, _ = cw.benchmark_plan_events(q, k, v, b, nl, ni, 768, lpw, s, warmup=0, iters=1)
    fp32_gate(res, oracle.attention_f64(q, k, v))


def test_empty_key_set_gives_zeros(cw, oracle):
    q, _, _ = oracle.make_inputs(2, 70, 1, 768, seed=4)
    k = np.zeros((2, 0, 768), np.float32)
    out = _events(cw, "vectorized", q, k, k)
    assert out.shape == (2, 70, 768) and np.all(out == 0)


def test_config2_legacy_seed42_sweep(cw, oracle):
    for nl in (64, 128, 256, 512, 1024):
        q, k, v = oracle.make_inputs_legacy(1, nl, 784, 768, seed=42)
        fp32_gate(cw.run_vectorized_kernel(q[0], k[0], v[0], nl, 784, 768),
                  oracle.attention_f64(q, k, v))


@pytest.mark.parametrize("b", [4, 8, 16, 32])
def test_config3_batched_sweep(cw, oracle, b):
    for nl in (64, 128, 256, 512, 1024):
        q, k, v = oracle.make_inputs_legacy(b, nl, 784, 768, seed=42)
        fp32_gate(_events(cw, "vectorized", q, k, v), oracle.attention_f64(q, k, v))


@pytest.mark.parametrize("lpw", [16, 32, 64])
def test_growing_scores_force_rescales(cw, oracle, lpw):
    """Scores rise by ~12 per key across the key axis, so the running max grows
    far past the lazy-rescale threshold many times within one row.  Each
    workgroup size (16, 32 or 64 latents) runs the keys unsplit through
    launch_optimized_plan_kernel: one workgroup walks all 200 keys and must
    rescale on the way.  The same inputs also run through the library's own
    plan (launch_optimized_kernel, which splits the keys at this shape) and
    launch_splitk_kernel with one split, whose partials must normalise to the
    output."""
    rng = np.random.RandomState(8)
    b, nl, ni = 2, 40, 200
    u = rng.randn(768)
    u /= np.linalg.norm(u)
    q = np.empty((1, nl, 768), np.float32)
    q[0] = (u * np.sqrt(768.0) * (1.0 + 0.01 * rng.randn(nl, 1)) + 0.1 * rng.randn(nl, 768))
    # raw dot q.k_j ~ 12 j, i.e. the score grows by 12/sqrt(768) = 0.43 per key
    k = (np.arange(ni)[:, None] * (12.0 / np.sqrt(768.0)) * u
         + 0.05 * rng.randn(ni, 768))[None].astype(np.float32)
    k = k[:, rng.permutation(ni)]  # rescales happen in every order
    v = rng.randn(1, ni, 768).astype(np.float32)
    ref = np.repeat(oracle.attention_f64(q, k, v), b, axis=0)
    order = np.argsort(k[0] @ u)
    k_sorted, v_sorted = k[:, order], v[:, order]
    q, k, v, k_sorted, v_sorted = (np.repeat(a, b, axis=0) for a in (q, k, v, k_sorted, v_sorted))
    for kk, vv in ((k, v), (k_sorted, v_sorted)):
        out, _, _ = cw.benchmark_plan_events(q, kk, vv, b, nl, ni, 768, lpw, 1, warmup=0, iters=1)
        fp32_gate(out, ref)
        fp32_gate(_events(cw, "vectorized", q, kk, vv), ref)
        out, (po, pm, pl) = cw.splitk_partials(q, kk, vv, b, nl, ni, 768, 1)
        fp32_gate(out, ref)
        fp32_gate(po.reshape(out.shape) / pl.reshape(b, nl, 1), ref)


def test_special_cases(cw, oracle):
    q, k, v = oracle.make_inputs(2, 33, 50, 768, seed=12)
    ones = np.ones_like(v)
    out = _events(cw, "vectorized", q, k, ones)
    assert np.max(np.abs(out - 1.0)) < 2e-6
    out = _events(cw, "vectorized", q, np.zeros_like(k), v)
    assert np.max(np.abs(out - v.mean(axis=1, keepdims=True))) < 1e-5


@pytest.mark.parametrize("lpw", [64, 32, 16])
@pytest.mark.parametrize("s", [1, 3])
def test_closed_forms_every_plan_form(cw, oracle, lpw, s):
    """The same closed forms through each fp32 workgroup form, unsplit and
    split (the merge included): V = 1 gives sum(p) / (sum(p) + 1e-6) = 1 to
    within 2e-6, and K = 0 gives every weight exp(0) = 1, i.e. the mean of
    V over the keys, on a ragged shape (a partial last key tile, latents
    past the last full block)."""
    b, nl, ni = 2, 70, 150
    q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=13)

    def run(kk, vv):
        out, _, _ = cw.benchmark_plan_events(q, kk, vv, b, nl, ni, 768, lpw, s,
                                             warmup=0, iters=1)
        return out

    out = run(k, np.ones_like(v))
    assert np.all(np.isfinite(out)) and np.max(np.abs(out - 1.0)) < 2e-6
    out = run(np.zeros_like(k), v)
    mean = v.astype(np.float64).sum(axis=1, keepdims=True) / (ni + 1e-6)
    assert np.max(np.abs(out - mean)) < 1e-5


# ---------------------------------------------------------------------------
# split-K (launch_splitk_kernel): output and the caller-visible partials
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("s", [1, 3, 8, 19, 64, 100])
def test_splitk_output_and_partials(cw, oracle, s):
    b, nl, ni = 2, 70, 300
    q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=s)
    out, (po, pm, pl) = cw.splitk_partials(q, k, v, b, nl, ni, 768, s)
    fp32_gate(out, oracle.attention_f64(q, k, v))
    rpo, rpm, rpl = oracle.splitk_partials(q, k, v, s)
    live = rpm > -oracle.FLT_MAX
    assert np.array_equal(pm[~live], np.full((~live).sum(), -oracle.FLT_MAX, np.float32))
    assert np.all(pl[~live] == 0) and np.all(po[~live] == 0)
    assert np.max(np.abs(pm[live] - rpm[live])) < 1e-5
    assert np.max(np.abs(pl[live] - rpl[live]) / rpl[live]) < 1e-5
    fp32_gate(po[live] / pl[live][:, None], rpo[live] / rpl[live][:, None])


def test_splitk_golden(cw, oracle):
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "splitk_small.npz"))
    b, nl, ni, d, s = [int(x) for x in g["shape"]]
    q, k, v = oracle.make_inputs(b, nl, ni, d, seed=3)
    out, (po, pm, pl) = cw.splitk_partials(q, k, v, b, nl, ni, d, s)
    fp32_gate(out, g["out"])
    fp32_gate(po, g["po"])
    assert np.allclose(pm, g["pm"], atol=1e-5) and np.allclose(pl, g["pl"], rtol=1e-5)


@pytest.mark.parametrize("b,nl,ni,q_std", [(1, 64, 784, 1.0), (1, 256, 4096, 0.02),
                                           (2, 70, 300, 1.0), (1, 1000, 784, 1.0)])
def test_merge_column_parts_bit_identical(cw, oracle, b, nl, ni, q_std):
    """The LSE merge split over 2 or 4 workgroups per row (and the library's
    choice) gives the one-workgroup-per-row merge's output bit for bit, on
    the partials of configuration 1, of configuration 4 at N_input 4,096
    (the library plan's split counts), of a ragged shape and of a shape with
    rows enough for one workgroup per row; the split launch's own output
    equals them."""
    q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=7, q_std=q_std)
    cu, _ = cw.device_info()
    s = cw.plan_num_splits(nl, ni, b, cu)
    if s == 1:
        s = 5
    out, (po, pm, pl) = cw.splitk_partials(q, k, v, b, nl, ni, 768, s)
    rows = b * nl
    po, pm, pl = po.reshape(rows, s, 768), pm.reshape(rows, s), pl.reshape(rows, s)
    merged = {c: cw.lse_combine(po, pm, pl, c) for c in (1, 2, 4, 0)}
    for c in (2, 4, 0):
        assert np.array_equal(merged[c], merged[1]), f"{c} column parts differ from 1"
    assert np.array_equal(out.reshape(rows, 768), merged[1])
    fp32_gate(out, oracle.attention_f64(q, k, v))
    assert cw.lib.xattn_lse_combine_parts(rows, s, cu) in (1, 2, 4)


@pytest.mark.parametrize("ni", [4096, 16384, 50176])
def test_config4_long_input(cw, oracle, ni):
    cu, _ = cw.device_info()
    q, k, v = oracle.make_inputs(1, 256, ni, 768, seed=ni, q_std=0.02)
    out, _, _, s = cw.benchmark_splitk_events(q, k, v, 1, 256, ni, 768, warmup=1, iters=1,
                                              sm_count=cu)
    assert s > 1
    fp32_gate(out, oracle.attention_f64(q, k, v))
    fp32_gate(_events(cw, "vectorized", q, k, v), oracle.attention_f64(q, k, v))


# ---------------------------------------------------------------------------
# ladder rungs
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("impl", ["naive", "warp", "tiled"])
@pytest.mark.parametrize("b,nl,ni,d", [(2, 9, 50, 768), (1, 5, 33, 64), (1, 7, 17, 100),
                                       (1, 4, 0, 768)])
def test_rungs(cw, oracle, impl, b, nl, ni, d):
    q, k, v = oracle.make_inputs(b, nl, ni, d, seed=nl * ni + d)
    out = _events(cw, impl, q, k, v)
    fp32_gate(out, oracle.attention_f64(q, k, v))


@pytest.mark.parametrize("fn", ["run_naive_kernel", "run_warp_parallel_kernel",
                                "run_tiled_kernel", "run_vectorized_kernel"])
def test_legacy_drivers_2d_inputs(cw, oracle, fn):
    q, k, v = oracle.make_inputs_legacy(1, 64, 784, 768, seed=42)
    out = getattr(cw, fn)(q[0], k[0], v[0], 64, 784, 768)
    assert out.shape == (1, 64, 768)
    fp32_gate(out, oracle.attention_f64(q, k, v))


def test_nan_stays_where_the_reference_puts_it(cw, oracle):
    """A NaN in one batch element's K makes that element's whole output NaN
    (every latent scores the key); a NaN in its V makes only that output
    column NaN (each weight times it).  The reference's softmax formulation
    (the oracle) puts them there; every other value must match it.  Through
    the planned launch (B=3 N_latent=64 N_input=100: a split plan) and
    launch_splitk_kernel with 3 splits."""
    b, nl, ni = 3, 64, 100
    for where in ("K", "V"):
        q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=77)
        (k if where == "K" else v)[1, 37, 5] = np.nan
        ref = oracle.attention_f64(q, k, v)
        nan = np.isnan(ref)
        assert nan[1].any() and not nan[[0, 2]].any()
        for name, out in (("planned", _events(cw, "vectorized", q, k, v)),
                          ("split-K", cw.splitk_partials(q, k, v, b, nl, ni, 768, 3)[0])):
            assert np.array_equal(np.isnan(out), nan), f"NaN in {where}: {name} NaN pattern"
            fp32_gate(np.where(nan, 0.0, out), np.where(nan, 0.0, ref))
