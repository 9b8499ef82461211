"""GPU parity of the fp16 / bf16 MFMA entry points.

Gates: rel <= 2e-2 against the fp32 oracle on the unrounded inputs (the
build's reduced-precision contract), plus a tighter check against the oracle
evaluated on exactly the rounded inputs the kernel sees, which isolates the
kernel's own error (P rounded to 16 bits, fp32 accumulation):
rel <= 4e-3 for bf16 and <= 1e-3 for fp16.
"""

import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from conftest import GATE16 as GATE, TIGHT16 as TIGHT


def _rounded_ref(oracle, cw, q, k, v, bf16):
    """float64 attention on the rounded inputs (Q pre-scaled then rounded)."""
    qh, kh, vh = cw._half_inputs(q, k, v, q.shape[0], q.shape[-1], bf16)
    if bf16:
        f = oracle.bf16_bits_to_f32
        qf, kf, vf = f(qh), f(kh), f(vh)
    else:
        qf, kf, vf = (a.astype(np.float32) for a in (qh, kh, vh))
    return oracle.attention_f64(qf.astype(np.float64) * math.sqrt(q.shape[-1]), kf, vf)


def _run(cw, q, k, v, bf16):
    b, nl, d = q.shape
    fn = cw.benchmark_wmma_bf16_events if bf16 else cw.benchmark_wmma_events
    out, _, _ = fn(q, k, v, b, nl, k.shape[1], d, warmup=1, iters=1)
    return out


def _check(oracle, cw, out, q, k, v, bf16):
    assert np.all(np.isfinite(out))
    rel = oracle.rel_err(out, oracle.attention_f64(q, k, v))
    tight = oracle.rel_err(out, _rounded_ref(oracle, cw, q, k, v, bf16))
    assert rel <= GATE, f"rel vs fp32 oracle {rel:.3e}"
    assert tight <= TIGHT[bf16], f"rel vs rounded-input oracle {tight:.3e}"
    return rel, tight


@pytest.mark.parametrize("bf16", [False, True], ids=["fp16", "bf16"])
def test_config5(cw, oracle, bf16):
    q, k, v = oracle.make_inputs(16, 512, 784, 768, seed=5)
    _check(oracle, cw, _run(cw, q, k, v, bf16), q, k, v, bf16)


@pytest.mark.parametrize("bf16", [False, True], ids=["fp16", "bf16"])
@pytest.mark.parametrize("b,nl,ni", [(1, 1, 1), (2, 17, 33), (1, 100, 785), (3, 64, 31),
                                     (1, 65, 64), (1, 64, 784), (32, 1024, 784)])
def test_shapes(cw, oracle, bf16, b, nl, ni):
    q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=b + nl + ni)
    _check(oracle, cw, _run(cw, q, k, v, bf16), q, k, v, bf16)


@pytest.mark.parametrize("bf16", [False, True], ids=["fp16", "bf16"])
@pytest.mark.parametrize("b,nl,ni,s", [(16, 512, 784, 0), (1, 64, 784, 0), (2, 48, 500, 9)],
                         ids=["config5", "split-plan", "splitk-9"])
def test_bitwise_repeatable(cw, oracle, bf16, b, nl, ni, s):
    """Two runs on the same inputs give identical bits: no reduction order
    depends on timing (the two owners of a latent block, the split partials
    and their merge are combined in a fixed order).  s = 0: the plain entry
    point with the library's own plan; s > 0: the split-K entry point."""
    q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=77)
    if s == 0:
        a, c = _run(cw, q, k, v, bf16), _run(cw, q, k, v, bf16)
    else:
        a, pa = cw.wmma_splitk_partials(q, k, v, b, nl, ni, 768, s, bf16=bf16)
        c, pc = cw.wmma_splitk_partials(q, k, v, b, nl, ni, 768, s, bf16=bf16)
        for x, y in zip(pa, pc):
            assert np.array_equal(x, y)
    assert np.array_equal(a, c)
    _check(oracle, cw, a, q, k, v, bf16)


def _run_plan(cw, q, k, v, bf16, lpw, cp, s):
    """One launch_wmma_plan_kernel call with the given plan; the output."""
    b, nl, d = q.shape
    out, _, _ = cw.benchmark_plan_events(q, k, v, b, nl, k.shape[1], d, lpw, s, cp,
                                         "bf16" if bf16 else "fp16", warmup=0, iters=1)
    return out


@pytest.mark.parametrize("bf16", [False, True], ids=["fp16", "bf16"])
@pytest.mark.parametrize("lpw,cp", [(64, 1), (64, 2), (32, 1)], ids=["64", "64x2cols", "32"])
@pytest.mark.parametrize("s", [1, 3, 7])
def test_every_plan_form(cw, oracle, bf16, lpw, cp, s):
    """Each workgroup form the planner may pick (64 latents, 64 latents in
    two column halves, 32 latents), unsplit and split, on a ragged shape
    (latents past the last full block, a partial last key tile), checked
    against the oracle.  Unsplit, the column halves give the full-width
    form's bits (the same scores, weights and MFMAs per output column)."""
    b, nl, ni = 2, 80, 200
    q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=41)
    out = _run_plan(cw, q, k, v, bf16, lpw, cp, s)
    _check(oracle, cw, out, q, k, v, bf16)
    if s == 1 and cp == 2:
        assert np.array_equal(out, _run_plan(cw, q, k, v, bf16, 64, 1, 1))


@pytest.mark.parametrize("bf16", [False, True], ids=["fp16", "bf16"])
@pytest.mark.parametrize("plan", [None, (64, 1, 1), (64, 2, 1), (32, 1, 1), (64, 1, 3)],
                         ids=["library", "64", "64x2cols", "32", "64split3"])
def test_closed_forms(cw, oracle, bf16, plan):
    """Results fixed by the mathematics, not by the oracle:
    * V = 1 everywhere: every output is sum(round16(p)) / (sum(p) + 1e-6),
      within one 16-bit rounding of the weights (2^-9 relative in bf16,
      2^-11 in fp16) of 1;
    * K = 0: every score is 0, every weight exp2(0) = 1 exactly, so each
      output row is the mean over the keys of the rounded V the kernel
      sees, accumulated in fp32 (the reference's 1/(l + 1e-6) included)."""
    b, nl, ni = 2, 80, 200
    q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=43)
    run = (lambda q, k, v: _run(cw, q, k, v, bf16)) if plan is None else \
        (lambda q, k, v: _run_plan(cw, q, k, v, bf16, *plan))
    out = run(q, k, np.ones_like(v))
    assert np.all(np.isfinite(out))
    assert np.max(np.abs(out - 1.0)) <= (2.0 ** -8 if bf16 else 2.0 ** -10)
    out = run(q, np.zeros_like(k), v)
    vr = oracle.round_bf16(v) if bf16 else oracle.round_fp16(v).astype(np.float32)
    mean = vr.astype(np.float64).sum(axis=1, keepdims=True) / (ni + 1e-6)
    assert np.max(np.abs(out - mean)) <= 1e-5


@pytest.mark.parametrize("bf16", [False, True], ids=["fp16", "bf16"])
def test_empty_keys(cw, oracle, bf16):
    q, _, _ = oracle.make_inputs(1, 20, 1, 768, seed=1)
    k = np.zeros((1, 0, 768), np.float32)
    assert np.all(_run(cw, q, k, k, bf16) == 0)


@pytest.mark.parametrize("bf16", [False, True], ids=["fp16", "bf16"])
@pytest.mark.parametrize("s", [1, 4, 9, 35, 64])
def test_splitk_partials(cw, oracle, bf16, s):
    b, nl, ni = 2, 48, 500
    q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=s)
    out, (po, pm, pl) = cw.wmma_splitk_partials(q, k, v, b, nl, ni, 768, s, bf16=bf16)
    _check(oracle, cw, out, q, k, v, bf16)
    # partials on the rounded inputs, chunk rounded up to 16 keys
    qh, kh, vh = cw._half_inputs(q, k, v, b, 768, bf16)
    f = oracle.bf16_bits_to_f32 if bf16 else (lambda a: a.astype(np.float32))
    rpo, rpm, rpl = oracle.splitk_partials(f(qh).astype(np.float64) * math.sqrt(768), f(kh),
                                           f(vh), s, align=16)
    live = rpm > -oracle.FLT_MAX
    assert np.all(pm[~live] == -oracle.FLT_MAX) and np.all(pl[~live] == 0)
    assert np.all(po[~live] == 0)
    assert np.max(np.abs(pm[live] - rpm[live])) < 1e-3  # scores are q.k with Q pre-scaled
    assert np.max(np.abs(pl[live] / rpl[live] - 1)) < TIGHT[bf16]
    rel = oracle.rel_err(po[live] / pl[live][:, None], rpo[live] / rpl[live][:, None])
    assert rel < TIGHT[bf16]


@pytest.mark.parametrize("bf16", [False, True], ids=["fp16", "bf16"])
def test_splitk_long_input(cw, oracle, bf16):
    cu, _ = cw.device_info()
    q, k, v = oracle.make_inputs(1, 256, 16384, 768, seed=2, q_std=0.02)
    fn = cw.benchmark_wmma_splitk_bf16_events if bf16 else cw.benchmark_wmma_splitk_events
    out, _, _, s = fn(q, k, v, 1, 256, 16384, 768, warmup=1, iters=1, sm_count=cu)
    assert s > 1
    _check(oracle, cw, out, q, k, v, bf16)


@pytest.mark.parametrize("bf16", [False, True], ids=["fp16", "bf16"])
def test_growing_scores_force_restarts(cw, oracle, bf16):
    """Scores rise by ~0.43 per key (~124 in exp2 units over the row), far past
    the reference the weights are taken against.  launch_wmma_kernel splits
    these 200 keys over workgroups at this shape, so the inputs also run
    through the split-K entry with one split: one workgroup walks all seven
    tiles and, in key order, restarts its pass (twice for fp16, whose weights
    are bounded by 2^15)."""
    rng = np.random.RandomState(8)
    nl, ni = 40, 200
    u = rng.randn(768)
    u /= np.linalg.norm(u)
    q = (u * np.sqrt(768.0) * (1.0 + 0.01 * rng.randn(nl, 1))
         + 0.1 * rng.randn(nl, 768))[None].astype(np.float32)
    k = (np.arange(ni)[:, None] * (12.0 / np.sqrt(768.0)) * u
         + 0.05 * rng.randn(ni, 768))[None].astype(np.float32)
    v = rng.randn(1, ni, 768).astype(np.float32)
    for perm in (rng.permutation(ni), np.arange(ni)):
        kp, vp = k[:, perm], v[:, perm]
        ref = _rounded_ref(oracle, cw, q, kp, vp, bf16)
        out = _run(cw, q, kp, vp, bf16)
        tight = oracle.rel_err(out, ref)
        assert np.all(np.isfinite(out)) and tight <= 2 * TIGHT[bf16], tight
        one, _ = cw.wmma_splitk_partials(q, kp, vp, 1, nl, ni, 768, 1, bf16=bf16)
        tight = oracle.rel_err(one, ref)
        assert np.all(np.isfinite(one)) and tight <= 2 * TIGHT[bf16], tight


@pytest.mark.parametrize("bf16", [False, True], ids=["fp16", "bf16"])
@pytest.mark.parametrize("lpw,cp", [(64, 1), (64, 2), (32, 1)], ids=["64", "64x2cols", "32"])
def test_restarts_in_every_form(cw, oracle, bf16, lpw, cp):
    """The growing-scores problem above (keys in rising order, so every
    workgroup restarts its pass) through each workgroup form, unsplit and
    in two splits, via launch_wmma_plan_kernel."""
    rng = np.random.RandomState(8)
    nl, ni = 40, 200
    u = rng.randn(768)
    u /= np.linalg.norm(u)
    q = (u * np.sqrt(768.0) * (1.0 + 0.01 * rng.randn(nl, 1))
         + 0.1 * rng.randn(nl, 768))[None].astype(np.float32)
    k = (np.arange(ni)[:, None] * (12.0 / np.sqrt(768.0)) * u
         + 0.05 * rng.randn(ni, 768))[None].astype(np.float32)
    v = rng.randn(1, ni, 768).astype(np.float32)
    ref = _rounded_ref(oracle, cw, q, k, v, bf16)
    for s in (1, 2):
        out = _run_plan(cw, q, k, v, bf16, lpw, cp, s)
        tight = oracle.rel_err(out, ref)
        assert np.all(np.isfinite(out)) and tight <= 2 * TIGHT[bf16], (s, tight)


@pytest.mark.parametrize("bf16", [False, True], ids=["fp16", "bf16"])
def test_wide_workgroups_split_and_restart(cw, oracle, bf16):
    """Split-K partials and pass restarts on 64-latent workgroups: 64 copies
    of an 80-latent, 400-key problem whose scores rise by ~0.62 per key in
    exp2 units, keys in rising order, in two splits (208 and 192 keys).
    64 x 2 row blocks x 2 splits fill 256 CUs once with 64-latent workgroups
    (32-latent ones would need two rounds), so the split-K entry takes the
    8-wavefront kernel; each split spans over 118 exp2 units, past both
    types' restart bound."""
    rng = np.random.RandomState(9)
    b, nl, ni = 64, 80, 400
    u = rng.randn(768)
    u /= np.linalg.norm(u)
    q = (u * np.sqrt(768.0) * (1.0 + 0.01 * rng.randn(nl, 1))
         + 0.1 * rng.randn(nl, 768))[None].astype(np.float32)
    k = (np.arange(ni)[:, None] * (12.0 / np.sqrt(768.0)) * u
         + 0.05 * rng.randn(ni, 768))[None].astype(np.float32)
    v = rng.randn(1, ni, 768).astype(np.float32)
    ref = np.repeat(_rounded_ref(oracle, cw, q, k, v, bf16), b, axis=0)
    qb, kb, vb = (np.repeat(a, b, axis=0) for a in (q, k, v))
    cu, _ = cw.device_info()
    if cu == 256:
        assert cw.lib.xattn_wmma_split_latents(b, nl, ni, 2, cu) == 64
    out, (po, pm, pl) = cw.wmma_splitk_partials(qb, kb, vb, b, nl, ni, 768, 2, bf16=bf16)
    tight = oracle.rel_err(out, ref)
    assert np.all(np.isfinite(out)) and tight <= 2 * TIGHT[bf16], tight
    # both splits are live and every batch copy holds the same partials
    assert np.all(pm > -oracle.FLT_MAX) and np.all(pl > 0)
    pm = pm.reshape(b, nl, 2)
    assert np.array_equal(pm, np.broadcast_to(pm[:1], pm.shape))


@pytest.mark.parametrize("bf16", [False, True], ids=["fp16", "bf16"])
def test_nan_stays_where_the_reference_puts_it(cw, oracle, bf16):
    """As the fp32 test of the same name: a NaN in one batch element's K
    (whole output of that element NaN) or V (one column NaN), through the
    16-bit planned launch (B=3 N_latent=64 N_input=100: a split plan); every
    other value within the 16-bit gate."""
    b, nl, ni = 3, 64, 100
    for where in ("K", "V"):
        q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=78)
        (k if where == "K" else v)[1, 37, 5] = np.nan
        ref = oracle.attention_f64(q, k, v)
        nan = np.isnan(ref)
        assert nan[1].any() and not nan[[0, 2]].any()
        out = _run(cw, q, k, v, bf16)
        assert np.array_equal(np.isnan(out), nan), f"NaN in {where}: NaN pattern"
        rel = oracle.rel_err(np.where(nan, 0.0, out), np.where(nan, 0.0, ref))
        assert rel <= GATE, f"NaN in {where}: rel {rel:.3e}"
