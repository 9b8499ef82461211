"""Pins the CPU oracle (oracle/xattn_oracle.py) without retyping its formulas.

Each check compares the oracle with something computed a different way: a
pure-Python brute force, a library routine (scipy softmax, torch SDPA, torch's
bfloat16 cast, numpy's float16 cast), a closed-form special case, or an
invariant the mathematics fixes.  ``test_planted_mistakes_are_caught`` plants
plausible bugs in copies of the oracle and checks the same battery fails.
"""

import math
import os

import numpy as np
import pytest
import scipy.special

import xattn_oracle as o

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _rand(b, nl, ni, d, seed):
    return o.make_inputs(b, nl, ni, d, seed=seed)


# ---------------------------------------------------------------------------
# Battery of independent checks, parameterised by the attention function so it
# can also be run against planted mistakes.
# ---------------------------------------------------------------------------

def _check_bruteforce(fn):
    g = np.load(os.path.join(GOLDEN, "tiny_bruteforce.npz"))
    ok = np.allclose(fn(g["q"], g["k"], g["v"]), g["out"], atol=1e-10, rtol=1e-9)
    ok &= np.allclose(fn(g["q768"], g["k768"], g["v768"]), g["out768"], atol=1e-10, rtol=1e-9)
    return ok


def _check_scipy(fn):
    q, k, v = _rand(2, 7, 19, 48, 11)
    s = np.einsum("bid,bjd->bij", q.astype(np.float64), k.astype(np.float64)) / math.sqrt(48)
    ref = np.einsum("bij,bjd->bid", scipy.special.softmax(s, axis=-1), v.astype(np.float64))
    return np.allclose(fn(q, k, v), ref, atol=1e-10, rtol=1e-9)


def _check_special_cases(fn):
    rng = np.random.RandomState(5)
    q = rng.randn(2, 4, 32).astype(np.float32)
    k = rng.randn(2, 9, 32).astype(np.float32)
    ok = True
    # V constant per column -> O equals that row
    row = rng.randn(32)
    v = np.broadcast_to(row, (2, 9, 32)).astype(np.float32)
    ok &= np.allclose(fn(q, k, v), np.broadcast_to(row.astype(np.float32), (2, 4, 32)),
                      atol=1e-6)
    # K = 0 -> uniform weights -> mean of V rows
    v = rng.randn(2, 9, 32).astype(np.float32)
    ok &= np.allclose(fn(q, np.zeros_like(k), v),
                      np.broadcast_to(v.astype(np.float64).mean(axis=1, keepdims=True),
                                      (2, 4, 32)), atol=1e-9)
    # NI = 1 -> O = V[0]
    ok &= np.allclose(fn(q, k[:, :1], v[:, :1]), np.broadcast_to(v[:, :1], (2, 4, 32)),
                      atol=1e-9)
    # Q_i = c * K_j with large c -> weight concentrates on j
    qq = (40.0 * k[:, [3, 0, 8, 5]]).astype(np.float32)
    ok &= np.allclose(fn(qq, k, v), v[:, [3, 0, 8, 5]], atol=1e-4)
    # asymmetry check: the result must depend on which side is Q
    ok &= not np.allclose(fn(q, k, v), fn(k[:, :4], q, v[:, :4]), atol=1e-3)
    return bool(ok)


def _check_invariants(fn):
    rng = np.random.RandomState(9)
    q = rng.randn(3, 5, 24).astype(np.float32)
    k = rng.randn(3, 11, 24).astype(np.float32)
    v = rng.randn(3, 11, 24).astype(np.float32)
    base = fn(q, k, v)
    ok = True
    perm = rng.permutation(11)
    ok &= np.allclose(fn(q, k[:, perm], v[:, perm]), base, atol=1e-10)
    v2 = rng.randn(3, 11, 24)
    ok &= np.allclose(fn(q, k, 2.0 * v.astype(np.float64) + v2), 2.0 * base + fn(q, k, v2),
                      atol=1e-9)
    ok &= np.allclose(fn(q[1:2], k[1:2], v[1:2]), base[1:2], atol=1e-12)
    return bool(ok)


BATTERY = (_check_bruteforce, _check_scipy, _check_special_cases, _check_invariants)


@pytest.mark.parametrize("check", BATTERY, ids=lambda f: f.__name__)
def test_attention_f64_pinned(check):
    assert check(o.attention_f64)


def test_online_softmax_equals_two_pass():
    for ni in (1, 15, 16, 17, 33):
        q, k, v = _rand(2, 6, ni, 64, ni)
        ref = o.attention_f64(q, k, v)
        for tile in (1, 4, 16):
            got = o.online_softmax_f64(q, k, v, tile=tile, eps=0.0)
            assert np.allclose(got, ref, atol=1e-12), (ni, tile)
        # the reference's 1e-6 in the denominator moves the result by <= 1e-6 rel
        got = o.online_softmax_f64(q, k, v, tile=16)
        assert np.max(np.abs(got - ref)) <= 1e-6 * np.max(np.abs(ref)) + 1e-12


def test_online_softmax_battery():
    fn = lambda q, k, v: o.online_softmax_f64(q, k, v, tile=16, eps=0.0)  # noqa: E731
    for check in BATTERY:
        assert check(fn), check.__name__


def test_float32_restatements_match_f64():
    q, k, v = o.make_inputs(1, 64, 784, 768, seed=0)
    ref = o.attention_f64(q, k, v)
    for fn in (o.attention_torch_f32, o.attention_numpy_f32, o.sdpa_cpu):
        got = fn(q, k, v)
        assert got.dtype == np.float32
        assert o.max_abs(got, ref) < 2e-6, fn.__name__


def test_generators():
    g = np.load(os.path.join(GOLDEN, "cfg1_seed0.npz"))
    q, k, v = o.make_inputs(1, 64, 784, 768, seed=0)
    from make_golden import checksums
    assert np.allclose(checksums(q, k, v), g["checksums"], rtol=0, atol=0)
    assert np.allclose(o.attention_f64(q, k, v), g["out"], atol=1e-6)
    g = np.load(os.path.join(GOLDEN, "legacy_seed42_nl64.npz"))
    q, k, v = o.make_inputs_legacy(1, 64, 784, 768, seed=42)
    assert np.allclose(checksums(q, k, v), g["checksums"], rtol=0, atol=0)
    assert np.allclose(o.attention_f64(q, k, v), g["out"], atol=1e-6)
    # legacy draw order: Q first, then K, then V from one seeded stream
    np.random.seed(42)
    assert np.array_equal(q[0], np.random.randn(64, 768).astype(np.float32))
    # q_std scales Q only
    q2, k2, v2 = o.make_inputs(1, 4, 8, 16, seed=1, q_std=0.02)
    q1, k1, v1 = o.make_inputs(1, 4, 8, 16, seed=1)
    assert np.allclose(q2, q1 * np.float32(0.02)) and np.array_equal(k1, k2)
    assert np.array_equal(v1, v2)


# ---------------------------------------------------------------------------
# split-K
# ---------------------------------------------------------------------------

def test_splitk_bounds_partition():
    for ni in (1, 16, 33, 784, 4096):
        for s in (1, 2, 3, 7, 8, 35, 64, 300):
            for align in (1, 16):
                bounds, chunk = o.splitk_bounds(ni, s, align)
                covered = []
                for k0, k1 in bounds:
                    covered.extend(range(k0, k1))
                assert covered == list(range(ni)), (ni, s, align)
                assert chunk >= 1 and (align == 1 or chunk % align == 0)


def test_splitk_bounds_known_cases():
    # long-input fp16 split-K at NI=4096 with S=35: chunk rounds up to 128 and
    # splits 32..34 are empty (kernel_wmma_splitk.cu:52-54)
    bounds, chunk = o.splitk_bounds(4096, 35, align=16)
    assert chunk == 128
    assert [s for s, (a, b) in enumerate(bounds) if b <= a] == [32, 33, 34]
    # fp32 split-K: chunk = ceil(NI/S) with no rounding (kernel_splitk.cu:59)
    bounds, chunk = o.splitk_bounds(33, 8)
    assert chunk == 5 and bounds[6] == (30, 33) and bounds[7][1] <= bounds[7][0]


@pytest.mark.parametrize("ni,s,align", [(37, 8, 1), (37, 1, 1), (50, 7, 16), (16, 5, 1),
                                        (100, 13, 1)])
def test_splitk_merge_equals_unsplit(ni, s, align):
    q, k, v = _rand(2, 5, ni, 32, ni + s)
    po, pm, pl = o.splitk_partials(q, k, v, s, align)
    got = o.splitk_combine(po, pm, pl, eps=0.0)
    assert np.allclose(got, o.attention_f64(q, k, v), atol=1e-12)
    bounds, _ = o.splitk_bounds(ni, s, align)
    for j, (k0, k1) in enumerate(bounds):
        if k1 <= k0:  # empty split sentinel
            assert np.all(pm[..., j] == -o.FLT_MAX) and np.all(pl[..., j] == 0)
            assert np.all(po[..., j, :] == 0)
        else:  # per-split max is the max score of that key range
            sc = np.einsum("bid,bjd->bij", q.astype(np.float64),
                           k[:, k0:k1].astype(np.float64)) / math.sqrt(32)
            assert np.allclose(pm[..., j], sc.max(-1), atol=1e-12)
            assert np.all(pl[..., j] >= 1.0 - 1e-12)  # the max key contributes exp(0)
    # order independence of the merge
    perm = np.random.RandomState(0).permutation(s)
    got2 = o.splitk_combine(po[..., perm, :], pm[..., perm], pl[..., perm], eps=0.0)
    assert np.allclose(got2, got, atol=1e-12)


def test_splitk_single_split_identity():
    q, k, v = _rand(1, 4, 21, 16, 2)
    po, pm, pl = o.splitk_partials(q, k, v, 1)
    assert np.allclose(po[:, :, 0] / pl[:, :, 0, None], o.attention_f64(q, k, v), atol=1e-12)


def test_splitk_golden():
    g = np.load(os.path.join(GOLDEN, "splitk_small.npz"))
    b, nl, ni, d, s = [int(x) for x in g["shape"]]
    q, k, v = o.make_inputs(b, nl, ni, d, seed=3)
    po, pm, pl = o.splitk_partials(q, k, v, s)
    assert np.allclose(po, g["po"], atol=1e-5) and np.allclose(pm, g["pm"], atol=1e-12)
    assert np.allclose(pl, g["pl"], atol=1e-12)
    assert np.allclose(o.splitk_combine(po, pm, pl), g["out"], atol=1e-6)
    assert np.allclose(g["out"], o.attention_f64(q, k, v), atol=1e-5)


# ---------------------------------------------------------------------------
# reduced precision
# ---------------------------------------------------------------------------

def test_bf16_rounding_matches_torch():
    import torch
    rng = np.random.RandomState(0)
    x = np.concatenate([rng.randn(100000).astype(np.float32) * 10.0 ** rng.randint(-8, 8, 100000),
                        np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-40],
                                 np.float32)]).astype(np.float32)
    ours = o.round_bf16(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))
    # ties go to even: 1 + 2^-8 -> 1, 1 + 3*2^-8 -> 1 + 2^-6
    ties = np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8], np.float32)
    assert list(o.round_bf16(ties)) == [1.0, 1 + 2 ** -6]
    assert np.isnan(o.round_bf16(np.array([np.nan], np.float32)))[0]


def test_fp16_rounding_is_ieee():
    x = np.array([1 + 2 ** -11, 1 + 3 * 2 ** -11, 65520.0, 1e-8], np.float32)
    got = o.round_fp16(x).astype(np.float32)
    assert list(got[:2]) == [1.0, 1 + 2 ** -9]
    assert np.isinf(got[2]) and got[3] == np.float32(np.float16(1e-8))


def test_reduced_precision_headroom():
    """Rounding Q/K/V alone (B=2 NL=128 NI=784) stays well inside the 2e-2 gate."""
    q, k, v = o.make_inputs(2, 128, 784, 768, seed=5)
    ref = o.attention_f64(q, k, v)
    qs = o.prescale_q_f16(q).astype(np.float32) * np.float32(math.sqrt(768))
    r16 = o.rel_err(o.attention_f64(qs, o.round_fp16(k), o.round_fp16(v)), ref)
    rb = o.rel_err(o.attention_f64(o.round_bf16(q), o.round_bf16(k), o.round_bf16(v)), ref)
    assert r16 < 2e-3 and rb < 1e-2, (r16, rb)


# ---------------------------------------------------------------------------
# planted mistakes: each must be caught by the battery
# ---------------------------------------------------------------------------

def _mut_no_scale(q, k, v):
    q = q.astype(np.float64); k = k.astype(np.float64); v = v.astype(np.float64)
    s = np.matmul(q, np.swapaxes(k, 1, 2))
    p = scipy.special.softmax(s, axis=-1)
    return np.matmul(p, v)


def _mut_wrong_axis(q, k, v):
    q = o._as3(q).astype(np.float64); k = o._as3(k).astype(np.float64)
    v = o._as3(v).astype(np.float64)
    s = np.matmul(q, np.swapaxes(k, 1, 2)) / math.sqrt(q.shape[-1])
    p = scipy.special.softmax(s, axis=-2)
    return np.matmul(p, v)


def _mut_k_read_transposed(q, k, v):
    # K's [N_input, D] rows read as if the buffer held K^T ([D, N_input]
    # row-major): the element at (j, d) is taken from flat index d * NI + j
    k = o._as3(k).astype(np.float64)
    b, ni, d = k.shape
    k_wrong = k.reshape(b, d, ni).swapaxes(1, 2)
    return o.attention_f64(q, k_wrong, v)


def _mut_dropped_max_term(q, k, v):
    # online softmax that forgets to rescale the accumulator when the max grows
    q = o._as3(q).astype(np.float64); k = o._as3(k).astype(np.float64)
    v = o._as3(v).astype(np.float64)
    b, nl, d = q.shape
    acc = np.zeros((b, nl, v.shape[-1])); m = np.full((b, nl, 1), -1e300)
    l = np.zeros((b, nl, 1))
    for t0 in range(0, k.shape[1], 2):
        s = np.matmul(q, np.swapaxes(k[:, t0:t0 + 2], 1, 2)) / math.sqrt(d)
        nm = np.maximum(m, s.max(-1, keepdims=True))
        l *= np.exp(m - nm)  # acc not rescaled
        e = np.exp(s - nm); l += e.sum(-1, keepdims=True); acc += np.matmul(e, v[:, t0:t0 + 2])
        m = nm
    return acc / l


def _mut_wrong_sqrt(q, k, v):
    q = o._as3(q).astype(np.float64)
    return o.attention_f64(q * math.sqrt(math.sqrt(q.shape[-1])) / q.shape[-1] ** 0.25 * 1.01,
                           k, v)


@pytest.mark.parametrize("mutant", [_mut_no_scale, _mut_wrong_axis, _mut_k_read_transposed,
                                    _mut_dropped_max_term, _mut_wrong_sqrt],
                         ids=lambda f: f.__name__)
def test_planted_mistakes_are_caught(mutant):
    results = []
    for check in BATTERY:
        try:
            results.append(bool(check(mutant)))
        except Exception:
            results.append(False)
    assert not all(results), f"{mutant.__name__} slipped through every check"


def test_planted_merge_mistakes_are_caught():
    q, k, v = _rand(1, 3, 40, 16, 1)
    po, pm, pl = o.splitk_partials(q, k, v, 4)
    ref = o.attention_f64(q, k, v)
    assert np.allclose(o.splitk_combine(po, pm, pl, eps=0.0), ref, atol=1e-12)
    # forgetting the exp(pm - M) weights must be visible
    bad1 = po.sum(-2) / pl.sum(-1)[..., None]
    assert not np.allclose(bad1, ref, atol=1e-6)
    # An empty split must carry the sentinel pm = -FLT_MAX: a partial writer
    # that leaves (0, 0, 0) there instead moves the merge's reference max to
    # 0.  With every real score far below 0 (all pm shifted by -1000, which
    # leaves the exact result unchanged) the real splits' weights then
    # underflow and the merge loses the output.
    po2, pm2, pl2 = o.splitk_partials(q, k, v, 64)  # splits 40..63 are empty
    empty = pm2 == -o.FLT_MAX
    assert empty.any() and (~empty).any()
    shifted = np.where(empty, pm2, pm2 - 1000.0)
    assert np.allclose(o.splitk_combine(po2, shifted, pl2, eps=0.0), ref, atol=1e-12)
    zero_sentinel = np.where(empty, 0.0, shifted)
    with np.errstate(divide="ignore", invalid="ignore"):
        bad2 = o.splitk_combine(po2, zero_sentinel, pl2, eps=0.0)
    assert not np.allclose(bad2, ref, atol=1e-6)
