"""Seeded random shapes through every launch plan: the fp32, fp16 and bf16
entry points choose their workgroup size (64 / 32 / 16 latents) and key
splits from the shape, and the split-K entry points their workgroup size from the
caller's num_splits, so random (B, N_latent, N_input, num_splits) draws reach
plans the fixed-shape tests do not.  Each output is checked against the
float64 oracle: the fp32 gate, or for 16-bit both gates of conftest.gate16
(2e-2 relative against the unrounded inputs, twice the kernel's own 1e-3 /
4e-3 bound against the oracle on the rounded inputs)."""

import math

import numpy as np
import pytest

from conftest import TIGHT16, fp32_gate, gate16

pytestmark = pytest.mark.gpu


def _shapes(seed, n):
    rng = np.random.RandomState(seed)
    out = []
    while len(out) < n:
        b = int(rng.randint(1, 9))
        nl = int(rng.randint(1, 400))
        ni = int(rng.randint(1, 3000))
        if b * nl * ni <= 400_000:  # keeps the float64 oracle to a fraction of a second
            out.append((b, nl, ni, int(rng.randint(1, 65))))
    return out


SHAPES = _shapes(20261201, 16)


@pytest.mark.parametrize("b,nl,ni,s", SHAPES)
def test_fp32_plans(cw, oracle, b, nl, ni, s):
    q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=b * 7919 + nl * 31 + ni)
    ref = oracle.attention_f64(q, k, v)
    out, _, _ = cw.benchmark_kernel_events("vectorized", q, k, v, b, nl, ni, 768, warmup=0,
                                           iters=1)
    fp32_gate(out, ref)
    out, _ = cw.splitk_partials(q, k, v, b, nl, ni, 768, min(s, ni))
    fp32_gate(out, ref)


@pytest.mark.parametrize("bf16", [False, True], ids=["fp16", "bf16"])
@pytest.mark.parametrize("b,nl,ni,s", SHAPES)
def test_16bit_plans(cw, oracle, b, nl, ni, s, bf16):
    q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=b * 7919 + nl * 31 + ni + 1)
    qh, kh, vh = cw._half_inputs(q, k, v, b, 768, bf16)
    f = oracle.bf16_bits_to_f32 if bf16 else (lambda a: a.astype(np.float32))
    ref = oracle.attention_f64(f(qh).astype(np.float64) * math.sqrt(768), f(kh), f(vh))
    run = cw.benchmark_wmma_bf16_events if bf16 else cw.benchmark_wmma_events
    ref32 = oracle.attention_f64(q, k, v)
    out, _, _ = run(q, k, v, b, nl, ni, 768, warmup=0, iters=1)
    gate16(out, ref32, ref, bf16)
    out, _ = cw.wmma_splitk_partials(q, k, v, b, nl, ni, 768, min(s, ni), bf16=bf16)
    gate16(out, ref32, ref, bf16)


@pytest.mark.parametrize("i", range(8))
def test_every_plan_form(cw, oracle, i):
    """Every workgroup form of both paths (fp32: 64, 32, 16 latents; 16-bit:
    64 latents in one or two column parts, 32 latents) under a random split
    count from 1 to the number of key tiles -- counts that leave trailing
    splits empty included -- through the plan-override entry points, at the
    random shapes above."""
    b, nl, ni, _ = SHAPES[i]
    rng = np.random.RandomState(1000 + i)
    q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=b * 7919 + nl * 31 + ni + 2)
    ref = oracle.attention_f64(q, k, v)
    for lpw in (64, 32, 16):
        s = int(rng.randint(1, -(-ni // 16) + 1))
        out, _, _ = cw.benchmark_plan_events(q, k, v, b, nl, ni, 768, lpw, s, warmup=0,
                                             iters=1)
        fp32_gate(out, ref)
    precision = "bf16" if i % 2 else "fp16"
    qh, kh, vh = cw._half_inputs(q, k, v, b, 768, precision == "bf16")
    f = oracle.bf16_bits_to_f32 if precision == "bf16" else (lambda a: a.astype(np.float32))
    ref16 = oracle.attention_f64(f(qh).astype(np.float64) * math.sqrt(768), f(kh), f(vh))
    for lpw, cp in ((64, 1), (64, 2), (32, 1)):
        s = int(rng.randint(1, -(-ni // 32) + 1))
        out, _, _ = cw.benchmark_plan_events(q, k, v, b, nl, ni, 768, lpw, s, cp, precision,
                                             warmup=0, iters=1)
        try:
            gate16(out, ref, ref16, precision == "bf16")
        except AssertionError as e:
            raise AssertionError(f"plan {lpw}/{cp}/{s}: {e}") from None


@pytest.mark.parametrize("i", range(6))
def test_scaled_scores_every_plan_form(cw, oracle, i):
    """Large-magnitude scores (Q scaled by 8 or 16: scaled scores span up to
    about 70, so 16-bit rows outgrow the first tile's reference by more than
    the fp16 bound of 2^15 and their passes restart) at seeded ragged shapes,
    through every workgroup form of both paths under a random split count;
    16-bit outputs are held to the kernel's own bound against the oracle on
    the rounded inputs (the unrounded-input contract assumes unit-scale
    scores)."""
    rng = np.random.RandomState(4242 + i)
    b = int(rng.randint(1, 5))
    nl = int(rng.choice([1, 17, 33, 65, 100]))
    ni = int(rng.choice([17, 49, 200, 785, 1569]))
    scale = (8.0, 16.0)[i % 2]
    q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=9000 + i)
    q = (q * scale).astype(np.float32)
    ref = oracle.attention_f64(q, k, v)
    for lpw in (64, 32, 16):
        s = int(rng.randint(1, -(-ni // 16) + 1))
        out, _, _ = cw.benchmark_plan_events(q, k, v, b, nl, ni, 768, lpw, s, warmup=0,
                                             iters=1)
        try:
            fp32_gate(out, ref)
        except AssertionError as e:
            raise AssertionError(f"fp32 plan {lpw}/{s}: {e}") from None
    for precision in ("fp16", "bf16"):
        bf16 = precision == "bf16"
        qh, kh, vh = cw._half_inputs(q, k, v, b, 768, bf16)
        f = oracle.bf16_bits_to_f32 if bf16 else (lambda a: a.astype(np.float32))
        ref16 = oracle.attention_f64(f(qh).astype(np.float64) * math.sqrt(768), f(kh), f(vh))
        for lpw, cp in ((64, 1), (64, 2), (32, 1)):
            s = int(rng.randint(1, -(-ni // 32) + 1))
            out, _, _ = cw.benchmark_plan_events(q, k, v, b, nl, ni, 768, lpw, s, cp, precision,
                                                 warmup=0, iters=1)
            rel = oracle.rel_err(out, ref16)
            assert np.all(np.isfinite(out)) and rel <= 2 * TIGHT16[bf16], \
                f"{precision} plan {lpw}/{cp}/{s}: rel vs rounded-input oracle {rel:.3e}"
