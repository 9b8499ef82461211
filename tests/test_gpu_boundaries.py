"""Shapes on every tile and workgroup boundary of the launch plans: N_latent
around the 16-, 32- and 64-latent workgroup sizes and N_input around the 16-
and 32-key tiles (a partial last tile is shifted back and masked), for the
fp32 entry point and both 16-bit ones, each against the float64 oracle.  The
plans pick plain or split launches by shape, so the grid reaches both."""

import math

import numpy as np
import pytest

from conftest import fp32_gate, gate16

pytestmark = pytest.mark.gpu

NLS = [1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 129]
NIS = [1, 2, 15, 16, 17, 31, 32, 33, 47, 785]


def _grid(b):
    return [(b, nl, ni) for nl in NLS for ni in NIS]


@pytest.mark.parametrize("b", [1, 3])
def test_fp32_boundaries(cw, oracle, b):
    bad = []
    for _, nl, ni in _grid(b):
        q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=1000 * nl + ni + b)
        ref = oracle.attention_f64(q, k, v)
        out, _, _ = cw.benchmark_kernel_events("vectorized", q, k, v, b, nl, ni, 768,
                                               warmup=0, iters=1)
        try:
            fp32_gate(out, ref)
        except AssertionError as e:
            bad.append(f"B={b} NL={nl} NI={ni}: {e}")
    assert not bad, "\n".join(bad)


@pytest.mark.parametrize("bf16", [False, True], ids=["fp16", "bf16"])
@pytest.mark.parametrize("b", [1, 3])
def test_16bit_boundaries(cw, oracle, b, bf16):
    f = oracle.bf16_bits_to_f32 if bf16 else (lambda a: a.astype(np.float32))
    run = cw.benchmark_wmma_bf16_events if bf16 else cw.benchmark_wmma_events
    bad = []
    for _, nl, ni in _grid(b):
        q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=1000 * nl + ni + b + 7)
        qh, kh, vh = cw._half_inputs(q, k, v, b, 768, bf16)
        ref = oracle.attention_f64(f(qh).astype(np.float64) * math.sqrt(768), f(kh), f(vh))
        out, _, _ = run(q, k, v, b, nl, ni, 768, warmup=0, iters=1)
        try:
            gate16(out, oracle.attention_f64(q, k, v), ref, bf16)
        except AssertionError as e:
            bad.append(f"B={b} NL={nl} NI={ni}: {e}")
    assert not bad, "\n".join(bad)
