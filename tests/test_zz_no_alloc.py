"""launch_optimized_kernel_noalloc through the C ABI: the same plan and
kernels as launch_optimized_kernel with the split partials in the library's
static scratch, so its output must equal launch_optimized_kernel's bit for
bit.  Two calls in a row, the second on a smaller input, both with key
splits (the second reuses the scratch the first left behind); then a shape
without splits; then a plan whose partials exceed the 64 MiB scratch, which
is refused before anything is launched."""

import ctypes

import numpy as np
import pytest

from conftest import fp32_gate

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20
XATTN_ERR_UNSUPPORTED = 2


def _run(cw, entry, q, k, v):
    b, nl, d = q.shape
    ni = k.shape[1]
    bufs = [cw.DeviceBuffer.holding(a) for a in (q, k, v)]
    out = cw.DeviceBuffer(b * nl * d * 4).zero()
    try:
        getattr(cw.lib, entry)(*(p.f32 for p in bufs), out.f32, b, nl, ni, d,
                               ctypes.c_void_p(0))
        cw._lib_error_check(entry)
        assert cw.cudart.hipDeviceSynchronize() == 0
        return out.download((b, nl, d))
    finally:
        for p in bufs + [out]:
            p.close()


@pytest.mark.parametrize("shapes", [[(1, 256, 4096), (1, 64, 784)],
                                    [(2, 100, 3000), (1, 48, 500)]],
                         ids=["cfg4-then-cfg1", "ragged"])
def test_noalloc_matches_optimized(cw, oracle, shapes):
    assert cw.HAS_NOALLOC
    cu, _ = cw.device_info()
    for i, (b, nl, ni) in enumerate(shapes):
        lpw, s = cw.f32_plan(b, nl, ni, cu)
        assert s > 1 and b * nl * s * (768 + 2) * 4 <= SCRATCH_BYTES, (b, nl, ni, s)
        q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=31 + i)
        got = _run(cw, "launch_optimized_kernel_noalloc", q, k, v)
        ref = _run(cw, "launch_optimized_kernel", q, k, v)
        assert np.array_equal(got, ref), (b, nl, ni)
        fp32_gate(got, oracle.attention_f64(q, k, v))


def test_noalloc_without_splits(cw, oracle):
    cu, _ = cw.device_info()
    b, nl, ni = 16, 1024, 784
    assert cw.f32_plan(b, nl, ni, cu)[1] == 1
    q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=7)
    got = _run(cw, "launch_optimized_kernel_noalloc", q, k, v)
    assert np.array_equal(got, _run(cw, "launch_optimized_kernel", q, k, v))
    rows = [0, 9, 15]
    fp32_gate(got[rows, :32], oracle.attention_f64(q[rows, :32], k[rows], v[rows]))


def test_noalloc_refuses_oversized_plan(cw):
    cu, _ = cw.device_info()
    b, nl, ni = 28, 1792, 50176
    lpw, s = cw.f32_plan(b, nl, ni, cu)
    need = b * nl * s * (768 + 2) * 4
    if s == 1 or need <= SCRATCH_BYTES:
        pytest.skip(f"the plan on this device ({lpw}, {s}) fits the scratch")
    null = ctypes.cast(ctypes.c_void_p(256), ctypes.POINTER(ctypes.c_float))
    assert cw.lib.xattn_get_last_error() == 0
    cw.lib.launch_optimized_kernel_noalloc(null, null, null, null, b, nl, ni, 768,
                                           ctypes.c_void_p(0))
    code = cw.lib.xattn_get_last_error()
    msg = cw.lib.xattn_get_last_error_string().decode()
    assert code == XATTN_ERR_UNSUPPORTED and "static scratch" in msg, (code, msg)
