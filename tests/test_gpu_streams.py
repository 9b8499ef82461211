"""The library's internal split workspace under concurrent streams: shapes
that launch_optimized_kernel and launch_wmma_bf16_kernel split over the keys
(partials in the one per-device workspace) are launched alternately on two
streams with different inputs.  Each split launch on the other stream waits
for the previous one's merge, so both outputs must match the reference
exactly as when run alone."""

import ctypes

import numpy as np
import pytest

from conftest import fp32_gate

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p


def _hip(cw):
    hip = cw._load_hip()
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(P)]
    hip.hipStreamCreate.restype = ctypes.c_int
    hip.hipStreamDestroy.argtypes = [P]
    hip.hipStreamDestroy.restype = ctypes.c_int
    return hip


@pytest.mark.parametrize("entry", ["launch_optimized_kernel", "launch_wmma_bf16_kernel"])
def test_split_launches_on_two_streams(cw, oracle, entry):
    b, nl, ni, d = 1, 64, 784, 768
    cu, _ = cw.device_info()
    if entry == "launch_optimized_kernel":
        assert cw.f32_plan(b, nl, ni, cu)[1] > 1  # the shape splits
    else:
        assert cw.wmma_plan(b, nl, ni, cu)[1] > 1
    hip = _hip(cw)
    streams = [P(), P()]
    for s in streams:
        assert hip.hipStreamCreate(ctypes.byref(s)) == 0
    bufs, outs, refs = [], [], []
    try:
        for i in range(2):
            q, k, v = oracle.make_inputs(b, nl, ni, d, seed=100 + i)
            if entry == "launch_optimized_kernel":
                ins = [cw.DeviceBuffer.holding(a) for a in (q, k, v)]
                args = [p.f32 for p in ins]
                refs.append(oracle.attention_f64(q, k, v))
            else:
                host = cw._half_inputs(q, k, v, b, d, bf16=True)
                ins = [cw.DeviceBuffer.holding(a) for a in host]
                args = [p.ptr for p in ins]
                f = oracle.bf16_bits_to_f32
                refs.append(oracle.attention_f64(
                    f(host[0]).astype(np.float64) * np.sqrt(d), f(host[1]), f(host[2])))
            out = cw.DeviceBuffer(b * nl * d * 4)
            bufs += ins + [out]
            outs.append((args, out))
        fn = getattr(cw.lib, entry)
        for _ in range(40):
            for (args, out), s in zip(outs, streams):
                fn(*args, out.f32, b, nl, ni, d, s)
        cw._lib_error_check(entry)
        assert cw.cudart.cudaDeviceSynchronize() == 0
        for (args, out), ref in zip(outs, refs):
            got = out.download((b, nl, d))
            if entry == "launch_optimized_kernel":
                fp32_gate(got, ref)
            else:
                assert oracle.rel_err(got, ref) < 4e-3
    finally:
        assert cw.cudart.cudaDeviceSynchronize() == 0
        for p in bufs:
            p.close()
        for s in streams:
            hip.hipStreamDestroy(s)
