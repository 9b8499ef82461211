"""Split launches on two streams at once.  launch_optimized_kernel and
launch_wmma_bf16_kernel keep split partials in a workspace per (device,
stream); here a small and a larger split shape are launched alternately on
two streams (and on the null stream), so each stream's workspace is grown
while the other stream's launches are in flight; and from four host threads
at once, each on its own stream.  Every output must match the float64
oracle as when run alone."""

import ctypes

import numpy as np
import pytest

from conftest import fp32_gate

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p
SHAPES = [(1, 64, 784), (1, 256, 4096), (2, 48, 1500)]


def _hip(cw):
    hip = cw._load_hip()
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(P)]
    hip.hipStreamCreate.restype = ctypes.c_int
    hip.hipStreamDestroy.argtypes = [P]
    hip.hipStreamDestroy.restype = ctypes.c_int
    return hip


@pytest.mark.parametrize("entry", ["launch_optimized_kernel", "launch_wmma_bf16_kernel"])
def test_split_launches_on_two_streams(cw, oracle, entry):
    cu, _ = cw.device_info()
    plan = cw.f32_plan if entry == "launch_optimized_kernel" else cw.wmma_plan
    for b, nl, ni in SHAPES:
        assert plan(b, nl, ni, cu)[1] > 1, (b, nl, ni)  # every shape splits
    hip = _hip(cw)
    streams = [P(), P(), P(0)]
    for s in streams[:2]:
        assert hip.hipStreamCreate(ctypes.byref(s)) == 0
    cases = []  # (shape, args, out, ref) per (stream, shape)
    try:
        for i in range(len(streams)):
            row = []
            for j, (b, nl, ni) in enumerate(SHAPES):
                q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=100 + 10 * i + j)
                if entry == "launch_optimized_kernel":
                    ins = [cw.DeviceBuffer.holding(a) for a in (q, k, v)]
                    args = [p.f32 for p in ins]
                    ref = oracle.attention_f64(q, k, v)
                else:
                    host = cw._half_inputs(q, k, v, b, 768, bf16=True)
                    ins = [cw.DeviceBuffer.holding(a) for a in host]
                    args = [p.ptr for p in ins]
                    f = oracle.bf16_bits_to_f32
                    ref = oracle.attention_f64(
                        f(host[0]).astype(np.float64) * np.sqrt(768), f(host[1]), f(host[2]))
                out = cw.DeviceBuffer(b * nl * 768 * 4).zero()
                row.append(((b, nl, ni), ins, args, out, ref))
            cases.append(row)
        fn = getattr(cw.lib, entry)
        for rep in range(12):
            for i, s in enumerate(streams):
                (b, nl, ni), _, args, out, _ = cases[i][(rep + i) % len(SHAPES)]
                fn(*args, out.f32, b, nl, ni, 768, s)
        cw._lib_error_check(entry)
        assert cw.cudart.hipDeviceSynchronize() == 0
        for row in cases:
            for (b, nl, ni), _, _, out, ref in row:
                got = out.download((b, nl, 768))
                if entry == "launch_optimized_kernel":
                    fp32_gate(got, ref)
                else:
                    assert oracle.rel_err(got, ref) < 4e-3, (b, nl, ni)
    finally:
        assert cw.cudart.hipDeviceSynchronize() == 0
        for row in cases:
            for _, ins, _, out, _ in row:
                for p in ins + [out]:
                    p.close()
        for s in streams[:2]:
            hip.hipStreamDestroy(s)


def test_host_threads_on_their_own_streams(cw, oracle):
    """Four host threads launch concurrently (ctypes releases the GIL during
    the call), each on its own created stream, alternating the split shapes
    above -- two threads through launch_optimized_kernel, two through
    launch_wmma_bf16_kernel -- so workspaces are created and grown from
    several threads at once.  Each thread reads its own error state; every
    output must match the float64 oracle."""
    import threading

    hip = _hip(cw)
    hip.hipStreamSynchronize.argtypes = [P]
    hip.hipStreamSynchronize.restype = ctypes.c_int
    entries = ["launch_optimized_kernel", "launch_optimized_kernel",
               "launch_wmma_bf16_kernel", "launch_wmma_bf16_kernel"]
    streams = [P() for _ in entries]
    for s in streams:
        assert hip.hipStreamCreate(ctypes.byref(s)) == 0
    cases = []  # per thread: (shape, ins, args, out, ref) per shape
    try:
        for t, entry in enumerate(entries):
            row = []
            for j, (b, nl, ni) in enumerate(SHAPES):
                q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=300 + 10 * t + j)
                if entry == "launch_optimized_kernel":
                    ins = [cw.DeviceBuffer.holding(a) for a in (q, k, v)]
                    args = [p.f32 for p in ins]
                    ref = oracle.attention_f64(q, k, v)
                else:
                    host = cw._half_inputs(q, k, v, b, 768, bf16=True)
                    ins = [cw.DeviceBuffer.holding(a) for a in host]
                    args = [p.ptr for p in ins]
                    f = oracle.bf16_bits_to_f32
                    ref = oracle.attention_f64(
                        f(host[0]).astype(np.float64) * np.sqrt(768), f(host[1]), f(host[2]))
                out = cw.DeviceBuffer(b * nl * 768 * 4).zero()
                row.append(((b, nl, ni), ins, args, out, ref))
            cases.append(row)
        failures = []

        def work(t):
            try:
                fn = getattr(cw.lib, entries[t])
                for rep in range(9):
                    (b, nl, ni), _, args, out, _ = cases[t][(rep + t) % len(SHAPES)]
                    fn(*args, out.f32, b, nl, ni, 768, streams[t])
                code = cw.lib.xattn_get_last_error()
                if code != 0:
                    failures.append((t, code, cw.lib.xattn_get_last_error_string()))
                if hip.hipStreamSynchronize(streams[t]) != 0:
                    failures.append((t, "stream"))
            except Exception as e:  # reported after the join
                failures.append((t, repr(e)))

        threads = [threading.Thread(target=work, args=(t,)) for t in range(len(entries))]
        for th in threads:
            th.start()
        for th in threads:
            th.join()
        assert not failures, failures
        assert cw.cudart.hipDeviceSynchronize() == 0
        for t, row in enumerate(cases):
            for (b, nl, ni), _, _, out, ref in row:
                got = out.download((b, nl, 768))
                if entries[t] == "launch_optimized_kernel":
                    fp32_gate(got, ref)
                else:
                    assert oracle.rel_err(got, ref) < 4e-3, (t, b, nl, ni)
    finally:
        assert cw.cudart.hipDeviceSynchronize() == 0
        for row in cases:
            for _, ins, _, out, _ in row:
                for p in ins + [out]:
                    p.close()
        for s in streams:
            hip.hipStreamDestroy(s)


def test_host_threads_on_the_per_thread_stream(cw, oracle):
    """Four host threads launch split shapes at once on hipStreamPerThread
    (handle 2), which names a different stream in every thread: two threads
    through launch_optimized_kernel, two through launch_wmma_bf16_kernel.
    The library keys that handle's workspace by thread as well, so no two
    threads share partials; every output must match the float64 oracle."""
    import threading

    hip = _hip(cw)
    hip.hipStreamSynchronize.argtypes = [P]
    hip.hipStreamSynchronize.restype = ctypes.c_int
    per_thread = P(2)
    entries = ["launch_optimized_kernel", "launch_optimized_kernel",
               "launch_wmma_bf16_kernel", "launch_wmma_bf16_kernel"]
    cases = []  # per thread, per repetition: (shape, ins, args, out, ref)
    try:
        for t, entry in enumerate(entries):
            row = []
            for rep in range(6):
                b, nl, ni = SHAPES[(rep + t) % len(SHAPES)]
                q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=500 + 10 * t + rep)
                if entry == "launch_optimized_kernel":
                    ins = [cw.DeviceBuffer.holding(a) for a in (q, k, v)]
                    args = [p.f32 for p in ins]
                    ref = oracle.attention_f64(q, k, v)
                else:
                    host = cw._half_inputs(q, k, v, b, 768, bf16=True)
                    ins = [cw.DeviceBuffer.holding(a) for a in host]
                    args = [p.ptr for p in ins]
                    f = oracle.bf16_bits_to_f32
                    ref = oracle.attention_f64(
                        f(host[0]).astype(np.float64) * np.sqrt(768), f(host[1]), f(host[2]))
                out = cw.DeviceBuffer(b * nl * 768 * 4).zero()
                row.append(((b, nl, ni), ins, args, out, ref))
            cases.append(row)
        failures = []

        def work(t):
            try:
                fn = getattr(cw.lib, entries[t])
                for (b, nl, ni), _, args, out, _ in cases[t]:
                    fn(*args, out.f32, b, nl, ni, 768, per_thread)
                code = cw.lib.xattn_get_last_error()
                if code != 0:
                    failures.append((t, code, cw.lib.xattn_get_last_error_string()))
                if hip.hipStreamSynchronize(per_thread) != 0:
                    failures.append((t, "per-thread stream"))
            except Exception as e:  # reported after the join
                failures.append((t, repr(e)))

        threads = [threading.Thread(target=work, args=(t,)) for t in range(len(entries))]
        for th in threads:
            th.start()
        for th in threads:
            th.join()
        assert not failures, failures
        assert cw.cudart.hipDeviceSynchronize() == 0
        for t, row in enumerate(cases):
            for (b, nl, ni), _, _, out, ref in row:
                got = out.download((b, nl, 768))
                if entries[t] == "launch_optimized_kernel":
                    fp32_gate(got, ref)
                else:
                    assert oracle.rel_err(got, ref) < 4e-3, (t, b, nl, ni)
    finally:
        assert cw.cudart.hipDeviceSynchronize() == 0
        for row in cases:
            for _, ins, _, out, _ in row:
                for p in ins + [out]:
                    p.close()
