"""launch_optimized_kernel_noalloc through the C ABI: the same plan and
kernels as launch_optimized_kernel with the split partials in the library's
static scratch, so its output must equal launch_optimized_kernel's bit for
bit.  Two calls in a row, the second on a smaller input, both with key
splits (the second reuses the scratch the first left behind); then a shape
without splits; then a plan whose partials exceed the 64 MiB scratch, which
is refused before anything is launched.  Overlapping split calls from two
streams and from two host threads, which the library orders on the GPU
through its event; and, in a fresh process, a first call under stream
capture (refused) and a capture after xattn_noalloc_prepare (replayed)."""

import ctypes
import os
import subprocess
import sys
import threading

import numpy as np
import pytest

from conftest import PKG, ROOT, fp32_gate

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


P = ctypes.c_void_p


def _hip(cw):
    h = cw._load_hip()
    for name, args in {"hipStreamCreate": [ctypes.POINTER(P)], "hipStreamDestroy": [P],
                       "hipStreamSynchronize": [P]}.items():
        getattr(h, name).argtypes = args
        getattr(h, name).restype = ctypes.c_int
    return h


class _Inputs:
    """One split shape's inputs on the device, the oracle and
    launch_optimized_kernel's output for them."""

    def __init__(self, cw, oracle, b, nl, ni, seed):
        self.shape = (b, nl, ni)
        q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=seed)
        self.oracle = oracle.attention_f64(q, k, v)
        self.ref = _run(cw, "launch_optimized_kernel", q, k, v)
        self.bufs = [cw.DeviceBuffer.holding(a) for a in (q, k, v)]

    def noalloc(self, cw, out, stream):
        b, nl, ni = self.shape
        cw.lib.launch_optimized_kernel_noalloc(*(p.f32 for p in self.bufs), out.f32, b, nl, ni,
                                               768, stream)

    def close(self):
        for p in self.bufs:
            p.close()


SPLIT_SHAPES = [(1, 64, 784), (1, 256, 4096), (2, 100, 3000)]


def test_noalloc_overlapping_calls_from_two_streams(cw, oracle):
    """Split calls enqueued on two streams with no host wait between them
    (two shapes per stream, six calls each, every call into its own output):
    each output must equal launch_optimized_kernel's bit for bit."""
    cu, _ = cw.device_info()
    h = _hip(cw)
    streams = [P(), P()]
    for st in streams:
        assert h.hipStreamCreate(ctypes.byref(st)) == 0
    cases = [_Inputs(cw, oracle, *sh, seed=60 + i) for i, sh in enumerate(SPLIT_SHAPES)]
    for c in cases:
        assert cw.f32_plan(*c.shape, cu)[1] > 1, c.shape
    outs = []  # (case, stream, output) per call, all cleared before the first call
    for rep in range(6):
        for i, st in enumerate(streams):
            c = cases[(rep + i) % len(cases)]
            b, nl, _ = c.shape
            outs.append((c, st, cw.DeviceBuffer(b * nl * 768 * 4).zero()))
    try:
        for c, st, out in outs:
            c.noalloc(cw, out, st)
        cw._lib_error_check("launch_optimized_kernel_noalloc")
        assert cw.cudart.hipDeviceSynchronize() == 0
        for c, _, out in outs:
            b, nl, _ = c.shape
            got = out.download((b, nl, 768))
            assert np.array_equal(got, c.ref), c.shape
        for c in cases:
            fp32_gate(c.ref, c.oracle)
    finally:
        assert cw.cudart.hipDeviceSynchronize() == 0
        for _, _, out in outs:
            out.close()
        for c in cases:
            c.close()
        for st in streams:
            h.hipStreamDestroy(st)


def test_noalloc_calls_from_two_host_threads(cw, oracle):
    """Two host threads, each on its own stream, make five split calls each
    at once (ctypes releases the GIL during a call), every call into its own
    output: each must equal launch_optimized_kernel's bit for bit."""
    h = _hip(cw)
    streams = [P(), P()]
    for st in streams:
        assert h.hipStreamCreate(ctypes.byref(st)) == 0
    cases = [_Inputs(cw, oracle, *sh, seed=70 + i) for i, sh in enumerate(SPLIT_SHAPES)]
    work = []  # per thread: (case, out) per call
    for t in range(2):
        row = []
        for rep in range(5):
            c = cases[(rep + t) % len(cases)]
            b, nl, _ = c.shape
            row.append((c, cw.DeviceBuffer(b * nl * 768 * 4).zero()))
        work.append(row)
    failures = []

    def run(t):
        try:
            for c, out in work[t]:
                c.noalloc(cw, out, streams[t])
            code = cw.lib.xattn_get_last_error()
            if code != 0:
                failures.append((t, code, cw.lib.xattn_get_last_error_string()))
            if h.hipStreamSynchronize(streams[t]) != 0:
                failures.append((t, "stream"))
        except Exception as e:  # reported after the join
            failures.append((t, repr(e)))

    try:
        threads = [threading.Thread(target=run, args=(t,)) for t in range(2)]
        for th in threads:
            th.start()
        for th in threads:
            th.join()
        assert not failures, failures
        assert cw.cudart.hipDeviceSynchronize() == 0
        for row in work:
            for c, out in row:
                b, nl, _ = c.shape
                assert np.array_equal(out.download((b, nl, 768)), c.ref), c.shape
    finally:
        assert cw.cudart.hipDeviceSynchronize() == 0
        for row in work:
            for _, out in row:
                out.close()
        for c in cases:
            c.close()
        for st in streams:
            h.hipStreamDestroy(st)


_CAPTURE_SCRIPT = r"""
import ctypes, sys
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[2])
import numpy as np
import cuda_wrappers as cw
import xattn_oracle as oracle
P = ctypes.c_void_p
h = cw._load_hip()
for name, args in {"hipStreamCreate": [ctypes.POINTER(P)], "hipStreamDestroy": [P],
                   "hipStreamSynchronize": [P], "hipStreamBeginCapture": [P, ctypes.c_int],
                   "hipStreamEndCapture": [P, ctypes.POINTER(P)],
                   "hipGraphInstantiate": [ctypes.POINTER(P), P, P, P, ctypes.c_size_t],
                   "hipGraphLaunch": [P, P], "hipGraphExecDestroy": [P], "hipGraphDestroy": [P],
                   "hipGraphGetNodes": [P, P, ctypes.POINTER(ctypes.c_size_t)]}.items():
    getattr(h, name).argtypes = args
    getattr(h, name).restype = ctypes.c_int
b, nl, ni = 1, 64, 784
q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=51)
bufs = [cw.DeviceBuffer.holding(a) for a in (q, k, v)]
out = cw.DeviceBuffer(b * nl * 768 * 4).zero()
st = P()
assert h.hipStreamCreate(ctypes.byref(st)) == 0

def call():
    cw.lib.launch_optimized_kernel_noalloc(*(x.f32 for x in bufs), out.f32, b, nl, ni, 768, st)

def capture():
    g = P()
    assert h.hipStreamBeginCapture(st, 1) == 0
    call()
    code = cw.lib.xattn_get_last_error()
    msg = cw.lib.xattn_get_last_error_string().decode()
    assert h.hipStreamEndCapture(st, ctypes.byref(g)) == 0
    return g, code, msg

g, code, msg = capture()
assert code == 5 and "xattn_noalloc_prepare" in msg, (code, msg)
n = ctypes.c_size_t(0)
assert h.hipGraphGetNodes(g, None, ctypes.byref(n)) == 0 and n.value == 0, n.value
h.hipGraphDestroy(g)
assert cw.lib.xattn_noalloc_prepare(0) == 0
g, code, msg = capture()
assert code == 0, (code, msg)
exe = P()
assert h.hipGraphInstantiate(ctypes.byref(exe), g, None, None, 0) == 0
ref = cw.run_vectorized_kernel(q[0], k[0], v[0], nl, ni, 768)
for rep in range(3):
    out.zero()
    assert h.hipGraphLaunch(exe, st) == 0
    assert h.hipStreamSynchronize(st) == 0
    got = out.download((b, nl, 768))
    assert np.array_equal(got, ref), rep
h.hipGraphExecDestroy(exe)
h.hipGraphDestroy(g)
h.hipStreamDestroy(st)
print("NOALLOC-CAPTURE-OK", flush=True)
"""


def test_noalloc_first_call_under_capture_in_a_fresh_process(cw):
    """A process whose first split call of launch_optimized_kernel_noalloc is
    made under stream capture: refused with XATTN_ERR_CAPTURE, nothing
    recorded; after xattn_noalloc_prepare(0) the same call is captured and
    the graph's replays equal launch_optimized_kernel bit for bit."""
    r = subprocess.run([sys.executable, "-u", "-c", _CAPTURE_SCRIPT, PKG,
                        os.path.join(ROOT, "oracle")],
                       cwd=ROOT, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "NOALLOC-CAPTURE-OK" in r.stdout, r.stdout + r.stderr
