"""Split launches inside HIP stream capture: launch_optimized_kernel, and
(last test) launch_wmma_bf16_kernel, launch_splitk_kernel with caller
scratch and launch_optimized_kernel_noalloc in one graph.

The shape B=1, N_latent=64, N_input=784 is planned with key splits, so the
launch uses its stream's library workspace.  With the workspace already
sized by an eager launch on the stream, the launch is captured into a graph
and replayed several times, with eager work and synchronisations between
replays; every replay must match the float64 oracle.  The stream's workspace
then grows (an eager launch of a larger split shape) and the graph, which
still points at the replaced block, is replayed again.  A capture whose
launch would have to allocate is refused with XATTN_ERR_CAPTURE and
enqueues nothing (that test runs first: the library keys workspaces by
stream handle, and a new stream may reuse a destroyed one's handle)."""

import ctypes

import numpy as np
import pytest

from conftest import fp32_gate, gate16

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p
XATTN_ERR_CAPTURE = 5
CAPTURE_THREAD_LOCAL = 1


def _hip(cw):
    h = cw._load_hip()
    sigs = {
        "hipStreamCreate": [ctypes.POINTER(P)],
        "hipStreamDestroy": [P],
        "hipStreamSynchronize": [P],
        "hipStreamBeginCapture": [P, ctypes.c_int],
        "hipStreamEndCapture": [P, ctypes.POINTER(P)],
        "hipGraphInstantiate": [ctypes.POINTER(P), P, P, P, ctypes.c_size_t],
        "hipGraphLaunch": [P, P],
        "hipGraphExecDestroy": [P],
        "hipGraphDestroy": [P],
    }
    for name, args in sigs.items():
        fn = getattr(h, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    return h


class _Case:
    """Inputs of one shape on the device, its output buffer and the oracle."""

    def __init__(self, cw, oracle, b, nl, ni, seed, ref_rows=None, ref_latents=None):
        self.shape = (b, nl, ni)
        q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=seed)
        # the oracle on a subset (batch rows x first latents) for large shapes
        self.rows = list(range(b)) if ref_rows is None else list(ref_rows)
        self.lat = nl if ref_latents is None else ref_latents
        r = self.rows
        self.ref = oracle.attention_f64(q[r, :self.lat], k[r], v[r])
        self.bufs = [cw.DeviceBuffer.holding(a) for a in (q, k, v)]
        self.out = cw.DeviceBuffer(b * nl * 768 * 4)

    def launch(self, cw, stream):
        b, nl, ni = self.shape
        q, k, v = self.bufs
        cw.lib.launch_optimized_kernel(q.f32, k.f32, v.f32, self.out.f32, b, nl, ni, 768, stream)

    def check(self, cw):
        b, nl, _ = self.shape
        got = self.out.download((b, nl, 768))
        fp32_gate(got[self.rows, :self.lat], self.ref)

    def close(self):
        for p in self.bufs + [self.out]:
            p.close()


def _capture(h, stream, body):
    graph = P()
    assert h.hipStreamBeginCapture(stream, CAPTURE_THREAD_LOCAL) == 0
    try:
        body()
    finally:
        end = h.hipStreamEndCapture(stream, ctypes.byref(graph))
    assert end == 0
    return graph


def test_capture_that_would_allocate_is_refused(cw, oracle):
    # A split plan whose partials (B * N_latent * splits * 770 * 4 bytes)
    # exceed any workspace an earlier test can have left on a stream handle
    # that the new stream may reuse.
    b, nl, ni = 10, 832, 784
    cu, _ = cw.device_info()
    _, s = cw.f32_plan(b, nl, ni, cu)
    assert s > 1 and b * nl * s * 770 * 4 > 120e6
    h = _hip(cw)
    stream = P()
    assert h.hipStreamCreate(ctypes.byref(stream)) == 0
    case = _Case(cw, oracle, b, nl, ni, seed=13, ref_rows=(0, 5, 9), ref_latents=64)
    graph = P()
    try:
        assert cw.lib.xattn_get_last_error() == 0
        case.out.zero()
        graph = _capture(h, stream, lambda: case.launch(cw, stream))
        code = cw.lib.xattn_get_last_error()
        msg = cw.lib.xattn_get_last_error_string().decode()
        assert code == XATTN_ERR_CAPTURE, (code, msg)
        assert "capturing" in msg
        # nothing was enqueued: the captured graph has no kernel nodes
        num = ctypes.c_size_t(0)
        h.hipGraphGetNodes.argtypes = [P, P, ctypes.POINTER(ctypes.c_size_t)]
        h.hipGraphGetNodes.restype = ctypes.c_int
        assert h.hipGraphGetNodes(graph, None, ctypes.byref(num)) == 0
        assert num.value == 0
        # outside capture the same launch allocates and runs
        case.launch(cw, stream)
        cw._lib_error_check("eager launch")
        assert h.hipStreamSynchronize(stream) == 0
        case.check(cw)
    finally:
        assert cw.cudart.hipDeviceSynchronize() == 0
        if graph:
            h.hipGraphDestroy(graph)
        case.close()
        h.hipStreamDestroy(stream)


def test_captured_split_launch_replays(cw, oracle):
    cu, _ = cw.device_info()
    assert cw.f32_plan(1, 64, 784, cu)[1] > 1
    assert cw.f32_plan(1, 256, 4096, cu)[1] > 1
    h = _hip(cw)
    stream = P()
    assert h.hipStreamCreate(ctypes.byref(stream)) == 0
    small = _Case(cw, oracle, 1, 64, 784, seed=11)
    large = _Case(cw, oracle, 1, 256, 4096, seed=12)
    graph, exe = P(), P()
    try:
        small.launch(cw, stream)  # sizes this stream's workspace
        cw._lib_error_check("eager launch")
        assert h.hipStreamSynchronize(stream) == 0
        small.check(cw)

        small.out.zero()
        graph = _capture(h, stream, lambda: small.launch(cw, stream))
        cw._lib_error_check("captured launch")
        assert h.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for rep in range(4):
            small.out.zero()
            assert h.hipGraphLaunch(exe, stream) == 0
            assert h.hipStreamSynchronize(stream) == 0
            small.check(cw)
            # eager work between replays, on the same and on the null stream
            large.launch(cw, stream if rep % 2 else P(0))
            cw._lib_error_check("eager launch between replays")
            assert cw.cudart.hipDeviceSynchronize() == 0
            large.check(cw)
        # the large shape grew this stream's workspace; the graph still uses
        # the replaced block, which the library keeps
        small.out.zero()
        assert h.hipGraphLaunch(exe, stream) == 0
        assert h.hipStreamSynchronize(stream) == 0
        small.check(cw)
    finally:
        assert cw.cudart.hipDeviceSynchronize() == 0
        if exe:
            h.hipGraphExecDestroy(exe)
        if graph:
            h.hipGraphDestroy(graph)
        small.close()
        large.close()
        h.hipStreamDestroy(stream)




def test_graph_replayed_on_another_stream_beside_eager_launches(cw, oracle):
    """A split launch captured on stream A owns A's workspace block from
    then on: replays of the graph on stream B, each overlapping an eager
    split launch of the same shape (other inputs) on A with no
    synchronisation between the two, must both match the float64 oracle,
    since the eager launches on A take a fresh block."""
    cu, _ = cw.device_info()
    assert cw.f32_plan(1, 64, 784, cu)[1] > 1
    h = _hip(cw)
    sa, sb = P(), P()
    assert h.hipStreamCreate(ctypes.byref(sa)) == 0
    assert h.hipStreamCreate(ctypes.byref(sb)) == 0
    graphed = _Case(cw, oracle, 1, 64, 784, seed=41)
    eager = _Case(cw, oracle, 1, 64, 784, seed=42)
    graph, exe = P(), P()
    try:
        graphed.launch(cw, sa)  # sizes A's workspace
        cw._lib_error_check("eager launch")
        assert h.hipStreamSynchronize(sa) == 0
        graph = _capture(h, sa, lambda: graphed.launch(cw, sa))
        cw._lib_error_check("captured launch")
        assert h.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for rep in range(6):
            graphed.out.zero()
            eager.out.zero()
            assert h.hipGraphLaunch(exe, sb) == 0
            eager.launch(cw, sa)
            cw._lib_error_check("eager launch beside a replay")
            assert cw.cudart.hipDeviceSynchronize() == 0
            graphed.check(cw)
            eager.check(cw)
    finally:
        assert cw.cudart.hipDeviceSynchronize() == 0
        if exe:
            h.hipGraphExecDestroy(exe)
        if graph:
            h.hipGraphDestroy(graph)
        graphed.close()
        eager.close()
        h.hipStreamDestroy(sa)
        h.hipStreamDestroy(sb)


def test_captured_16bit_scratch_and_noalloc_launches_replay(cw, oracle):
    """One graph holding three split launches of B=1 N_latent=64
    N_input=784: launch_wmma_bf16_kernel (its plan splits the keys, so it
    uses the stream's workspace, sized by an eager launch first),
    launch_splitk_kernel with caller-owned scratch (7 splits) and
    launch_optimized_kernel_noalloc (static scratch).  Replayed four times,
    outputs cleared before each replay (outside the graph) and eager launches
    of the same entry points on the null stream between replays; every
    replay must match the float64 oracle."""
    import math

    b, nl, ni, s = 1, 64, 784, 7
    cu, _ = cw.device_info()
    assert cw.wmma_plan(b, nl, ni, cu)[1] > 1 and cw.f32_plan(b, nl, ni, cu)[1] > 1
    assert cw.HAS_NOALLOC
    q, k, v = oracle.make_inputs(b, nl, ni, 768, seed=21)
    ref32 = oracle.attention_f64(q, k, v)
    hq, hk, hv = cw._half_inputs(q, k, v, b, 768, True)
    f = oracle.bf16_bits_to_f32
    ref16 = oracle.attention_f64(f(hq).astype(np.float64) * math.sqrt(768), f(hk), f(hv))
    h = _hip(cw)
    stream = P()
    assert h.hipStreamCreate(ctypes.byref(stream)) == 0
    bufs = []
    graph, exe = P(), P()
    try:
        d32 = [cw.DeviceBuffer.holding(a) for a in (q, k, v)]
        d16 = [cw.DeviceBuffer.holding(a) for a in (hq, hk, hv)]
        o16, osk, ona = (cw.DeviceBuffer(b * nl * 768 * 4) for _ in range(3))
        po = cw.DeviceBuffer(b * nl * s * 768 * 4)
        pm, pl = cw.DeviceBuffer(b * nl * s * 4), cw.DeviceBuffer(b * nl * s * 4)
        bufs = d32 + d16 + [o16, osk, ona, po, pm, pl]
        outs = (o16, osk, ona)

        def launches(st):
            cw.lib.launch_wmma_bf16_kernel(*[x.ptr for x in d16], o16.f32, b, nl, ni, 768, st)
            cw.lib.launch_splitk_kernel(*[x.f32 for x in d32], osk.f32, po.f32, pm.f32, pl.f32,
                                        b, nl, ni, 768, s, st)
            cw.lib.launch_optimized_kernel_noalloc(*[x.f32 for x in d32], ona.f32, b, nl, ni,
                                                   768, st)

        def check():
            gate16(o16.download((b, nl, 768)), ref32, ref16, True)
            fp32_gate(osk.download((b, nl, 768)), ref32)
            fp32_gate(ona.download((b, nl, 768)), ref32)

        launches(stream)  # sizes this stream's workspace for the bf16 plan
        cw._lib_error_check("eager launches")
        assert h.hipStreamSynchronize(stream) == 0
        check()
        graph = _capture(h, stream, lambda: launches(stream))
        cw._lib_error_check("captured launches")
        assert h.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for rep in range(4):
            for o in outs:
                o.zero()
            assert h.hipGraphLaunch(exe, stream) == 0
            assert h.hipStreamSynchronize(stream) == 0
            check()
            launches(P(0))  # eager work between replays
            cw._lib_error_check("eager launches between replays")
            assert cw.cudart.hipDeviceSynchronize() == 0
            check()
    finally:
        assert cw.cudart.hipDeviceSynchronize() == 0
        if exe:
            h.hipGraphExecDestroy(exe)
        if graph:
            h.hipGraphDestroy(graph)
        for x in bufs:
            x.close()
        h.hipStreamDestroy(stream)
