"""Offsets past 2**31 elements and 2**32 bytes.  The reference forms batch
offsets in 32-bit int (kernel_vectorized.cu:38-40, kernel_splitk.cu:73-74),
which wraps once B * N * 768 passes 2**31; here every tensor of one launch
passes it: Q and O (B=3600, N_latent=800) and K and V (N_input=784), through
launch_optimized_kernel (fp32), launch_wmma_kernel (fp16) and
launch_wmma_bf16_kernel.  The batch
elements repeat a few distinct blocks (device-to-device copies of random
blocks), chosen per tensor with different periods, so an offset that wrapped
would read rows of another block, or straddle two, and fail the check against
the float64 oracle on the first batch element, those around the 2**32-byte
and 2**31-element marks, and the last."""

import ctypes
import math

import numpy as np
import pytest

from conftest import fp32_gate, gate16

pytestmark = pytest.mark.gpu

B, NL, NI, D = 3600, 800, 784, 768
NQ, NKV = 5, 7  # distinct Q blocks, distinct K/V blocks
D2H, D2D = 2, 3  # hipMemcpyKind


def _checked(b_elems):
    """Batch elements to check: the first, those whose tensor start crosses
    2**32 bytes (fp32) and 2**31 elements, and the last."""
    bs = {0, B - 1}
    for mark in (2 ** 30, 2 ** 31):  # fp32 2**32 bytes; 2**31 elements (16-bit 2**32 bytes)
        first = -(-mark // b_elems)
        bs.update({first - 1, first})
    return sorted(b for b in bs if 0 <= b < B)


def _filled(cw, blocks, period, nbytes_each):
    """A device buffer of B batch elements, element b a copy of
    blocks[b % period] (host arrays of nbytes_each bytes each)."""
    src = cw.DeviceBuffer.holding(np.ascontiguousarray(np.stack(blocks[:period])))
    dst = cw.DeviceBuffer(B * nbytes_each)
    try:
        for b in range(B):
            err = cw.cudart.hipMemcpy(ctypes.c_void_p(dst.ptr.value + b * nbytes_each),
                                      ctypes.c_void_p(src.ptr.value + (b % period) * nbytes_each),
                                      nbytes_each, D2D)
            assert err == 0, f"device copy {b}: HIP error {err}"
    except Exception:
        dst.close()
        raise
    finally:
        src.close()
    return dst


def _row_block(cw, out, b):
    host = np.empty((NL, D), np.float32)
    err = cw.cudart.hipMemcpy(host.ctypes.data_as(ctypes.c_void_p),
                              ctypes.c_void_p(out.ptr.value + b * NL * D * 4), host.nbytes, D2H)
    assert err == 0, f"copy back {b}: HIP error {err}"
    return host


def _widen(oracle, precision, a):
    """16-bit host values as float32."""
    return oracle.bf16_bits_to_f32(a) if precision == "bf16" else a.astype(np.float32)


@pytest.mark.parametrize("precision", ["fp32", "fp16", "bf16"])
def test_offsets_past_2_31_elements(cw, oracle, precision):
    assert B * NL * D > 2 ** 31 and B * NI * D > 2 ** 31
    rng = np.random.RandomState(31)
    qs = [rng.randn(NL, D).astype(np.float32) for _ in range(NQ)]
    ks = [rng.randn(NI, D).astype(np.float32) for _ in range(NKV)]
    vs = [rng.randn(NI, D).astype(np.float32) for _ in range(NKV)]
    if precision == "fp32":
        hq, hk, hv, esize = qs, ks, vs, 4
    else:
        # the 16-bit paths' host side: Q pre-scaled by 1/sqrt(D), all rounded to
        # fp16 / bf16 (one call per block, the other two tensors padded with block 0)
        bf = precision == "bf16"
        hq = [cw._half_inputs(q[None], ks[0][None], vs[0][None], 1, D, bf)[0][0] for q in qs]
        hk = [cw._half_inputs(qs[0][None], k[None], vs[0][None], 1, D, bf)[1][0] for k in ks]
        hv = [cw._half_inputs(qs[0][None], ks[0][None], v[None], 1, D, bf)[2][0] for v in vs]
        esize = 2
    bufs = []
    try:
        for blocks, period, rows in ((hq, NQ, NL), (hk, NKV, NI), (hv, NKV, NI)):
            bufs.append(_filled(cw, blocks, period, rows * D * esize))
        out = cw.DeviceBuffer(B * NL * D * 4).zero()
        bufs.append(out)
        q, k, v = bufs[:3]
        if precision == "fp32":
            cw.lib.launch_optimized_kernel(q.f32, k.f32, v.f32, out.f32, B, NL, NI, D, None)
        else:
            fn = cw.lib.launch_wmma_bf16_kernel if precision == "bf16" else cw.lib.launch_wmma_kernel
            fn(q.ptr, k.ptr, v.ptr, out.f32, B, NL, NI, D, None)
        cw._raise_launch_errors(f"{precision} launch")
        assert cw.cudart.hipDeviceSynchronize() == 0
        bad = []
        for b in sorted(set(_checked(NL * D)) | set(_checked(NI * D))):
            got = _row_block(cw, out, b)
            iq, ik = b % NQ, b % NKV
            if precision == "fp32":
                ref = oracle.attention_f64(qs[iq][None], ks[ik][None], vs[ik][None])[0]
                try:
                    fp32_gate(got, ref)
                except AssertionError as e:
                    bad.append(f"b={b}: {e}")
            else:
                ref = oracle.attention_f64(
                    _widen(oracle, precision, hq[iq])[None].astype(np.float64) * math.sqrt(D),
                    _widen(oracle, precision, hk[ik])[None],
                    _widen(oracle, precision, hv[ik])[None])[0]
                ref32 = oracle.attention_f64(qs[iq][None], ks[ik][None], vs[ik][None])[0]
                try:
                    gate16(got, ref32, ref, precision == "bf16")
                except AssertionError as e:
                    bad.append(f"b={b}: {e}")
        assert not bad, "\n".join(bad)
    finally:
        for buf in bufs:
            buf.close()


@pytest.mark.parametrize("precision", ["fp32", "fp16", "bf16"])
def test_split_partials_past_2_31_elements(cw, oracle, precision):
    """Caller-owned split partials of B * N_latent * num_splits * 768 > 2**31
    elements (B=64, N_latent=1024, 64 splits of N_input=784: chunks of 13
    keys for fp32, so 61 splits carry keys, and of 16 for fp16 / bf16, so 49
    do; the rest are empty and write sentinels) through launch_splitk_kernel,
    launch_wmma_splitk_kernel and launch_wmma_splitk_bf16_kernel; the merged
    output is checked against the float64 oracle on batch elements whose
    partials lie before, across and past the 2**31-element mark."""
    b, nl, ni, s = 64, 1024, 784, 64
    assert b * nl * s * D > 2 ** 31
    rng = np.random.RandomState(64)
    q = rng.randn(b, nl, D).astype(np.float32)
    k = rng.randn(b, ni, D).astype(np.float32)
    v = rng.randn(b, ni, D).astype(np.float32)
    host = ((q, k, v) if precision == "fp32"
            else cw._half_inputs(q, k, v, b, D, precision == "bf16"))
    rows = b * nl
    bufs = []
    try:
        bufs = [cw.DeviceBuffer.holding(a) for a in host]
        out = cw.DeviceBuffer(rows * D * 4).zero()
        po = cw.DeviceBuffer(rows * s * D * 4)
        pm, pl = cw.DeviceBuffer(rows * s * 4), cw.DeviceBuffer(rows * s * 4)
        bufs += [out, po, pm, pl]
        if precision == "fp32":
            cw.lib.launch_splitk_kernel(*[x.f32 for x in bufs[:3]], out.f32, po.f32, pm.f32,
                                        pl.f32, b, nl, ni, D, s, None)
        else:
            fn = (cw.lib.launch_wmma_splitk_bf16_kernel if precision == "bf16"
                  else cw.lib.launch_wmma_splitk_kernel)
            fn(*[x.ptr for x in bufs[:3]], out.f32, po.f32, pm.f32, pl.f32, b, nl, ni, D, s, None)
        cw._raise_launch_errors(f"{precision} split launch")
        assert cw.cudart.hipDeviceSynchronize() == 0
        mark = 2 ** 31 // (s * D * nl)  # the batch element whose partials cross 2**31
        res = out.download((b, nl, D))
        bad = []
        for bi in sorted({0, mark - 1, mark, mark + 1, b - 1}):
            if precision == "fp32":
                ref = oracle.attention_f64(q[bi:bi + 1], k[bi:bi + 1], v[bi:bi + 1])
                try:
                    fp32_gate(res[bi:bi + 1], ref)
                except AssertionError as e:
                    bad.append(f"b={bi}: {e}")
            else:
                qh, kh, vh = (_widen(oracle, precision, a[bi:bi + 1]) for a in host)
                ref = oracle.attention_f64(qh.astype(np.float64) * math.sqrt(D), kh, vh)
                ref32 = oracle.attention_f64(q[bi:bi + 1], k[bi:bi + 1], v[bi:bi + 1])
                try:
                    gate16(res[bi:bi + 1], ref32, ref, precision == "bf16")
                except AssertionError as e:
                    bad.append(f"b={bi}: {e}")
        assert not bad, "\n".join(bad)
    finally:
        for buf in bufs:
            buf.close()
