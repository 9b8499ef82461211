"""
Roofline quantities of one cross-attention call, softmax(Q K^T / sqrt(D)) V,
with Q [B, Nl, D], K and V [B, Ni, D], out [B, Nl, D].

FLOP (the two products; the softmax's O(B Nl Ni) work is left out, as in the
reference's convention, experiments/roofline.py:25-27):

    4 * B * Nl * Ni * D

HBM bytes, one pass (experiments/roofline.py:30-36):

    fused         read Q, K, V once, write out once:
                  B * (Nl*D*in + 2*Ni*D*in + Nl*D*out)
    materialized  fused + write and read back the B*Nl*Ni score matrix (in
                  the input precision)

``out_precision`` defaults to the input precision (the reference's model);
this library's fp16/bf16 entry points write fp32 rows, so their callers pass
out_precision="fp32".
"""

BYTES_PER_ELEM = {"fp32": 4, "fp16": 2, "bf16": 2}


def flops(B, Nl, Ni, D):
    """FLOP of the two matrix products: 4*B*Nl*Ni*D."""
    return 4.0 * B * Nl * Ni * D


def bytes_moved(B, Nl, Ni, D, precision="fp32", materialized=False, out_precision=None):
    """HBM bytes of one call under the fused or materialized model."""
    bi = BYTES_PER_ELEM[precision]
    bo = BYTES_PER_ELEM[out_precision or precision]
    fused = float(B) * (Nl * D * bi + 2.0 * Ni * D * bi + Nl * D * bo)
    if not materialized:
        return fused
    return fused + 2.0 * B * Nl * Ni * bi


def arithmetic_intensity(B, Nl, Ni, D, precision="fp32", materialized=False,
                         out_precision=None):
    """FLOP per HBM byte."""
    return flops(B, Nl, Ni, D) / bytes_moved(B, Nl, Ni, D, precision, materialized,
                                             out_precision)


def achieved_flops(B, Nl, Ni, D, latency_s):
    """FLOP/s at a measured latency (seconds)."""
    return flops(B, Nl, Ni, D) / latency_s


def achieved_bw(B, Nl, Ni, D, latency_s, precision="fp32", materialized=False,
                out_precision=None):
    """Model HBM bytes/s at a measured latency (seconds)."""
    return bytes_moved(B, Nl, Ni, D, precision, materialized, out_precision) / latency_s


def roofline_row(B, Nl, Ni, D, latency_s, gpu_key, precision="fp32", materialized=False,
                 out_precision=None):
    """Derived metrics of one measured point: flops, bytes, arithmetic
    intensity, achieved GFLOP/s and GB/s, and -- when ``gpu_key`` names a
    GPU_SPECS entry -- % of the compute and bandwidth peaks, the ridge point
    and which side of it the point lies on ('compute' or 'memory')."""
    try:
        from gpu_specs import GPU_SPECS, PRECISION_PEAK_KEY, ridge_point
    except ImportError:  # imported as part of the experiments package
        from .gpu_specs import GPU_SPECS, PRECISION_PEAK_KEY, ridge_point

    f = flops(B, Nl, Ni, D)
    nbytes = bytes_moved(B, Nl, Ni, D, precision, materialized, out_precision)
    ai = f / nbytes
    row = {
        "flops": f,
        "bytes": nbytes,
        "arithmetic_intensity": ai,
        "achieved_gflops": f / latency_s / 1e9,
        "achieved_gbs": nbytes / latency_s / 1e9,
    }
    spec = GPU_SPECS.get(gpu_key) if gpu_key is not None else None
    if spec is not None:
        peak = spec.get(PRECISION_PEAK_KEY[precision])
        rp = ridge_point(gpu_key, precision)
        row["pct_peak_compute"] = 100.0 * f / latency_s / peak if peak else None
        row["pct_peak_bw"] = 100.0 * nbytes / latency_s / spec["peak_bw_bytes"]
        row["ridge_point"] = rp
        row["bound"] = "compute" if (rp is not None and ai >= rp) else "memory"
    return row


if __name__ == "__main__":
    import os
    import sys
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    # the headline shape at a hypothetical 1 ms
    for k, v in roofline_row(32, 1024, 784, 768, 1e-3, "MI355X").items():
        print(f"  {k}: {v}")
