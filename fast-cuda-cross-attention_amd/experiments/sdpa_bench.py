"""
PyTorch-ROCm scaled_dot_product_attention timed on one forced backend: the
framework baseline of the comparison (the reference's experiments/
sdpa_bench.py:28-70).  Single head, head_dim = D = 768, layout [B, 1, N, D],
scale 1/sqrt(D); timed with events on torch's current stream; returns the
output as float32 numpy for the accuracy check.

Backends: 'math' (materialized: score matrix in HBM), 'efficient' and
'flash' (fused; the ones that refuse head_dim 768 raise, and the caller logs
that).  SDPA's math backend in fp16 / bf16 is switched off here and raises
before touching the GPU: it multiplies by a transposed view of K, and 16-bit
batched products whose right operand is a transposed view are reported to
fault GPUs on this ROCm stack.  The 16-bit materialized baseline is instead
the product spelled out by hand -- bmm(Q, contiguous K^T), softmax in the
input type, bmm(P, V) -- under its own name, ``bmm_fp16`` / ``bmm_bf16``
(benchmark_bmm_events); it is not SDPA.
"""

import math
import statistics

import numpy as np

BACKENDS = ("math", "efficient", "flash")


def _prep(a, batch):
    """float32 C-contiguous [batch, N, D]; a 2-D or batch-1 input is repeated."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    if a.ndim == 2:
        a = a[None]
    if a.shape[0] == 1 and batch > 1:
        a = np.repeat(a, batch, axis=0)
    return a


def torch_dtype(precision):
    import torch
    return {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}[precision]


def materialized_bmm(q, k, v, scale):
    """softmax(q k^T * scale) v as two torch.bmm calls whose operands are all
    contiguous (K^T is copied out first); q, k, v: [B, 1, N, D], any dtype."""
    import torch
    qb, kb, vb = (t.squeeze(1) for t in (q, k, v))
    kt = kb.transpose(1, 2).contiguous()
    s = torch.bmm(qb, kt) * scale
    p = torch.softmax(s, dim=-1)
    return torch.bmm(p, vb).unsqueeze(1)


MATH_16BIT_OFF = ("SDPA math in 16 bit is switched off: its batched product takes a "
                  "transposed K view, which is reported to fault GPUs on this stack "
                  "(use bmm_fp16 / bmm_bf16, the hand-written materialized product)")


def sdpa_callable(backend, precision):
    """f(q, k, v, scale) running SDPA on ``backend``; raises for 16-bit
    'math' (see the module note)."""
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    if backend not in BACKENDS:
        raise ValueError(f"unknown SDPA backend {backend!r}")
    if backend == "math" and precision != "fp32":
        raise RuntimeError(MATH_16BIT_OFF)
    forced = {"math": SDPBackend.MATH, "efficient": SDPBackend.EFFICIENT_ATTENTION,
              "flash": SDPBackend.FLASH_ATTENTION}[backend]

    def run(q, k, v, scale):
        with sdpa_kernel(forced):
            return F.scaled_dot_product_attention(q, k, v, scale=scale)

    return run


def time_events(fn, warmup, iters):
    """warmup calls, then ``iters`` calls each between two events on torch's
    current stream; per-call milliseconds."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for s, e in zip(starts, ends):
        s.record()
        fn()
        e.record()
    torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in zip(starts, ends)]


def _time_torch(fn, Q, K, V, batch_size, N_latent, N_input, D, precision, warmup, iters):
    """Shared body: inputs to the GPU in ``precision`` as [B, 1, N, D],
    ``fn(q, k, v, scale)`` timed with events; (out float32 numpy, mean_ms,
    std_ms)."""
    import torch

    dt = torch_dtype(precision)
    q, k, v = (torch.from_numpy(_prep(a, batch_size)).to("cuda", dt).unsqueeze(1)
               for a in (Q, K, V))
    if q.shape[2] != N_latent or k.shape[2] != N_input or q.shape[3] != D:
        raise ValueError(f"shapes {tuple(q.shape)}, {tuple(k.shape)} do not match "
                         f"N_latent={N_latent} N_input={N_input} D={D}")
    scale = 1.0 / math.sqrt(D)
    out = fn(q, k, v, scale)  # an ineligible backend raises here
    times = time_events(lambda: fn(q, k, v, scale), warmup, iters)
    out = fn(q, k, v, scale)
    torch.cuda.synchronize()
    out_np = out.squeeze(1).float().cpu().numpy()
    del q, k, v, out
    torch.cuda.empty_cache()
    return (out_np, statistics.mean(times),
            statistics.pstdev(times) if len(times) > 1 else 0.0)


def benchmark_sdpa_events(Q, K, V, batch_size, N_latent, N_input, D, backend="math",
                          precision="fp32", warmup=20, iters=100):
    """Time SDPA on a forced backend.  Returns (out[B, Nl, D] float32 numpy,
    mean_ms, std_ms); raises what SDPA raises for an ineligible backend, and
    RuntimeError for the switched-off 16-bit math path."""
    fn = sdpa_callable(backend, precision)
    return _time_torch(fn, Q, K, V, batch_size, N_latent, N_input, D, precision, warmup,
                       iters)


def benchmark_bmm_events(Q, K, V, batch_size, N_latent, N_input, D, precision="fp16",
                         warmup=20, iters=100):
    """Time the hand-written materialized product (materialized_bmm) in
    ``precision``: the 16-bit materialized baseline, in place of SDPA math."""
    return _time_torch(materialized_bmm, Q, K, V, batch_size, N_latent, N_input, D,
                       precision, warmup, iters)
