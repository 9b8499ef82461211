"""CPU oracle for fused single-head cross-attention  O = softmax(Q K^T / sqrt(D)) V.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module: only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and only as the checker (or, for ``sdpa_cpu``, as the
timed CPU baseline).  The HIP library never routes through it.

Every function restates one piece of the reference's algorithm and cites the
reference file:line it follows.  How each function is pinned (independently of
retyping its own formula) is listed here and exercised in
``tests/test_oracle.py``:

================================  ==========================================
function                          pinned by
================================  ==========================================
attention_f64                     pure-Python brute force on tiny shapes;
                                  scipy.special.softmax; closed-form special
                                  cases (V const, K=0, NI=1, one-hot peak);
                                  permutation / linearity / batch invariants
attention_torch_f32               agrees with attention_f64 (<=1e-6 abs) and
                                  with torch CPU SDPA, a separate library
                                  routine
attention_numpy_f32               agrees with attention_f64
online_softmax_f64                equals two-pass attention_f64 for NI in
                                  {1, 15, 16, 17, 33}, any tile size
splitk_bounds                     brute-force partition checks (cover, disjoint,
                                  empty-split positions) against hand-counted
                                  cases from the reference launch shapes
splitk_partials / splitk_combine  merge of any partition == unsplit
                                  attention_f64; S=1 identity; empty-split
                                  sentinel; order independence
round_fp16 / round_bf16           numpy float16 cast (IEEE RNE) and exhaustive
                                  bit-pattern checks for bf16 ties/NaN/Inf
================================  ==========================================
"""

from __future__ import annotations

import math

import numpy as np

D_MODEL = 768
FLT_MAX = float(np.finfo(np.float32).max)


# ---------------------------------------------------------------------------
# Input generation
# ---------------------------------------------------------------------------

def make_inputs_legacy(batch, n_latent, n_input, dim=D_MODEL, seed=42):
    """Seed-42 legacy-MT19937 draws in the order Q, K, V.

    Follows generate_references.py:25-31 (B=1, 2-D arrays) and
    generate_batch_references.py:28-34 (3-D arrays): ``np.random.seed(seed)``
    then ``randn`` for Q, K and V, cast to float32.  Returns 3-D arrays.
    """
    np.random.seed(seed)
    if batch == 1:
        q = np.random.randn(n_latent, dim).astype(np.float32)[None]
        k = np.random.randn(n_input, dim).astype(np.float32)[None]
        v = np.random.randn(n_input, dim).astype(np.float32)[None]
    else:
        q = np.random.randn(batch, n_latent, dim).astype(np.float32)
        k = np.random.randn(batch, n_input, dim).astype(np.float32)
        v = np.random.randn(batch, n_input, dim).astype(np.float32)
    return q, k, v


def make_inputs(batch, n_latent, n_input, dim=D_MODEL, seed=0, q_std=1.0):
    """``RandomState(seed)`` draws Q, K, V ~ N(0,1) (Q scaled by ``q_std``).

    Draw order and generator follow experiments/gen_perceiver_refs.py:43-49;
    ``q_std=0.02`` is the latent-init scale used for the long-input split-K
    workload.
    """
    rng = np.random.RandomState(seed)
    q = rng.randn(batch, n_latent, dim).astype(np.float32)
    k = rng.randn(batch, n_input, dim).astype(np.float32)
    v = rng.randn(batch, n_input, dim).astype(np.float32)
    if q_std != 1.0:
        q = (q * np.float32(q_std)).astype(np.float32)
    return q, k, v


# ---------------------------------------------------------------------------
# Closed forms
# ---------------------------------------------------------------------------

def _as3(a):
    a = np.asarray(a)
    return a[None] if a.ndim == 2 else a


def attention_f64(q, k, v):
    """float64 closed form of generate_references.py:17-23.

    ``bmm(Q, K^T) / sqrt(D)`` -> row softmax (max-subtracted, as
    experiments/gen_perceiver_refs.py:36-39) -> ``bmm(P, V)``.  Inputs are
    [B, N, D] or [N, D]; the result is float64 [B, NL, D].  An empty key set
    (NI = 0) yields zeros, which is what every reference kernel writes for it
    (running sum 0 times a finite normaliser).
    """
    q = _as3(q).astype(np.float64)
    k = _as3(k).astype(np.float64)
    v = _as3(v).astype(np.float64)
    d = q.shape[-1]
    if k.shape[1] == 0:
        return np.zeros(q.shape[:2] + (v.shape[-1],), np.float64)
    s = np.matmul(q, np.swapaxes(k, 1, 2)) / math.sqrt(d)
    s -= s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    p = e / e.sum(axis=-1, keepdims=True)
    return np.matmul(p, v)


def attention_torch_f32(q, k, v):
    """float32 restatement of the reference's PyTorch path on the CPU.

    generate_references.py:17-23 / generate_batch_references.py:20-26:
    ``torch.bmm(Q, K.transpose(1, 2)) / np.sqrt(D)`` -> ``torch.softmax(-1)``
    -> ``torch.bmm(attn, V)``, all float32 on the CPU.
    """
    import torch

    qt = torch.from_numpy(np.ascontiguousarray(_as3(q), np.float32))
    kt = torch.from_numpy(np.ascontiguousarray(_as3(k), np.float32))
    vt = torch.from_numpy(np.ascontiguousarray(_as3(v), np.float32))
    d = qt.shape[-1]
    scores = torch.bmm(qt, kt.transpose(1, 2).contiguous()) / np.sqrt(d)
    attn = torch.softmax(scores, dim=-1)
    return torch.bmm(attn, vt).numpy()


def attention_numpy_f32(q, k, v):
    """experiments/gen_perceiver_refs.py:30-40 in float32, batched."""
    q = _as3(q).astype(np.float32)
    k = _as3(k).astype(np.float32)
    v = _as3(v).astype(np.float32)
    d = q.shape[-1]
    s = np.matmul(q, np.swapaxes(k, 1, 2)) / np.sqrt(d).astype(np.float32)
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    p = e / e.sum(axis=-1, keepdims=True)
    return np.matmul(p, v).astype(np.float32)


def sdpa_cpu(q, k, v, threads=None):
    """PyTorch CPU ``scaled_dot_product_attention`` in float32.

    Layout [B, 1, N, D] and ``scale = 1/sqrt(D)`` as experiments/sdpa_bench.py:
    46-53, run on the host.  This is the reference's CPU path used as the
    reported CPU baseline.
    """
    import torch
    import torch.nn.functional as F

    if threads:
        torch.set_num_threads(int(threads))
    qt = torch.from_numpy(np.ascontiguousarray(_as3(q), np.float32)).unsqueeze(1)
    kt = torch.from_numpy(np.ascontiguousarray(_as3(k), np.float32)).unsqueeze(1)
    vt = torch.from_numpy(np.ascontiguousarray(_as3(v), np.float32)).unsqueeze(1)
    scale = 1.0 / math.sqrt(qt.shape[-1])
    with torch.no_grad():
        out = F.scaled_dot_product_attention(qt, kt, vt, scale=scale)
    return out.squeeze(1).numpy()


# ---------------------------------------------------------------------------
# Online softmax and split-K (the fused kernels' algorithm)
# ---------------------------------------------------------------------------

def online_softmax_f64(q, k, v, tile=16, eps=1e-6):
    """Tile-by-tile running max / running sum, as kernel_vectorized.cu:58-181.

    For each key tile: new_max = max(running_max, tile_max); the accumulator
    and running sum are rescaled by exp(running_max - new_max); tile weights
    exp(s - new_max) are summed and applied to V.  The result is normalised by
    1 / (running_sum + eps) (kernel_vectorized.cu:181).  float64.
    """
    q = _as3(q).astype(np.float64)
    k = _as3(k).astype(np.float64)
    v = _as3(v).astype(np.float64)
    b, nl, d = q.shape
    ni = k.shape[1]
    acc = np.zeros((b, nl, v.shape[-1]))
    run_max = np.full((b, nl, 1), -FLT_MAX)
    run_sum = np.zeros((b, nl, 1))
    for t0 in range(0, ni, tile):
        kt = k[:, t0:t0 + tile]
        vt = v[:, t0:t0 + tile]
        s = np.matmul(q, np.swapaxes(kt, 1, 2)) / math.sqrt(d)
        new_max = np.maximum(run_max, s.max(axis=-1, keepdims=True))
        scale = np.exp(run_max - new_max)
        acc *= scale
        run_sum *= scale
        e = np.exp(s - new_max)
        run_sum += e.sum(axis=-1, keepdims=True)
        acc += np.matmul(e, vt)
        run_max = new_max
    return acc / (run_sum + eps)


def splitk_bounds(n_input, num_splits, align=1):
    """Key range [k0, k1) of every split.

    kernel_splitk.cu:59-62: ``chunk = ceil(NI / S)``, ``k0 = s * chunk``,
    ``k1 = min(k0 + chunk, NI)``, a split with ``k0 >= NI`` is empty.
    kernel_wmma_splitk.cu:52-54 rounds ``chunk`` up to a multiple of 16
    (``align=16``).  Empty splits are returned as ``(k0, k0)`` with
    ``k0 >= NI`` kept, so callers can see where the sentinel goes.
    """
    chunk = (n_input + num_splits - 1) // num_splits if num_splits > 0 else 0
    if align > 1:
        chunk = (chunk + align - 1) // align * align
    out = []
    for s in range(num_splits):
        k0 = s * chunk
        k1 = min(k0 + chunk, n_input)
        out.append((k0, k1 if k0 < n_input else k0))
    return out, chunk


def splitk_partials(q, k, v, num_splits, align=1):
    """Unnormalised per-split partials, kernel_splitk.cu:42-181.

    Returns ``po [B, NL, S, D]`` (sum of exp(s - pm) * V over the split),
    ``pm [B, NL, S]`` (max score of the split, score = q.k / sqrt(D)) and
    ``pl [B, NL, S]`` (sum of exp(s - pm)).  An empty split holds the
    sentinel ``(pm, pl, po) = (-FLT_MAX, 0, 0)`` (kernel_splitk.cu:62-71).
    float64.  The flat index of (b, i, s) is ``(b * NL + i) * S + s``
    (kernel_splitk.cu:57), i.e. C order of these arrays.
    """
    q = _as3(q).astype(np.float64)
    k = _as3(k).astype(np.float64)
    v = _as3(v).astype(np.float64)
    b, nl, d = q.shape
    bounds, _ = splitk_bounds(k.shape[1], num_splits, align)
    po = np.zeros((b, nl, num_splits, v.shape[-1]))
    pm = np.full((b, nl, num_splits), -FLT_MAX)
    pl = np.zeros((b, nl, num_splits))
    for s, (k0, k1) in enumerate(bounds):
        if k1 <= k0:
            continue
        sc = np.matmul(q, np.swapaxes(k[:, k0:k1], 1, 2)) / math.sqrt(d)
        m = sc.max(axis=-1)
        e = np.exp(sc - m[..., None])
        pm[:, :, s] = m
        pl[:, :, s] = e.sum(axis=-1)
        po[:, :, s] = np.matmul(e, v[:, k0:k1])
    return po, pm, pl


def splitk_combine(po, pm, pl, eps=1e-6):
    """Log-sum-exp merge of split partials, kernel_splitk.cu:186-236.

    ``M = max_s pm``; ``L = sum over non-sentinel s of exp(pm_s - M) pl_s``;
    ``O = sum over non-sentinel s of exp(pm_s - M) po_s / (L + eps)``.
    float64.
    """
    po = np.asarray(po, np.float64)
    pm = np.asarray(pm, np.float64)
    pl = np.asarray(pl, np.float64)
    big_m = pm.max(axis=-1, keepdims=True)
    live = pm > -FLT_MAX
    w = np.where(live, np.exp(np.where(live, pm - big_m, 0.0)), 0.0)
    big_l = (w * pl).sum(axis=-1)
    acc = (w[..., None] * po).sum(axis=-2)
    return acc / (big_l[..., None] + eps)


# ---------------------------------------------------------------------------
# Reduced precision
# ---------------------------------------------------------------------------

def round_fp16(x):
    """IEEE binary16 round-to-nearest-even, as ``np.ascontiguousarray(x,
    dtype=np.float16)`` in cuda_wrappers.py:559-561 / 638-640."""
    return np.asarray(x, np.float32).astype(np.float16)


def round_bf16_bits(x):
    """bfloat16 round-to-nearest-even, returned as uint16 bit patterns.

    NaN stays a quiet NaN; overflow rounds to +-Inf as RNE dictates.
    """
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = np.where(nan, (u >> 16) | 0x40, rounded).astype(np.uint16)
    return out


def bf16_bits_to_f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x):
    """bfloat16 RNE value as float32."""
    return bf16_bits_to_f32(round_bf16_bits(x))


def prescale_q_f16(q):
    """Host-side Q pre-scale then fp16 cast, cuda_wrappers.py:635-640."""
    qs = np.asarray(q, np.float32) / np.sqrt(q.shape[-1]).astype(np.float32)
    return round_fp16(qs)


# ---------------------------------------------------------------------------
# Error metrics
# ---------------------------------------------------------------------------

def max_abs(out, ref):
    return float(np.max(np.abs(np.asarray(out, np.float64) - np.asarray(ref, np.float64))))


def rel_err(out, ref):
    """``max_abs / (max|ref| + 1e-6)``, experiments/bench_perceiver_ni.py:147-148."""
    ref = np.asarray(ref, np.float64)
    return max_abs(out, ref) / (float(np.max(np.abs(ref))) + 1e-6)
