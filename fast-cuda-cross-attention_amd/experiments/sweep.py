"""
What the sweep drivers share: running one implementation at one shape and
turning the timing into a log row (csvlog.FIELDS) plus a printed line.

Implementations (the reference's names, experiments/bench_perceiver_ni.py:
109-143, plus the bf16 twins and the SDPA backends in either 16-bit type):

    naive warp tiled vectorized   fp32 kernels   benchmark_kernel_events
    splitk                        fp32 split-K   benchmark_splitk_events
    wmma wmma_splitk              fp16 MFMA      benchmark_wmma[_splitk]_events
    wmma_bf16 wmma_splitk_bf16    bf16 MFMA      benchmark_wmma[_splitk]_bf16_events
    sdpa_math sdpa_efficient sdpa_flash  (fp32; suffix _fp16 or _bf16 for 16 bit;
                                  16-bit sdpa_math is switched off and logs an error)
    bmm_fp16 bmm_bf16             materialized bmm/softmax/bmm with a contiguous
                                  K^T (the 16-bit materialized baseline; not SDPA)

The split drivers take the library's planned split count for the device's
own CU count (num_splits="plan"), not the reference's choose_num_splits default.
"""

import numpy as np

D = 768


def precision_of(impl):
    """Input precision an implementation computes in."""
    if impl.endswith("bf16"):
        return "bf16"
    if impl.startswith("wmma") or impl.endswith("fp16") or impl.endswith("16"):
        return "fp16"
    return "fp32"


def sdpa_backend_of(impl):
    name = impl[len("sdpa_"):]
    for b in ("math", "efficient", "flash"):
        if name.startswith(b) or (b == "efficient" and name.startswith("eff")):
            return b
    raise ValueError(f"unknown SDPA implementation {impl!r}")


def run_impl(cw, impl, Q, K, V, B, nl, ni, warmup, iters, cu_count):
    """Times ``impl``; returns (out[B, nl, D], mean_ms, std_ms, note)."""
    note = ""
    if impl in ("naive", "warp", "tiled", "vectorized"):
        out, mean_ms, std_ms = cw.benchmark_kernel_events(impl, Q, K, V, B, nl, ni, D,
                                                          warmup, iters)
    elif impl == "splitk":
        out, mean_ms, std_ms, s = cw.benchmark_splitk_events(Q, K, V, B, nl, ni, D, warmup,
                                                             iters, num_splits="plan",
                                                             sm_count=cu_count)
        note = f"splits={s}"
    elif impl == "wmma":
        out, mean_ms, std_ms = cw.benchmark_wmma_events(Q, K, V, B, nl, ni, D, warmup, iters)
    elif impl == "wmma_bf16":
        out, mean_ms, std_ms = cw.benchmark_wmma_bf16_events(Q, K, V, B, nl, ni, D, warmup,
                                                             iters)
    elif impl in ("wmma_splitk", "wmma_splitk_bf16"):
        fn = (cw.benchmark_wmma_splitk_bf16_events if impl.endswith("bf16")
              else cw.benchmark_wmma_splitk_events)
        out, mean_ms, std_ms, s = fn(Q, K, V, B, nl, ni, D, warmup, iters, num_splits="plan",
                                     sm_count=cu_count)
        note = f"splits={s}"
    elif impl in ("bmm_fp16", "bmm_bf16"):
        from sdpa_bench import benchmark_bmm_events
        out, mean_ms, std_ms = benchmark_bmm_events(Q, K, V, B, nl, ni, D, precision_of(impl),
                                                    warmup, iters)
        note = "bmm(Q, K^T contiguous) / softmax / bmm"
    elif impl.startswith("sdpa_"):
        from sdpa_bench import benchmark_sdpa_events
        backend, prec = sdpa_backend_of(impl), precision_of(impl)
        out, mean_ms, std_ms = benchmark_sdpa_events(Q, K, V, B, nl, ni, D, backend, prec,
                                                     warmup, iters)
        note = f"{backend}/{prec}"
    else:
        raise ValueError(f"unknown implementation {impl!r}")
    return out, mean_ms, std_ms, note


def errors(out, ref, nl):
    """(max-abs, max-abs / max|ref|) of batch 0 against a [1, nl, D] reference."""
    o0 = out[0] if out.ndim == 3 else out
    r0 = np.asarray(ref).reshape(nl, D)
    max_abs = float(np.max(np.abs(o0 - r0)))
    return max_abs, max_abs / (float(np.max(np.abs(r0))) + 1e-6)


def measure(cw, experiment, gpu, impl, Q, K, V, ref, B, nl, ni, warmup, iters, cu_count,
            tol, use_rel=False):
    """Runs one point; returns the log row (strings, as csvlog writes them).
    ``status`` is 'ok' when the error (max-abs, or relative with use_rel) is
    within ``tol``, 'ACCURACY?' otherwise, 'design-limited' for a shape the
    implementation refuses, and 'error' (note = first line) for a failure."""
    import roofline

    prec = precision_of(impl)
    row = {"experiment": experiment, "gpu": gpu, "impl": impl, "precision": prec,
           "B": B, "N_latent": nl, "N_input": ni, "D": D}
    try:
        out, mean_ms, std_ms, note = run_impl(cw, impl, Q, K, V, B, nl, ni, warmup, iters,
                                              cu_count)
    except cw.DesignLimited as e:
        row.update(status="design-limited", note=str(e)[:120])
        return row
    except Exception as e:  # logged, the sweep goes on
        row.update(status="error", note=(str(e).splitlines() or [repr(e)])[0][:120])
        return row
    max_abs, rel = errors(out, ref, nl)
    materialized = impl.startswith("sdpa_math") or impl.startswith("bmm_")
    out_prec = "fp32" if impl.startswith("wmma") else None
    rl = roofline.roofline_row(B, nl, ni, D, mean_ms / 1e3, gpu, prec,
                               materialized=materialized, out_precision=out_prec)
    ok = (rel if use_rel else max_abs) <= tol
    row.update({
        "latency_ms_mean": f"{mean_ms:.4f}", "latency_ms_std": f"{std_ms:.4f}",
        "achieved_gflops": f"{rl['achieved_gflops']:.1f}",
        "achieved_gbs": f"{rl['achieved_gbs']:.1f}",
        "pct_peak_compute": f"{rl.get('pct_peak_compute') or 0:.2f}",
        "pct_peak_bw": f"{rl.get('pct_peak_bw') or 0:.2f}",
        "arithmetic_intensity": f"{rl['arithmetic_intensity']:.1f}",
        "ridge_point": f"{rl.get('ridge_point') or 0:.1f}",
        "bound": rl.get("bound", ""),
        "max_abs_err": f"{max_abs:.2e}", "rel_err": f"{rel:.2e}",
        "status": "ok" if ok else "ACCURACY?", "note": note,
    })
    return row


def device(cw):
    """(gpu label for the log, gpu_specs key or None, CU count)."""
    from gpu_specs import GPU_SPECS, detect_gpu_name, raw_gpu_name
    key = detect_gpu_name()
    label = key or raw_gpu_name() or "unknown"
    try:
        cu, _ = cw.device_info()
    except Exception:
        cu = GPU_SPECS.get(key, {}).get("sm_count", 256)
    return label, key, cu


def fmt_line(row, cols):
    """One printed table line: (field, width, kind) per column."""
    parts = []
    for field, width, kind in cols:
        v = row.get(field, "")
        if kind == "f" and v not in ("", None):
            v = f"{float(v):.4f}" if field.startswith("latency") else f"{float(v):.1f}"
        parts.append(f"{str(v):>{width}}")
    return "".join(parts)
