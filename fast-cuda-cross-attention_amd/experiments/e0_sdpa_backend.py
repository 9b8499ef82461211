"""
Which PyTorch-ROCm SDPA backends run single-head attention at head_dim 768?
(the reference's experiments/e0_sdpa_backend.py)

Fused flash kernels cap the head dimension, so at D = 768 the framework
baseline is whichever backend still accepts the shape.  Each backend is
forced in turn at the anchor point (B = 1, N_latent = 256, N_input = 4096) in
fp32, fp16 and bf16; a run is timed with events, a refusal is logged with
its message.  16-bit 'math' is not run (switched off, see sdpa_bench.py) and
is logged as such; the hand-written materialized product (bmm_fp16 /
bmm_bf16) is timed in its place under its own name.  Off a GPU box the
script says so and exits 0.

    python experiments/e0_sdpa_backend.py
    python experiments/e0_sdpa_backend.py --n-latent 256 --n-input 4096 --csv results/e0.csv
"""

import argparse
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
D = 768
PROBES = [
    ("sdpa_flash", "flash", ("fp16", "bf16")),
    ("sdpa_efficient", "efficient", ("fp32", "fp16", "bf16")),
    ("sdpa_math", "math", ("fp32", "fp16", "bf16")),
    ("bmm", None, ("fp16", "bf16")),
]


def probe(nl, ni, warmup, iters):
    """[(impl, precision, status, mean_ms, std_ms, note)] for every probe."""
    import math

    import torch
    from sdpa_bench import (MATH_16BIT_OFF, materialized_bmm, sdpa_callable, time_events,
                            torch_dtype)

    results = []
    scale = 1.0 / math.sqrt(D)
    gen = torch.Generator(device="cuda").manual_seed(0)
    for impl, backend, precisions in PROBES:
        for prec in precisions:
            if backend == "math" and prec != "fp32":
                results.append((impl, prec, "switched-off", None, None, MATH_16BIT_OFF[:160]))
                continue
            dt = torch_dtype(prec)
            q = torch.randn(1, 1, nl, D, device="cuda", generator=gen).to(dt)
            k = torch.randn(1, 1, ni, D, device="cuda", generator=gen).to(dt)
            v = torch.randn(1, 1, ni, D, device="cuda", generator=gen).to(dt)
            fn = materialized_bmm if backend is None else sdpa_callable(backend, prec)
            try:
                fn(q, k, v, scale)
                times = time_events(lambda: fn(q, k, v, scale), warmup, iters)
                mean = sum(times) / len(times)
                std = (sum((t - mean) ** 2 for t in times) / len(times)) ** 0.5
                results.append((impl, prec, "ok", mean, std, ""))
            except Exception as e:
                msg = (str(e).strip().splitlines() or [repr(e)])[0][:160]
                results.append((impl, prec, "unsupported", None, None, msg))
            del q, k, v
            torch.cuda.empty_cache()
    return results


def main(argv=None):
    ap = argparse.ArgumentParser(description="SDPA backends at head_dim 768")
    ap.add_argument("--n-latent", type=int, default=256)
    ap.add_argument("--n-input", type=int, default=4096)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--iters", type=int, default=100)
    ap.add_argument("--csv", default="results/e0_sdpa_backend.csv")
    args = ap.parse_args(argv)

    sys.path.insert(0, HERE)
    import csvlog
    try:
        import torch
    except ImportError:
        print("PyTorch is not installed; nothing to probe.")
        return 0
    if not torch.cuda.is_available():
        print("No GPU visible: the SDPA backend probe runs on the GPU box.")
        return 0
    from gpu_specs import detect_gpu_name

    gpu = detect_gpu_name() or torch.cuda.get_device_name(0)
    print(f"SDPA backends at head_dim={D} | {torch.cuda.get_device_name(0)} (key {gpu}) | "
          f"torch {torch.__version__} | B=1 N_latent={args.n_latent} N_input={args.n_input}")
    os.makedirs(os.path.dirname(args.csv) or ".", exist_ok=True)
    fh, w = csvlog.writer(args.csv)
    try:
        for impl, prec, status, mean, std, note in probe(args.n_latent, args.n_input,
                                                         args.warmup, args.iters):
            if status == "ok":
                print(f"  {impl:16s} {prec:5s} ok   {mean:8.3f} +/- {std:.3f} ms")
            else:
                print(f"  {impl:16s} {prec:5s} --   {note}")
            w.writerow({"experiment": "e0", "gpu": gpu, "impl": impl, "precision": prec,
                        "B": 1, "N_latent": args.n_latent, "N_input": args.n_input, "D": D,
                        "latency_ms_mean": f"{mean:.4f}" if mean is not None else "",
                        "latency_ms_std": f"{std:.4f}" if std is not None else "",
                        "status": status, "note": note})
    finally:
        fh.close()
    print(f"CSV -> {args.csv}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
