"""
Perceiver N_input sweep: N_latent fixed at the bottleneck, N_input over image
sizes 784 = 28^2 .. 50176 = 224^2, each implementation timed with HIP events
on resident data (the reference's experiments/bench_perceiver_ni.py).  The
wave-per-latent kernel keeps its whole score row in LDS and is expected to
report 'design-limited' once N_input outgrows it; that truncation is part of
the result.

One log row per (impl, N_input) with latency, roofline columns and the error
against the float32 reference of gen_perceiver_refs.py.  Runs from anywhere:
paths resolve against the package directory (kernels.so, data/, results/).

    python experiments/bench_perceiver_ni.py
    python experiments/bench_perceiver_ni.py --n-latent 64 \\
        --n-input 784 3136 12544 50176 --impls vectorized splitk wmma_bf16 sdpa_math
"""

import argparse
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
DEFAULT_NI = [784, 3136, 12544, 50176]
DEFAULT_IMPLS = ["warp", "tiled", "vectorized"]

COLS = [("impl", 18, "s"), ("N_input", 7, "s"), ("latency_ms_mean", 11, "f"),
        ("achieved_gflops", 11, "f"), ("achieved_gbs", 9, "f"), ("pct_peak_compute", 7, "s"),
        ("pct_peak_bw", 7, "s"), ("bound", 8, "s"), ("max_abs_err", 10, "s"),
        ("status", 15, "s")]


def main(argv=None):
    ap = argparse.ArgumentParser(description="Perceiver N_input sweep (HIP events)")
    ap.add_argument("--n-latent", type=int, default=64)
    ap.add_argument("--n-input", type=int, nargs="+", default=DEFAULT_NI)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--impls", nargs="+", default=DEFAULT_IMPLS)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--iters", type=int, default=100)
    ap.add_argument("--tol", type=float, default=1e-2)
    ap.add_argument("--data", default="data")
    ap.add_argument("--csv", default="results/perceiver_ni.csv")
    args = ap.parse_args(argv)

    os.chdir(ROOT)
    sys.path.insert(0, HERE)
    sys.path.insert(0, ROOT)
    import csvlog
    import sweep
    from gen_perceiver_refs import load_case
    try:
        import cuda_wrappers as cw
    except Exception as e:
        print(f"Could not load kernels.so ({e}); build it with `make` in {ROOT}.")
        return 1

    gpu, _, cu = sweep.device(cw)
    nl, B = args.n_latent, args.batch
    csv_path = os.path.join(ROOT, args.csv)
    os.makedirs(os.path.dirname(csv_path), exist_ok=True)
    fh, w = csvlog.writer(csv_path)
    print(f"Perceiver N_input sweep | GPU={gpu} ({cu} CUs) | N_latent={nl} | B={B} | "
          f"warmup={args.warmup} iters={args.iters}")
    header = "".join(f"{c[0][:c[1] - 1]:>{c[1]}}" for c in COLS)
    print(header)
    print("-" * len(header))
    try:
        for ni in args.n_input:
            case = load_case(args.data, nl, ni)
            if case is None:
                print(f"{'(all)':>18}{ni:>7}   missing reference: run gen_perceiver_refs.py "
                      f"--n-latent {nl} --n-input {ni}")
                continue
            Q, K, V, ref = case
            for impl in args.impls:
                row = sweep.measure(cw, "perceiver_ni", gpu, impl, Q, K, V, ref, B, nl, ni,
                                    args.warmup, args.iters, cu, args.tol)
                print(sweep.fmt_line(row, COLS)
                      + (f"  {row['note']}" if row.get("status") != "ok" else ""))
                w.writerow(row)
    finally:
        fh.close()
    print(f"CSV -> {csv_path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
