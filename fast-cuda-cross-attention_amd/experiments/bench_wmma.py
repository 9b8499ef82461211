"""
16-bit MFMA against the fp32 kernel (the reference's experiments/bench_wmma.py):
for each N_input, the fp32 'vectorized' entry point and the fused fp16 (and
bf16) MFMA entry points, with the speed-up over fp32 and the relative error
(max-abs / max|ref|) against the float32 reference.  Unlike the reference's
kernel these take any N_latent and N_input.

    python experiments/bench_wmma.py
    python experiments/bench_wmma.py --n-latent 256 --n-input 784 3136 12544 50176 \\
        --impls wmma wmma_bf16 wmma_splitk_bf16
"""

import argparse
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)

COLS = [("impl", 18, "s"), ("precision", 6, "s"), ("N_input", 7, "s"),
        ("latency_ms_mean", 11, "f"), ("achieved_gflops", 11, "f"),
        ("pct_peak_compute", 8, "s"), ("speedup", 9, "s"), ("rel_err", 10, "s"),
        ("status", 12, "s")]


def main(argv=None):
    ap = argparse.ArgumentParser(description="16-bit MFMA vs fp32")
    ap.add_argument("--n-latent", type=int, default=256)
    ap.add_argument("--n-input", type=int, nargs="+", default=[784, 3136, 12544, 50176])
    ap.add_argument("--impls", nargs="+", default=["wmma", "wmma_bf16"])
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--iters", type=int, default=100)
    ap.add_argument("--rtol", type=float, default=5e-2)
    ap.add_argument("--data", default="data")
    ap.add_argument("--csv", default="results/e7_wmma.csv")
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
    nl = args.n_latent
    csv_path = os.path.join(ROOT, args.csv)
    os.makedirs(os.path.dirname(csv_path), exist_ok=True)
    fh, w = csvlog.writer(csv_path)
    print(f"16-bit MFMA vs fp32 | GPU={gpu} ({cu} CUs) | N_latent={nl}")
    header = "".join(f"{c[0][:c[1] - 1]:>{c[1]}}" for c in COLS)
    print(header)
    print("-" * len(header))
    try:
        for ni in args.n_input:
            case = load_case(args.data, nl, ni)
            if case is None:
                print(f"{'(missing ref)':>18}{'':>6}{ni:>7}  run gen_perceiver_refs.py "
                      f"--n-latent {nl} --n-input {ni}")
                continue
            Q, K, V, ref = case
            base = sweep.measure(cw, "e7_wmma", gpu, "vectorized", Q, K, V, ref, 1, nl, ni,
                                 args.warmup, args.iters, cu, args.rtol, use_rel=True)
            base_ms = float(base["latency_ms_mean"]) if base.get("latency_ms_mean") else None
            print(sweep.fmt_line(dict(base, speedup="1.00x" if base_ms else ""), COLS))
            w.writerow(base)
            for impl in args.impls:
                row = sweep.measure(cw, "e7_wmma", gpu, impl, Q, K, V, ref, 1, nl, ni,
                                    args.warmup, args.iters, cu, args.rtol, use_rel=True)
                sp = ""
                if base_ms and row.get("latency_ms_mean"):
                    sp = f"{base_ms / float(row['latency_ms_mean']):.2f}x"
                print(sweep.fmt_line(dict(row, speedup=sp), COLS)
                      + (f"  {row['note']}" if row.get("status") not in ("ok",) else ""))
                w.writerow(row)
    finally:
        fh.close()
    print(f"CSV -> {csv_path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
