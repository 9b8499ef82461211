"""
The materialized-vs-fused comparison at the reference's anchor point
(report/comparison_table.tex:26-38: B = 1, N_latent = 256, N_input = 4096,
head_dim 768): this library's kernels against every PyTorch-ROCm SDPA
backend that accepts the shape (SDPA math in fp32; in fp16 / bf16 the
hand-written materialized product bmm_fp16 / bmm_bf16 stands in, since
16-bit SDPA math is switched off), each timed with events on resident data and
checked against the float64 reference.  Prints a markdown table sorted by
latency, with each row's speed relative to fp32 SDPA-math, and appends the
rows to the log.

    python experiments/compare_sdpa.py
    python experiments/compare_sdpa.py --n-latent 256 --n-input 4096 --md results/anchor.md
"""

import argparse
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)

IMPLS = [
    ("sdpa_math", "materialized (hipBLASLt GEMMs)"),
    ("bmm_fp16", "materialized bmm/softmax/bmm (contiguous K^T), fp16; not SDPA"),
    ("bmm_bf16", "materialized bmm/softmax/bmm (contiguous K^T), bf16; not SDPA"),
    ("sdpa_efficient", "fused"),
    ("sdpa_efficient_fp16", "fused, fp16"),
    ("sdpa_efficient_bf16", "fused, bf16"),
    ("sdpa_flash_fp16", "fused flash, fp16"),
    ("sdpa_flash_bf16", "fused flash, bf16"),
    ("vectorized", "fused, fp32 MFMA (this library)"),
    ("splitk", "fused, key-parallel fp32 MFMA (this library)"),
    ("wmma", "fused, fp16 MFMA (this library)"),
    ("wmma_splitk", "fused, key-parallel fp16 MFMA (this library)"),
    ("wmma_bf16", "fused, bf16 MFMA (this library)"),
    ("wmma_splitk_bf16", "fused, key-parallel bf16 MFMA (this library)"),
]


def table(rows, kinds):
    """Markdown table of the measured rows (fastest first) and the refused ones."""
    base = next((float(r["latency_ms_mean"]) for r in rows
                 if r["impl"] == "sdpa_math" and r.get("latency_ms_mean")), None)
    ran = sorted((r for r in rows if r.get("latency_ms_mean")),
                 key=lambda r: float(r["latency_ms_mean"]))
    out = ["| Implementation | Type | Precision | Latency (ms) | GFLOP/s | x SDPA-math fp32 "
           "| rel err |",
           "|---|---|---|---:|---:|---:|---:|"]
    for r in ran:
        ms = float(r["latency_ms_mean"])
        rel = f"{base / ms:.2f}" if base else "n/a"
        out.append(f"| {r['impl']} | {kinds[r['impl']]} | {r['precision']} | {ms:.4f} | "
                   f"{float(r['achieved_gflops']):.0f} | {rel} | {r['rel_err']} |")
    refused = [r for r in rows if not r.get("latency_ms_mean")]
    if refused:
        out.append("")
        out.append("Not run at this shape:")
        for r in refused:
            out.append(f"- {r['impl']} ({r['precision']}): {r['status']}: {r.get('note', '')}")
    return "\n".join(out)


def main(argv=None):
    ap = argparse.ArgumentParser(description="Materialized vs fused at the anchor point")
    ap.add_argument("--n-latent", type=int, default=256)
    ap.add_argument("--n-input", type=int, default=4096)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--iters", type=int, default=100)
    ap.add_argument("--impls", nargs="+", default=[i for i, _ in IMPLS])
    ap.add_argument("--csv", default="results/anchor_comparison.csv")
    ap.add_argument("--md", default=None, help="also write the table to this file")
    args = ap.parse_args(argv)

    os.chdir(ROOT)
    sys.path.insert(0, HERE)
    sys.path.insert(0, ROOT)
    import csvlog
    import sweep
    from gen_perceiver_refs import draw, reference_output
    try:
        import cuda_wrappers as cw
    except Exception as e:
        print(f"Could not load kernels.so ({e}); build it with `make` in {ROOT}.")
        return 1

    gpu, _, cu = sweep.device(cw)
    nl, ni = args.n_latent, args.n_input
    Q, K, V = draw(nl, ni)
    ref = reference_output(Q, K, V).reshape(1, nl, sweep.D)
    kinds = dict(IMPLS)
    rows = []
    csv_path = os.path.join(ROOT, args.csv)
    os.makedirs(os.path.dirname(csv_path), exist_ok=True)
    fh, w = csvlog.writer(csv_path)
    try:
        for impl in args.impls:
            tol = 1e-3 if sweep.precision_of(impl) == "fp32" else 2e-2
            row = sweep.measure(cw, "anchor", gpu, impl, Q, K, V, ref, 1, nl, ni,
                                args.warmup, args.iters, cu, tol, use_rel=True)
            print(f"  {impl:22s} {row.get('latency_ms_mean') or row['status']:>10}  "
                  f"{row.get('note', '')}", flush=True)
            rows.append(row)
            w.writerow(row)
    finally:
        fh.close()
    text = (f"Anchor: B=1, N_latent={nl}, N_input={ni}, head_dim={sweep.D}, GPU={gpu}\n\n"
            + table(rows, kinds))
    print(text)
    if args.md:
        with open(args.md, "w") as f:
            f.write(text + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
