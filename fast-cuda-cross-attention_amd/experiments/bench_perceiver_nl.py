"""
Perceiver N_latent sweep (occupancy): N_input fixed at a small, L2-resident
size (default 3136 = 56^2), N_latent swept, as in the reference's
experiments/bench_perceiver_nl.py.  The workgroup count of each kernel grows
with N_latent, so small N_latent cannot fill the 256 CUs; each row records
the workgroups the implementation launches and how many CUs they can occupy.

Workgroups per call: naive ceil(Nl/4)*B*12 (64-column blocks); warp and
tiled ceil(Nl/4)*B; vectorized ceil(Nl/64)*B times the key splits it plans
when that alone would leave CUs idle; splitk ceil(Nl/64)*B*S; the 16-bit
entry points ceil(Nl/64 or Nl/32)*B times their planned splits (wmma_plan).  act_cu =
min(workgroups, CUs) is the number of CUs that get any work.

    python experiments/bench_perceiver_nl.py
    python experiments/bench_perceiver_nl.py --n-input 3136 \\
        --n-latent 16 32 64 128 256 512 1024 --impls warp tiled vectorized splitk
"""

import argparse
import math
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
DEFAULT_NL = [16, 32, 64, 128, 256, 512, 1024]
DEFAULT_IMPLS = ["warp", "tiled", "vectorized"]

COLS = [("impl", 18, "s"), ("N_latent", 7, "s"), ("blocks", 8, "s"), ("act_cu", 7, "s"),
        ("latency_ms_mean", 11, "f"), ("achieved_gflops", 11, "f"),
        ("pct_peak_compute", 7, "s"), ("pct_peak_bw", 7, "s"), ("max_abs_err", 10, "s"),
        ("status", 15, "s")]


def workgroups(cw, impl, B, nl, ni, cu):
    """Workgroups one call of ``impl`` launches (before its combine pass)."""
    if impl in ("warp", "tiled"):
        return math.ceil(nl / 4) * B
    if impl == "naive":
        return math.ceil(nl / 4) * B * math.ceil(768 / 64)
    rows = math.ceil(nl / cw.LATENTS_PER_WORKGROUP) * B
    if impl == "vectorized":
        lpw, s = cw.f32_plan(B, nl, ni, cu)
        return math.ceil(nl / lpw) * B * s
    if impl == "splitk":
        s = cw.plan_num_splits(nl, ni, B, cu)
        return math.ceil(nl / cw.lib.xattn_f32_split_latents(B, nl, ni, s, cu)) * B * s
    if impl.startswith("wmma_splitk"):
        s = cw.plan_num_splits(nl, ni, B, cu, cw.KEYS_PER_TILE_F16)
        return math.ceil(nl / cw.lib.xattn_wmma_split_latents(B, nl, ni, s, cu)) * B * s
    if impl.startswith("wmma"):
        lpw, s = cw.wmma_plan(B, nl, ni, cu)
        return math.ceil(nl / lpw) * B * s
    return rows


def main(argv=None):
    ap = argparse.ArgumentParser(description="Perceiver N_latent sweep (occupancy)")
    ap.add_argument("--n-input", type=int, default=3136)
    ap.add_argument("--n-latent", type=int, nargs="+", default=DEFAULT_NL)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--impls", nargs="+", default=DEFAULT_IMPLS)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--iters", type=int, default=100)
    ap.add_argument("--tol", type=float, default=1e-2)
    ap.add_argument("--data", default="data")
    ap.add_argument("--csv", default="results/perceiver_nl.csv")
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
    ni, B = args.n_input, args.batch
    csv_path = os.path.join(ROOT, args.csv)
    os.makedirs(os.path.dirname(csv_path), exist_ok=True)
    fh, w = csvlog.writer(csv_path)
    print(f"Perceiver N_latent sweep | GPU={gpu} ({cu} CUs) | N_input={ni} | B={B} | "
          f"warmup={args.warmup} iters={args.iters}")
    header = "".join(f"{c[0][:c[1] - 1]:>{c[1]}}" for c in COLS)
    print(header)
    print("-" * len(header))
    try:
        for nl in args.n_latent:
            case = load_case(args.data, nl, ni)
            if case is None:
                print(f"{'(all)':>18}{nl:>7}   missing reference: run gen_perceiver_refs.py "
                      f"--n-latent {nl} --n-input {ni}")
                continue
            Q, K, V, ref = case
            for impl in args.impls:
                blocks = workgroups(cw, impl, B, nl, ni, cu)
                act = min(blocks, cu)
                row = sweep.measure(cw, "perceiver_nl", gpu, impl, Q, K, V, ref, B, nl, ni,
                                    args.warmup, args.iters, cu, args.tol)
                row["note"] = ";".join(x for x in (f"blocks={blocks}", f"act_cu={act}",
                                                   row.get("note", "")) if x)
                print(sweep.fmt_line(dict(row, blocks=blocks, act_cu=act), COLS))
                w.writerow(row)
    finally:
        fh.close()
    print(f"CSV -> {csv_path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
