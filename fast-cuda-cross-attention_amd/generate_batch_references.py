"""
Writes data/batches/batch_{B}/N_latent_{n}/ for the batched harness
(benchmark_batching.py); see generate_references.py for the format.

    python generate_batch_references.py [--out data] [--batch-sizes 4 8 16 32]
"""

import argparse

from generate_references import BATCH_SIZES, D, DATA_DIR, N_input, N_latent_values, write_batched


def main():
    ap = argparse.ArgumentParser(description="Generate batched reference data")
    ap.add_argument('--out', default=DATA_DIR)
    ap.add_argument('--batch-sizes', type=int, nargs='+', default=BATCH_SIZES)
    ap.add_argument('--n-latent', type=int, nargs='+', default=N_latent_values)
    args = ap.parse_args()
    print(f"Generating batched references: N_input={N_input} D={D} "
          f"B={args.batch_sizes} N_latent={args.n_latent}")
    write_batched(args.out, args.batch_sizes, args.n_latent)


if __name__ == "__main__":
    main()
