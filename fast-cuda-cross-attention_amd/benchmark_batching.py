"""
Batched benchmark of the four fp32 entry points across batch sizes
{4, 8, 16, 32} and N_latent in {64, ..., 1024} (N_input = 784, D = 768),
against data/batches/batch_{B}/N_latent_{n}/, plus throughput in samples/s.

Drop-in for the reference harness (benchmark_batching.py).  Host wall-clock
timing around the legacy drivers (allocation and PCIe copies included), as
in the reference.

    python generate_batch_references.py   # once
    python benchmark_batching.py [--batch-sizes 4 8] [--n-latent 64 128]
"""

import argparse
import os

import numpy as np

import benchmark as single

N_input = 784
D = 768
DATA_DIR = 'data'
BATCHES_DIR = 'batches'

BATCH_SIZES = [4, 8, 16, 32]

N_latent_values = [64, 128, 256, 512, 1024]

verify_output = single.verify_output
benchmark_kernel = single.benchmark_kernel
benchmark_naive = single.benchmark_naive


def load_batch_reference_data(BATCH_SIZE, N_latent):
    """Q, K, V and the reference output for one (batch size, N_latent), or four
    Nones when not generated."""
    subdir = os.path.join(DATA_DIR, BATCHES_DIR, f'batch_{BATCH_SIZE}', f'N_latent_{N_latent}')
    names = ('Q_matrix', 'K_matrix', 'V_matrix', 'output_reference')
    paths = [os.path.join(subdir, n + '.npy') for n in names]
    if not os.path.exists(paths[0]):
        return None, None, None, None
    return tuple(np.load(p) for p in paths)


def run_batch_benchmark(batch_sizes=None, n_latents=None):
    """Every kernel at every (batch size, N_latent): time, verify, tabulate."""
    batch_sizes = batch_sizes or BATCH_SIZES
    n_latents = n_latents or N_latent_values
    bar = "=" * 80
    print(bar)
    print("Perceiver Cross-Attention HIP Kernel Benchmark - Batch Size Analysis (MI355X)")
    print(bar)
    print(f"Fixed dimensions:\n  N_input:  {N_input}\n  D:         {D}")
    print(f"\nBatch sizes: {batch_sizes}\nN_latent values: {n_latents}")
    print(bar)
    if not single.CUDA_AVAILABLE:
        print("\nHIP kernels not available. Cannot run benchmarks.")
        return None

    import cuda_wrappers
    all_results = {}
    for B in batch_sizes:
        print(f"\n{bar}\nBatch Size = {B}\n{bar}")
        res = {'N_latent': []}
        res.update({key: [] for key, *_ in single.KERNELS})
        for N_latent in n_latents:
            Q, K, V, reference = load_batch_reference_data(B, N_latent)
            if Q is None:
                print(f"  Missing data/{BATCHES_DIR}/batch_{B}/N_latent_{N_latent}/ -- run "
                      f"'python generate_batch_references.py'")
                continue
            print(f"\n  N_latent = {N_latent}")
            res['N_latent'].append(N_latent)
            for key, name, driver, tol, short in single.KERNELS:
                try:
                    if short:
                        out, ms = benchmark_naive(Q, K, V, N_latent, N_input, D)
                    else:
                        out, ms = benchmark_kernel(getattr(cuda_wrappers, driver), Q, K, V,
                                                   N_latent, N_input, D)
                except Exception as e:
                    print(f"    {name}: Error: {e}")
                    res[key].append(None)
                    continue
                res[key].append(ms)
                print(f"    {name}: {ms:.3f} ms ({B / (ms / 1000.0):.1f} samples/sec)")
                verify_output(out, reference, name, tolerance=1e-3 if not short else 5e-3)
        single._print_tables(res, f'N_latent (batch {B})')
        print(f"\nThroughput (samples/sec), batch {B}")
        print(f"{'N_latent':<12} {'Naive':<15} {'Warp Parallel':<18} {'Tiled':<15} {'Vectorized':<18}")
        for i, nl in enumerate(res['N_latent']):
            thr = [(B / (res[k][i] / 1000.0)) if res[k][i] else 0.0
                   for k in ('naive', 'parallel', 'tiled', 'optimized')]
            print(f"{nl:<12} {thr[0]:<15.1f} {thr[1]:<18.1f} {thr[2]:<15.1f} {thr[3]:<18.1f}")
        all_results[B] = res
    return all_results


def main():
    parser = argparse.ArgumentParser(
        description='Benchmark the HIP kernel ladder across batch sizes')
    parser.add_argument('--batch-sizes', type=int, nargs='+', default=None)
    parser.add_argument('--n-latent', type=int, nargs='+', default=None)
    args = parser.parse_args()
    run_batch_benchmark(args.batch_sizes, args.n_latent)


if __name__ == "__main__":
    main()
