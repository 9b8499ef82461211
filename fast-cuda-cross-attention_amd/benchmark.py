"""
Single-batch benchmark of the four fp32 entry points (naive, warp-parallel,
tiled, vectorized) across N_latent in {64, ..., 1024} with N_input = 784 and
D = 768, against the pre-generated references in data/N_latent_*/.

Drop-in for the reference harness (benchmark.py): same functions, data layout
and report tables.  Timing here is host wall-clock around the legacy
``run_*_kernel`` drivers, i.e. it includes hipMalloc, PCIe copies and hipFree
exactly as the reference's does; kernel-only timing lives in
``cuda_wrappers.benchmark_kernel_events`` and the repository's bench.py.

    python generate_references.py   # once, writes data/N_latent_*/
    python benchmark.py
"""

import argparse
import os
import time

import numpy as np

try:
    from cuda_wrappers import (
        run_naive_kernel,
        run_warp_parallel_kernel,
        run_tiled_kernel,
        run_vectorized_kernel,
    )
    CUDA_AVAILABLE = True
except (ImportError, RuntimeError) as e:
    print(f"Warning: HIP kernels not available: {e}")
    print("Run 'make' to compile the kernels.")
    CUDA_AVAILABLE = False

N_input = 784
D = 768
DATA_DIR = 'data'

N_latent_values = [64, 128, 256, 512, 1024]

# (result key, display name, driver name, tolerance, use the short naive loop)
KERNELS = [
    ('naive', 'Naive', 'run_naive_kernel', 5e-3, True),
    ('parallel', 'Warp Parallel', 'run_warp_parallel_kernel', 1e-3, False),
    ('tiled', 'Tiled', 'run_tiled_kernel', 1e-3, False),
    ('optimized', 'Vectorized', 'run_vectorized_kernel', 1e-3, False),
]


def verify_output(output, reference, name, tolerance=5e-3):
    """Report whether ``output`` matches ``reference`` to ``tolerance`` (max
    abs difference).  Prints the verdict and returns it; never raises."""
    diff = np.abs(np.asarray(output, np.float64) - np.asarray(reference, np.float64))
    worst, mean = float(diff.max()), float(diff.mean())
    if worst > tolerance:
        print(f"  {name}: WARNING - Max difference {worst:.6f} exceeds tolerance {tolerance}")
        print(f"    Mean difference: {mean:.6f}")
        return False
    print(f"  {name}: Verification passed (max diff: {worst:.6f}, mean diff: {mean:.6f})")
    return True


def _timed(fn, args, iterations, warmup):
    for _ in range(warmup):
        fn(*args)
    t0 = time.time()
    for _ in range(iterations):
        out = fn(*args)
    return out, (time.time() - t0) / iterations * 1000.0


def benchmark_kernel(kernel_func, Q, K, V, N_latent, N_input, D, num_iterations=100, warmup=10):
    """Mean host wall-clock ms per call of a legacy driver."""
    return _timed(kernel_func, (Q, K, V, N_latent, N_input, D), num_iterations, warmup)


def benchmark_naive(Q, K, V, N_latent, N_input, D):
    """The naive kernel is slow: 3 warmup calls and 10 timed ones."""
    return _timed(run_naive_kernel, (Q, K, V, N_latent, N_input, D), 10, 3)


def load_reference_data(N_latent):
    """Q, K, V and the reference output from data/N_latent_{N_latent}/, or four
    Nones when the directory has not been generated."""
    subdir = os.path.join(DATA_DIR, f'N_latent_{N_latent}')
    names = ('Q_matrix', 'K_matrix', 'V_matrix', 'output_reference')
    paths = [os.path.join(subdir, n + '.npy') for n in names]
    if not os.path.exists(paths[0]):
        return None, None, None, None
    return tuple(np.load(p) for p in paths)


def _print_tables(results, label_first):
    cols = [('naive', 'Naive'), ('parallel', 'Warp Parallel'), ('tiled', 'Tiled'),
            ('optimized', 'Vectorized')]
    bar = "=" * 80
    print(f"\n{bar}\nPerformance Summary - All Kernels Across All {label_first} Values\n{bar}")
    print(f"{'N_latent':<12} {'Naive (ms)':<15} {'Warp Parallel (ms)':<20} "
          f"{'Tiled (ms)':<15} {'Vectorized (ms)':<18}")
    print("-" * 80)
    for i, nl in enumerate(results['N_latent']):
        vals = [results[k][i] if results[k][i] is not None else float('inf') for k, _ in cols]
        print(f"{nl:<12} {vals[0]:<15.3f} {vals[1]:<20.3f} {vals[2]:<15.3f} {vals[3]:<18.3f}")

    print(f"\n{bar}\nOptimization Speedups (vs Naive)\n{bar}")
    print(f"{'N_latent':<12} {'Warp Parallel':<18} {'Tiled':<15} {'Vectorized':<18}")
    print("-" * 80)
    for i, nl in enumerate(results['N_latent']):
        base = results['naive'][i]
        if not base:
            continue
        sp = [base / results[k][i] if results[k][i] else 0.0 for k, _ in cols[1:]]
        print(f"{nl:<12} {sp[0]:<18.2f} {sp[1]:<15.2f} {sp[2]:<18.2f}")

    print(f"\n{bar}\nScaling Analysis - Time per Latent Vector (μs)\n{bar}")
    print(f"{'N_latent':<12} {'Naive':<15} {'Warp Parallel':<18} {'Tiled':<15} {'Vectorized':<18}")
    print("-" * 80)
    for i, nl in enumerate(results['N_latent']):
        per = [(results[k][i] * 1000.0 / nl) if results[k][i] is not None else 0.0
               for k, _ in cols]
        print(f"{nl:<12} {per[0]:<15.2f} {per[1]:<15.2f} {per[2]:<15.2f} {per[3]:<15.2f}")
    print(bar)


def run_unified_benchmark():
    """All four kernels at every N_latent: time, verify, and tabulate."""
    bar = "=" * 80
    print(bar)
    print("Perceiver Cross-Attention HIP Kernel Benchmark (MI355X)")
    print("Optimization Comparison & Scaling Analysis")
    print(bar)
    print(f"Fixed dimensions:\n  N_input:  {N_input}\n  D:         {D}")
    print(f"\nTesting N_latent values: {N_latent_values}")
    print("Kernels: Naive, Warp Parallel, Tiled, Vectorized")
    print("Reference verification: Using pre-generated references from data/ subdirectories")
    print(bar)

    if not CUDA_AVAILABLE:
        print("\nHIP kernels not available. Cannot run benchmarks.")
        return None

    missing = [n for n in N_latent_values
               if not os.path.exists(os.path.join(DATA_DIR, f'N_latent_{n}',
                                                  'output_reference.npy'))]
    if missing:
        print(f"\nError: Pre-generated reference data not found for N_latent values: {missing}")
        print("Please run 'python generate_references.py' to generate the required reference data.")
        return None

    import cuda_wrappers
    results = {'N_latent': []}
    results.update({key: [] for key, *_ in KERNELS})
    for N_latent in N_latent_values:
        print(f"\n{bar}\nN_latent = {N_latent}\n{bar}")
        Q, K, V, reference = load_reference_data(N_latent)
        if reference.ndim == 2:
            reference = reference.reshape(1, N_latent, D)
        print(f"  Loaded pre-generated Q, K, V and reference from data/N_latent_{N_latent}/")
        results['N_latent'].append(N_latent)
        for key, name, driver, tol, short in KERNELS:
            print(f"\n  {name}...")
            try:
                if short:
                    out, ms = benchmark_naive(Q, K, V, N_latent, N_input, D)
                else:
                    out, ms = benchmark_kernel(getattr(cuda_wrappers, driver), Q, K, V,
                                               N_latent, N_input, D)
            except Exception as e:  # record and continue, as the reference does
                print(f"    Error: {e}")
                results[key].append(None)
                continue
            results[key].append(ms)
            print(f"    Time: {ms:.3f} ms")
            base = results['naive'][-1]
            if key != 'naive' and base:
                print(f"    Speedup over Naive: {base / ms:.2f}")
            verify_output(out, reference, name, tolerance=tol)
    _print_tables(results, 'N_latent')
    return results


def main():
    parser = argparse.ArgumentParser(
        description='Benchmark the HIP kernel ladder with optimization and scaling analysis',
        formatter_class=argparse.RawDescriptionHelpFormatter,
        epilog="Tests all 4 kernels (Naive, Warp Parallel, Tiled, Vectorized) across\n"
               "N_latent in {64..1024}.\n\nExample:\n  python benchmark.py")
    parser.parse_args()
    run_unified_benchmark()


if __name__ == "__main__":
    main()
