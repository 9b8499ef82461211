"""
Writes the harness's reference data: Q, K, V (seed-42 normal draws) and the
PyTorch CPU output of softmax(Q K^T / sqrt(D)) V for every N_latent, as

    data/N_latent_{n}/{Q,K,V}_matrix.npy, output_reference.npy          (B = 1)
    data/batches/batch_{B}/N_latent_{n}/...                              (batched)

Same directory layout, file names, seed and draw order (Q, then K, then V from
``np.random.seed(42)``) as the reference's generate_references.py:25-68 and
generate_batch_references.py:28-81, so benchmark.py / benchmark_batching.py
find their data.  The output is float32 computed on the CPU.

    python generate_references.py [--out data] [--n-latent 64 128 ...]
"""

import argparse
import math
import os

import numpy as np

N_input = 784
D = 768
DATA_DIR = 'data'
BATCHES_DIR = 'batches'
SEED = 42

N_latent_values = [64, 128, 256, 512, 1024]
BATCH_SIZES = [4, 8, 16, 32]


def compute_cross_attention(Q, K, V, D):
    """softmax(Q K^T / sqrt(D)) V for [B, N, D] torch tensors (CPU, float32)."""
    import torch
    scores = torch.bmm(Q, K.transpose(1, 2).contiguous()) / math.sqrt(D)
    return torch.bmm(torch.softmax(scores, dim=-1), V)


def _draw(shape_q, shape_kv, seed):
    np.random.seed(seed)
    Q = np.random.randn(*shape_q).astype(np.float32)
    K = np.random.randn(*shape_kv).astype(np.float32)
    V = np.random.randn(*shape_kv).astype(np.float32)
    return Q, K, V


def generate_reference_for_size(N_latent, N_input, D, seed=SEED):
    """B = 1 case: 2-D Q/K/V and a [1, N_latent, D] reference output."""
    import torch
    Q, K, V = _draw((N_latent, D), (N_input, D), seed)
    out = compute_cross_attention(*(torch.from_numpy(a)[None] for a in (Q, K, V)), D)
    return Q, K, V, out.numpy().astype(np.float32).reshape(1, N_latent, D)


def generate_reference_for_batch_size(BATCH_SIZE, N_latent, N_input, D, seed=SEED):
    """Batched case: 3-D Q/K/V and a [B, N_latent, D] reference output."""
    import torch
    Q, K, V = _draw((BATCH_SIZE, N_latent, D), (BATCH_SIZE, N_input, D), seed)
    out = compute_cross_attention(*(torch.from_numpy(a) for a in (Q, K, V)), D)
    return Q, K, V, out.numpy().astype(np.float32)


def _save(subdir, Q, K, V, out):
    os.makedirs(subdir, exist_ok=True)
    for name, arr in (('Q_matrix', Q), ('K_matrix', K), ('V_matrix', V),
                      ('output_reference', out)):
        np.save(os.path.join(subdir, name + '.npy'), arr)


def write_single(out_dir=DATA_DIR, n_latents=N_latent_values):
    for nl in n_latents:
        sub = os.path.join(out_dir, f'N_latent_{nl}')
        _save(sub, *generate_reference_for_size(nl, N_input, D, SEED))
        print(f"  wrote {sub}/")


def write_batched(out_dir=DATA_DIR, batch_sizes=BATCH_SIZES, n_latents=N_latent_values):
    for b in batch_sizes:
        for nl in n_latents:
            sub = os.path.join(out_dir, BATCHES_DIR, f'batch_{b}', f'N_latent_{nl}')
            _save(sub, *generate_reference_for_batch_size(b, nl, N_input, D, SEED))
            print(f"  wrote {sub}/")


def main():
    ap = argparse.ArgumentParser(description="Generate single-batch reference data")
    ap.add_argument('--out', default=DATA_DIR)
    ap.add_argument('--n-latent', type=int, nargs='+', default=N_latent_values)
    args = ap.parse_args()
    print(f"Generating references: N_input={N_input} D={D} N_latent={args.n_latent}")
    write_single(args.out, args.n_latent)


if __name__ == "__main__":
    main()
