"""
Writes the Perceiver sweep data: a fixed, small bank of latents attending to
inputs of image sizes 784 = 28^2 (MNIST) .. 50176 = 224^2 (ImageNet).

    <out>/perceiver/Nl{Nl}_Ni{Ni}/{Q,K,V}_matrix.npy    float32 [Nl|Ni, 768]
    <out>/perceiver/Nl{Nl}_Ni{Ni}/output_reference.npy  float32 [1, Nl, 768]

Same layout, file names, seed and draw order (RandomState(seed): Q, then K,
then V, standard normal, cast to float32) as the reference's generator
(experiments/gen_perceiver_refs.py:41-76), so bench_perceiver_ni.py /
bench_perceiver_nl.py / bench_wmma.py find their inputs.  The reference
output is softmax(Q K^T / sqrt(D)) V with the row max subtracted, evaluated
in float64 on the CPU from the float32 inputs and stored as float32.

    python experiments/gen_perceiver_refs.py
    python experiments/gen_perceiver_refs.py --n-latent 64 --n-input 784 3136 --out data
"""

import argparse
import os

import numpy as np

D = 768
DEFAULT_NL = [64]
DEFAULT_NI = [784, 3136, 12544, 50176]
SEED = 42


def reference_output(Q, K, V):
    """softmax(Q K^T / sqrt(D)) V for 2-D float32 Q [Nl, D], K/V [Ni, D]; the
    product is taken in float64 and returned as float32 [Nl, D]."""
    q, k, v = (np.asarray(a, np.float64) for a in (Q, K, V))
    s = (q @ k.T) / np.sqrt(q.shape[1])
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=1, keepdims=True)
    return (p @ v).astype(np.float32)


def draw(nl, ni, seed=SEED):
    """Q [nl, D], K and V [ni, D]: float32 normal draws in the order Q, K, V."""
    rng = np.random.RandomState(seed)
    Q = rng.randn(nl, D).astype(np.float32)
    K = rng.randn(ni, D).astype(np.float32)
    V = rng.randn(ni, D).astype(np.float32)
    return Q, K, V


def case_dir(out, nl, ni):
    return os.path.join(out, "perceiver", f"Nl{nl}_Ni{ni}")


def write_case(out, nl, ni, seed=SEED):
    """Writes one (Nl, Ni) case; returns its directory."""
    sub = case_dir(out, nl, ni)
    os.makedirs(sub, exist_ok=True)
    Q, K, V = draw(nl, ni, seed)
    ref = reference_output(Q, K, V).reshape(1, nl, D)
    for name, arr in (("Q_matrix", Q), ("K_matrix", K), ("V_matrix", V),
                      ("output_reference", ref)):
        np.save(os.path.join(sub, name + ".npy"), arr)
    return sub


def load_case(root, nl, ni):
    """(Q, K, V, ref) of a written case under ``root`` (the directory holding
    perceiver/), or None when it has not been generated."""
    sub = case_dir(root, nl, ni)
    if not os.path.exists(os.path.join(sub, "Q_matrix.npy")):
        return None
    return tuple(np.load(os.path.join(sub, f"{n}.npy"))
                 for n in ("Q_matrix", "K_matrix", "V_matrix", "output_reference"))


def main(argv=None):
    ap = argparse.ArgumentParser(description="Generate the Perceiver sweep references")
    ap.add_argument("--n-latent", type=int, nargs="+", default=DEFAULT_NL)
    ap.add_argument("--n-input", type=int, nargs="+", default=DEFAULT_NI)
    ap.add_argument("--out", default="data")
    ap.add_argument("--seed", type=int, default=SEED)
    args = ap.parse_args(argv)

    print(f"Perceiver references: D={D} N_latent={args.n_latent} N_input={args.n_input}")
    for nl in args.n_latent:
        for ni in args.n_input:
            side = int(round(ni ** 0.5))
            tag = f"{side}^2" if side * side == ni else ""
            sub = write_case(args.out, nl, ni, args.seed)
            mb = sum(os.path.getsize(os.path.join(sub, f)) for f in os.listdir(sub)) / 1e6
            print(f"  Nl={nl:5d} Ni={ni:6d} {tag:6s} -> {sub} ({mb:.0f} MB)")
    print("Next: python experiments/bench_perceiver_ni.py on the GPU box")


if __name__ == "__main__":
    main()
