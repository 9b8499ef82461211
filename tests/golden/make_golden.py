"""Writes the committed golden fixtures of the cross-attention oracle.

The reference ships no golden vectors (its data/ and *.npy are git-ignored and
regenerated from seed 42), so these fixtures are built here:

* ``tiny_bruteforce.npz`` -- small random inputs and the output of a
  pure-Python triple loop (math.exp / plain float sums, no numpy linear
  algebra), i.e. an evaluation of softmax(Q K^T / sqrt(D)) V that shares no
  code with the oracle.
* ``cfg1_seed0.npz`` -- the reference's CPU-runnable case, B=1 NL=64 NI=784
  D=768 with Q, K, V ~ N(0,1) from RandomState(0): float64 closed-form output
  (stored float32) plus float64 checksums of the regenerated inputs, so a
  drifting generator is caught.
* ``legacy_seed42_nl64.npz`` -- the seed-42 legacy draw of
  generate_references.py:25-31 at NL=64: output and input checksums.
* ``splitk_small.npz`` -- split-K partials (po, pm, pl) and merged output of
  B=1 NL=3 NI=37 S=8 (RandomState(3) inputs; chunk 5 leaves split 7 empty),
  from the float64 oracle.

Run:  python tests/golden/make_golden.py
"""

import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import xattn_oracle as o  # noqa: E402


def brute_force(q, k, v):
    """softmax(q k^T / sqrt(d)) v with Python floats only."""
    b_, nl, d = q.shape
    ni = k.shape[1]
    out = np.zeros((b_, nl, v.shape[2]), np.float64)
    for b in range(b_):
        for i in range(nl):
            qi = [float(x) for x in q[b, i]]
            scores = []
            for j in range(ni):
                kj = k[b, j]
                s = 0.0
                for e in range(d):
                    s += qi[e] * float(kj[e])
                scores.append(s / math.sqrt(d))
            m = max(scores)
            w = [math.exp(s - m) for s in scores]
            z = sum(w)
            for e in range(v.shape[2]):
                acc = 0.0
                for j in range(ni):
                    acc += w[j] * float(v[b, j, e])
                out[b, i, e] = acc / z
    return out


def checksums(*arrays):
    return np.array([[float(np.sum(a, dtype=np.float64)),
                      float(np.sum(np.abs(a), dtype=np.float64)),
                      float(np.sum(a.astype(np.float64) ** 2))] for a in arrays])


def main():
    rng = np.random.RandomState(1234)
    # tiny: D kept small so the pure-Python loop is quick; plus one D=768 row
    q = rng.randn(2, 3, 16).astype(np.float32)
    k = rng.randn(2, 5, 16).astype(np.float32)
    v = rng.randn(2, 5, 16).astype(np.float32)
    q768, k768, v768 = o.make_inputs(1, 2, 3, 768, seed=7)
    np.savez_compressed(os.path.join(HERE, "tiny_bruteforce.npz"),
                        q=q, k=k, v=v, out=brute_force(q, k, v),
                        q768=q768, k768=k768, v768=v768,
                        out768=brute_force(q768, k768, v768))

    q, k, v = o.make_inputs(1, 64, 784, 768, seed=0)
    np.savez_compressed(os.path.join(HERE, "cfg1_seed0.npz"),
                        out=o.attention_f64(q, k, v).astype(np.float32),
                        checksums=checksums(q, k, v), shape=np.array([1, 64, 784, 768]))

    q, k, v = o.make_inputs_legacy(1, 64, 784, 768, seed=42)
    np.savez_compressed(os.path.join(HERE, "legacy_seed42_nl64.npz"),
                        out=o.attention_f64(q, k, v).astype(np.float32),
                        checksums=checksums(q, k, v), shape=np.array([1, 64, 784, 768]))

    q, k, v = o.make_inputs(1, 3, 37, 768, seed=3)
    po, pm, pl = o.splitk_partials(q, k, v, 8)
    np.savez_compressed(os.path.join(HERE, "splitk_small.npz"),
                        po=po.astype(np.float32), pm=pm, pl=pl,
                        out=o.splitk_combine(po, pm, pl).astype(np.float32),
                        checksums=checksums(q, k, v), shape=np.array([1, 3, 37, 768, 8]))
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
