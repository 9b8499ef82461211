"""
Fits a planner's cost model (csrc/xattn_abi.hip: f32_cost for the fp32
path, h16_cost for the 16-bit one) to the timings
experiments/plan_campaign.py writes, and reports how well the fitted model
and the library's own plans pick among the timed plans.

    python fast-cuda-cross-attention_amd/experiments/fit_plan_cost.py plans.jsonl

Model, for a launch of W workgroups (B * row blocks * splits * column
parts) in R = ceil(W / CUs) rounds of ct key tiles each (16 keys fp32, 32
keys 16-bit):

    t = c0 + R * (r0 + ct * (tile[form] + full[form] * [S == 1 and W >= CUs]))
          + [S > 1] * (m0 + m1 * MB of partials + m2 * S * max(0, 1 - B*NL / CUs))

fitted by least squares on relative error with every coefficient >= 0.
"""

import json
import sys

import numpy as np
from scipy.optimize import lsq_linear

CU = 256
D = 768
# workgroup forms (latents per workgroup, column parts) and key-tile size
FORMS = {"fp32": [(64, 1), (32, 1), (16, 1)], "16bit": [(64, 1), (64, 2), (32, 1)]}
TILE = {"fp32": 16, "16bit": 32}


def path_of(r):
    return "fp32" if r.get("dtype") == "fp32" else "16bit"


def names(path):
    return (["c0", "r0"] + [f"tile{f}" for f in FORMS[path]] + [f"full{f}" for f in FORMS[path]]
            + ["m0", "m1_per_MB", "m2"])


def features(r):
    path = path_of(r)
    f = (r["lpw"], r["cp"])
    rows_blk = (r["NL"] + r["lpw"] - 1) // r["lpw"]
    w = r["B"] * rows_blk * r["S"] * r["cp"]
    rounds = -(-w // CU)
    tiles = (r["NI"] + TILE[path] - 1) // TILE[path]
    ct = -(-tiles // r["S"])
    full = r["S"] == 1 and w >= CU
    x = [1.0, float(rounds)]
    x += [rounds * ct if g == f else 0.0 for g in FORMS[path]]
    x += [rounds * ct if (g == f and full) else 0.0 for g in FORMS[path]]
    split = r["S"] > 1
    rows = r["B"] * r["NL"]
    x += [1.0 if split else 0.0, rows * r["S"] * D * 4e-6 if split else 0.0,
          r["S"] * max(0.0, 1.0 - rows / CU) if split else 0.0]
    return x


def fit(rows):
    x = np.array([features(r) for r in rows])
    y = np.array([r["us"] for r in rows])
    return lsq_linear(x / y[:, None], np.ones(len(y)), bounds=(0, np.inf)).x


def shape_of(r):
    return (r["B"], r["NL"], r["NI"])


def main():
    rows = [json.loads(line) for line in open(sys.argv[1])]
    timed = [r for r in rows if not r.get("planned")]
    planned = {shape_of(r): r for r in rows if r.get("planned")}
    shapes = sorted(set(shape_of(r) for r in timed))
    paths = set(path_of(r) for r in timed)
    if len(paths) != 1:
        raise SystemExit("one path (fp32 or 16-bit) per file")
    p = fit(timed)
    print("coefficients:", ", ".join(f"{n} {v:.3f}" for n, v in zip(names(paths.pop()), p)))

    def loss_table(params, label, show):
        losses = []
        for sh in shapes:
            rs = [r for r in timed if shape_of(r) == sh]
            best = min(rs, key=lambda r: r["us"])
            pick = min(rs, key=lambda r: float(np.dot(features(r), params(sh))))
            losses.append(pick["us"] / best["us"] - 1)
            if show:
                print(f"  B={sh[0]} NL={sh[1]} NI={sh[2]}: best {best['lpw']}/{best['cp']}/"
                      f"S={best['S']} {best['us']:.1f} us, model picks {pick['lpw']}/"
                      f"{pick['cp']}/S={pick['S']} {pick['us']:.1f} us "
                      f"(+{100 * losses[-1]:.1f} %)")
        print(f"{label}: best plan at {sum(l == 0 for l in losses)} of {len(shapes)} shapes, "
              f"mean loss {100 * np.mean(losses):.2f} %, worst {100 * max(losses):.1f} %")

    loss_table(lambda sh: p, "fitted model, all shapes", True)
    loo = {sh: fit([r for r in timed if shape_of(r) != sh]) for sh in shapes}
    loss_table(lambda sh: loo[sh], "fitted without the shape itself", False)
    if planned:
        losses = []
        for sh in shapes:
            if sh not in planned:
                continue
            best = min((r for r in timed if shape_of(r) == sh), key=lambda r: r["us"])
            pl = planned[sh]
            losses.append(pl["us"] / best["us"] - 1)
            print(f"  library plan B={sh[0]} NL={sh[1]} NI={sh[2]}: {pl['lpw']}/{pl['cp']}/"
                  f"S={pl['S']} {pl['us']:.1f} us against the best timed {best['us']:.1f} us "
                  f"({100 * losses[-1]:+.1f} %)")
        print(f"library plans: mean {100 * np.mean(losses):+.2f} %, worst "
              f"{100 * max(losses):+.1f} % against the best timed plan")


if __name__ == "__main__":
    main()
