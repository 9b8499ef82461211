"""
Times the fused path under every launch plan its planner weighs, at a grid
of shapes, and the planner's own choice beside them: the data the cost
models of xattn_f32_plan and xattn_wmma_plan (csrc/xattn_abi.hip, f32_cost
and h16_cost) are fitted to (experiments/fit_plan_cost.py).

    python fast-cuda-cross-attention_amd/experiments/plan_campaign.py --dtype fp32 > f32.jsonl
    python fast-cuda-cross-attention_amd/experiments/plan_campaign.py --dtype bf16 > bf16.jsonl

One JSON line per timed launch: the path, the shape, the plan (latents per
workgroup, column parts, key splits; "planned": true for the entry point's
own plan, launch_optimized_kernel or launch_wmma[_bf16]_kernel) and the
median µs per call over --steps launches after --warmup, each launch
between two HIP events recorded back to back, as bench.py times a call.
Plans: every workgroup form of the path (fp32: 64, 32 or 16 latents;
16-bit: 64 latents, 64 latents in two column halves, 32 latents) with every
split count that gives whole key tiles per split (16 keys fp32, 32 keys
16-bit; a log-spaced subset when there are more than 12) and at most four
rounds of workgroups, through launch_optimized_plan_kernel /
launch_wmma_plan_kernel.
"""

import argparse
import ctypes
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import cuda_wrappers as cw  # noqa: E402

D = 768
FORMS = {"fp32": [(64, 1), (32, 1), (16, 1)], "16bit": [(64, 1), (64, 2), (32, 1)]}
TILE = {"fp32": 16, "16bit": 32}
# fp32: the five configurations' shapes (B=1 N_latent sweep, the batched
# grid at N_input 784, the long-input split-K shapes) and a few between;
# 16-bit: a grid over the range the planner serves.
SHAPES = {
    "fp32": [(1, 64, 784), (1, 128, 784), (1, 256, 784), (1, 512, 784), (1, 1024, 784),
             (2, 256, 784), (4, 64, 784), (4, 128, 784), (4, 256, 784), (4, 512, 784),
             (4, 1024, 784), (8, 64, 784), (8, 128, 784), (8, 256, 784), (8, 512, 784),
             (8, 1024, 784), (16, 64, 784), (16, 128, 784), (16, 256, 784), (16, 512, 784),
             (16, 1024, 784), (32, 64, 784), (32, 128, 784), (32, 256, 784), (32, 512, 784),
             (32, 1024, 784), (1, 256, 4096), (1, 256, 16384), (1, 256, 50176),
             (4, 512, 4096), (2, 1024, 3136)],
    "16bit": [(1, 64, 784), (1, 256, 784), (1, 1024, 784), (2, 512, 784), (4, 512, 784),
              (4, 1024, 784), (8, 256, 784), (8, 512, 784), (8, 1024, 784), (16, 256, 784),
              (16, 512, 784), (16, 1024, 784), (32, 256, 784), (32, 512, 784),
              (24, 1024, 784), (32, 1024, 784), (4, 1024, 1568), (16, 512, 1568),
              (32, 1024, 1568), (16, 256, 3136), (8, 512, 3136), (2, 1024, 3136),
              (1, 256, 4096), (4, 512, 4096), (1, 256, 16384), (1, 1024, 16384),
              (2, 256, 50176)],
}


def split_counts(b, nl, ni, lpw, cp, cu, tile):
    """Split counts of whole key tiles (each count that no smaller chunk size
    also gives) with at most four rounds of workgroups."""
    tiles = (ni + tile - 1) // tile
    rows = (nl + lpw - 1) // lpw
    out = []
    for s in range(1, min(tiles, cu) + 1):
        ct = (tiles + s - 1) // s
        if (tiles + ct - 1) // ct != s:
            continue
        if s > 1 and b * rows * s * cp > 4 * cu:
            continue
        out.append(s)
    if len(out) <= 12:
        return out
    idx = sorted(set(int(round(x)) for x in np.geomspace(1, len(out), 14)) | {1})
    return sorted(set(out[i - 1] for i in idx))


def median_us(launch, steps, warmup):
    """Median µs per call of `launch` over `steps` calls after `warmup`."""
    launch()
    for _ in range(warmup):
        launch()
    if cw.cudart.cudaDeviceSynchronize() != 0:
        raise RuntimeError("warmup failed")
    evs = [(ctypes.c_void_p(), ctypes.c_void_p()) for _ in range(steps)]
    for a, b in evs:
        cw.cudart.cudaEventCreate(ctypes.byref(a))
        cw.cudart.cudaEventCreate(ctypes.byref(b))
    null = ctypes.c_void_p(0)
    for a, b in evs:
        cw.cudart.cudaEventRecord(a, null)
        launch()
        cw.cudart.cudaEventRecord(b, null)
    if cw.cudart.cudaDeviceSynchronize() != 0:
        raise RuntimeError("timed launches failed")
    ms = ctypes.c_float()
    per = []
    for a, b in evs:
        cw.cudart.cudaEventElapsedTime(ctypes.byref(ms), a, b)
        per.append(ms.value)
        cw.cudart.cudaEventDestroy(a)
        cw.cudart.cudaEventDestroy(b)
    cw._lib_error_check("launch")
    return float(np.median(per)) * 1e3


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--dtype", choices=("fp32", "bf16", "fp16"), default="bf16")
    ap.add_argument("--steps", type=int, default=None,
                    help="timed launches per plan (default 100 fp32, 200 16-bit)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed launches first (default 20 fp32, 50 16-bit)")
    ap.add_argument("--shapes", default=None,
                    help="comma-separated BxNLxNI (default: the path's grid)")
    args = ap.parse_args()
    path = "fp32" if args.dtype == "fp32" else "16bit"
    steps = args.steps or (100 if path == "fp32" else 200)
    warmup = args.warmup or (20 if path == "fp32" else 50)
    if not (cw.HAS_OPTIMIZED_PLAN if path == "fp32" else cw.HAS_WMMA_PLAN):
        raise RuntimeError("this kernels.so lacks the plan-override entry points")
    shapes = SHAPES[path] if args.shapes is None else [
        tuple(int(x) for x in s.split("x")) for s in args.shapes.split(",")]
    cu, _ = cw.device_info()
    bf16 = args.dtype == "bf16"
    null = ctypes.c_void_p(0)
    for (b, nl, ni) in shapes:
        rng = np.random.RandomState(0)
        q = rng.randn(b, nl, D).astype(np.float32)
        k = rng.randn(b, ni, D).astype(np.float32)
        v = rng.randn(b, ni, D).astype(np.float32)
        host = (q, k, v) if path == "fp32" else cw._half_inputs(q, k, v, b, D, bf16=bf16)
        bufs = [cw.DeviceBuffer.holding(a) for a in host]
        out = cw.DeviceBuffer(b * nl * D * 4).zero()
        if path == "fp32":
            ins = [p.f32 for p in bufs]

            def forced(lpw, cp, s):
                cw.lib.launch_optimized_plan_kernel(*ins, out.f32, b, nl, ni, D, lpw, s, null)

            def planned():
                cw.lib.launch_optimized_kernel(*ins, out.f32, b, nl, ni, D, null)

            lpw, s = cw.f32_plan(b, nl, ni, cu)
            plan = (lpw, 1, s)
        else:
            ins = [p.ptr for p in bufs]
            entry = cw.lib.launch_wmma_bf16_kernel if bf16 else cw.lib.launch_wmma_kernel

            def forced(lpw, cp, s):
                cw.lib.launch_wmma_plan_kernel(int(bf16), *ins, out.f32, b, nl, ni, D, lpw, cp, s,
                                               null)

            def planned():
                entry(*ins, out.f32, b, nl, ni, D, null)

            plan = cw.wmma_plan_form(b, nl, ni, cu)
        rec = {"dtype": args.dtype, "B": b, "NL": nl, "NI": ni}
        try:
            for lpw, cp in FORMS[path]:
                for s in split_counts(b, nl, ni, lpw, cp, cu, TILE[path]):
                    us = median_us(lambda: forced(lpw, cp, s), steps, warmup)
                    print(json.dumps({**rec, "lpw": lpw, "cp": cp, "S": s, "us": round(us, 2)}),
                          flush=True)
            us = median_us(planned, steps, warmup)
            print(json.dumps({**rec, "lpw": plan[0], "cp": plan[1], "S": plan[2],
                              "us": round(us, 2), "planned": True}), flush=True)
        finally:
            for p in bufs + [out]:
                p.close()


if __name__ == "__main__":
    main()
