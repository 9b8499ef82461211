"""
Times the 16-bit path under every launch plan its planner weighs, at a grid
of shapes, and the planner's own choice beside them: the data the cost
model of xattn_wmma_plan (csrc/xattn_abi.hip, h16_cost) is fitted to
(experiments/fit_wmma_cost.py).

    python fast-cuda-cross-attention_amd/experiments/wmma_plan_campaign.py > plans.jsonl

One JSON line per timed launch: the shape, the plan (latents per workgroup,
column parts, key splits; "planned": true for launch_wmma_bf16_kernel's own
plan) and the median µs per call over --steps launches after --warmup, each
launch between two HIP events recorded back to back, as bench.py times a
call.  Plans: the three workgroup forms (64 latents, 64 latents in two
column halves, 32 latents) with every split count that gives whole 32-key
tiles per split (a log-spaced subset of them when there are more than 12)
and at most four rounds of workgroups.
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
FORMS = [(64, 1), (64, 2), (32, 1)]
SHAPES = [(1, 64, 784), (1, 256, 784), (1, 1024, 784), (2, 512, 784), (4, 512, 784),
          (4, 1024, 784), (8, 256, 784), (8, 512, 784), (8, 1024, 784), (16, 256, 784),
          (16, 512, 784), (16, 1024, 784), (32, 256, 784), (32, 512, 784), (24, 1024, 784),
          (32, 1024, 784), (4, 1024, 1568), (16, 512, 1568), (32, 1024, 1568),
          (16, 256, 3136), (8, 512, 3136), (2, 1024, 3136), (1, 256, 4096), (4, 512, 4096),
          (1, 256, 16384), (1, 1024, 16384), (2, 256, 50176)]


def split_counts(b, nl, ni, lpw, cp, cu):
    """Split counts of whole 32-key tiles (each count that no smaller chunk
    size also gives) with at most four rounds of workgroups."""
    tiles = (ni + 31) // 32
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
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--dtype", choices=("bf16", "fp16"), default="bf16")
    ap.add_argument("--shapes", default=None,
                    help="comma-separated BxNLxNI (default: the fitted grid)")
    args = ap.parse_args()
    if not cw.HAS_WMMA_PLAN:
        raise RuntimeError("this kernels.so does not export launch_wmma_plan_kernel")
    shapes = SHAPES if args.shapes is None else [
        tuple(int(x) for x in s.split("x")) for s in args.shapes.split(",")]
    cu, _ = cw.device_info()
    bf16 = args.dtype == "bf16"
    planned_fn = cw.lib.launch_wmma_bf16_kernel if bf16 else cw.lib.launch_wmma_kernel
    null = ctypes.c_void_p(0)
    for (b, nl, ni) in shapes:
        rng = np.random.RandomState(0)
        q = rng.randn(b, nl, D).astype(np.float32)
        k = rng.randn(b, ni, D).astype(np.float32)
        v = rng.randn(b, ni, D).astype(np.float32)
        host = cw._half_inputs(q, k, v, b, D, bf16=bf16)
        bufs = [cw.DeviceBuffer.holding(a) for a in host]
        out = cw.DeviceBuffer(b * nl * D * 4).zero()
        qkv = [p.ptr for p in bufs]
        try:
            for lpw, cp in FORMS:
                for s in split_counts(b, nl, ni, lpw, cp, cu):
                    us = median_us(lambda: cw.lib.launch_wmma_plan_kernel(
                        int(bf16), *qkv, out.f32, b, nl, ni, D, lpw, cp, s, null),
                        args.steps, args.warmup)
                    print(json.dumps({"B": b, "NL": nl, "NI": ni, "lpw": lpw, "cp": cp, "S": s,
                                      "us": round(us, 2)}), flush=True)
            lpw, cp, s = cw.wmma_plan_form(b, nl, ni, cu)
            us = median_us(lambda: planned_fn(*qkv, out.f32, b, nl, ni, D, null),
                           args.steps, args.warmup)
            print(json.dumps({"B": b, "NL": nl, "NI": ni, "lpw": lpw, "cp": cp, "S": s,
                              "us": round(us, 2), "planned": True}), flush=True)
        finally:
            for p in bufs + [out]:
                p.close()


if __name__ == "__main__":
    main()
