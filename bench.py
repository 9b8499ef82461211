#!/usr/bin/env python3
"""Headline benchmark: fp32 fused cross-attention on one MI355X.

Workload: O = softmax(Q K^T / sqrt(768)) V with B=32, N_latent=1024,
N_input=784, D=768, fp32 in/out, fp32 MFMA (launch_optimized_kernel through
kernels.so).  One step = one call over the whole batch; inputs are resident in
HBM before timing starts.  Prints one JSON line.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--cpu-seconds 10]
    python bench.py --case cfg5-bf16      # other workloads (profiling; no CPU leg)
    python bench.py --copy-calibration 1024   # D2D copy of 1 GiB, for HBM counters

Algorithmic work per call: FLOP = 4*B*NL*NI*D = 78.92 GFLOP; bytes =
B*(NL*D + 2*NI*D)*4 + B*NL*D*4 = 355.5 MB.
"""

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "fast-cuda-cross-attention_amd")
sys.path.insert(0, PKG)

B, NL, NI, D = 32, 1024, 784, 768
PEAK_FP32_MFMA_TFLOPS = 157.3
METRIC = "TFLOP/s + % of MFMA roofline at B=32 NL=1024 NI=784 D=768; µs/call"


def algorithmic_flop(b, nl, ni, d):
    return 4.0 * b * nl * ni * d


def algorithmic_bytes(b, nl, ni, d, bpe_in=4):
    return b * (nl * d + 2 * ni * d) * bpe_in + b * nl * d * 4


def load_traffic():
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    scaled by the copy-kernel calibration), committed under profiles/."""
    path = os.path.join(ROOT, "profiles", "flash_f32_b32_nl1024_ni784_traffic.json")
    try:
        with open(path) as f:
            return float(json.load(f)["hbm_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def _time_cpu(fn, seconds):
    """(calls, elapsed s) of ``fn`` repeated for ~``seconds`` after 3 warmups."""
    for _ in range(3):
        fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 5) or el >= 3 * seconds:
            return n, el


def cpu_model():
    """The host CPU's model name (Linux /proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(seconds):
    """PyTorch CPU SDPA (the reference's CPU path) on a bounded sample: one
    batch element of the headline workload, repeated for ~``seconds``.  The
    reference's own bmm -> softmax -> bmm formulation (generate_references.py:
    17-23) is timed beside it for a third of that, reported under "also"."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import torch
    import xattn_oracle

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    q, k, v = xattn_oracle.make_inputs(1, NL, NI, D, seed=0)
    flop = algorithmic_flop(1, NL, NI, D)
    n, el = _time_cpu(lambda: xattn_oracle.sdpa_cpu(q, k, v), seconds)
    n2, el2 = _time_cpu(lambda: xattn_oracle.attention_torch_f32(q, k, v), seconds / 3)
    return {
        "value": flop / (el / n) / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": (f"torch CPU scaled_dot_product_attention fp32 on B=1 of the workload "
                   f"(NL={NL} NI={NI} D={D}), {n} calls in {el:.1f} s, "
                   f"{el / n * 1e3:.2f} ms/call"),
        "also": {
            "value": flop / (el2 / n2) / 1e12,
            "unit": "TFLOP/s",
            "sample": (f"torch CPU bmm -> /sqrt(D) -> softmax -> bmm fp32 (the reference's "
                       f"oracle formulation), same input, {n2} calls in {el2:.1f} s, "
                       f"{el2 / n2 * 1e3:.2f} ms/call"),
        },
    }


# Secondary workloads (split-K long input, 16-bit, small batch): name ->
# (B, NL, NI, element type, entry point, Q std)
CASES = {
    "cfg1": (1, 64, 784, "fp32", "launch_optimized_kernel", 1.0),
    "cfg4-4096": (1, 256, 4096, "fp32", "launch_optimized_kernel", 0.02),
    "cfg4-16384": (1, 256, 16384, "fp32", "launch_optimized_kernel", 0.02),
    "cfg4-50176": (1, 256, 50176, "fp32", "launch_optimized_kernel", 0.02),
    "cfg4-splitk-4096": (1, 256, 4096, "fp32", "launch_splitk_kernel", 0.02),
    "cfg4-splitk-16384": (1, 256, 16384, "fp32", "launch_splitk_kernel", 0.02),
    "cfg4-splitk-50176": (1, 256, 50176, "fp32", "launch_splitk_kernel", 0.02),
    "cfg5-fp16": (16, 512, 784, "fp16", "launch_wmma_kernel", 1.0),
    "cfg5-bf16": (16, 512, 784, "bf16", "launch_wmma_bf16_kernel", 1.0),
    "headline-bf16": (32, 1024, 784, "bf16", "launch_wmma_bf16_kernel", 1.0),
    "headline-fp16": (32, 1024, 784, "fp16", "launch_wmma_kernel", 1.0),
    "headline-fp32": (32, 1024, 784, "fp32", "launch_optimized_kernel", 1.0),
}


def time_launches(cw, launch, steps, warmup):
    """Exactly `warmup` untimed launches (the first one's error state checked),
    then `steps` launches each bracketed by HIP events on the launch stream
    (the null stream); returns (wall_s, per-launch ms)."""
    stream = ctypes.c_void_p(0)
    for i in range(warmup):
        launch()
        if i == 0:
            cw._lib_error_check("launch")
    if cw.cudart.cudaDeviceSynchronize() != 0:
        raise RuntimeError("warmup failed")
    evs = [(ctypes.c_void_p(), ctypes.c_void_p()) for _ in range(steps)]
    for a, b in evs:
        cw.cudart.cudaEventCreate(ctypes.byref(a))
        cw.cudart.cudaEventCreate(ctypes.byref(b))
    cw.cudart.cudaDeviceSynchronize()
    t0 = time.perf_counter()
    for a, b in evs:
        cw.cudart.cudaEventRecord(a, stream)
        launch()
        cw.cudart.cudaEventRecord(b, stream)
    cw.cudart.cudaDeviceSynchronize()
    wall = time.perf_counter() - t0
    ms = ctypes.c_float()
    per = []
    for a, b in evs:
        cw.cudart.cudaEventElapsedTime(ctypes.byref(ms), a, b)
        per.append(ms.value)
        cw.cudart.cudaEventDestroy(a)
        cw.cudart.cudaEventDestroy(b)
    cw._lib_error_check("launch")
    return wall, per


def launch_stats(per_ms):
    """Per-launch event times (µs): mean, median, extremes and the means of
    the first and last quarter of the timed launches (a clock that is still
    ramping shows as a first quarter slower than the last)."""
    us = np.asarray(per_ms, dtype=np.float64) * 1e3
    q = max(1, len(us) // 4)
    return {
        "mean": round(float(us.mean()), 2),
        "median": round(float(np.median(us)), 2),
        "min": round(float(us.min()), 2),
        "max": round(float(us.max()), 2),
        "first_quarter_mean": round(float(us[:q].mean()), 2),
        "last_quarter_mean": round(float(us[-q:].mean()), 2),
    }


def parse_plan(text):
    """'LPW/CP/S' -> (latents per workgroup, column parts, key splits)."""
    try:
        lpw, cp, s = (int(x) for x in text.split("/"))
    except ValueError:
        raise argparse.ArgumentTypeError(f"plan {text!r} is not LPW/CP/S (e.g. 64/2/1)")
    return lpw, cp, s


def run_case(cw, name, steps, warmup, plan=None):
    """Time case `name`; `plan` (16-bit cases only): run it through
    launch_wmma_plan_kernel with that (latents per workgroup, column parts,
    key splits) instead of the entry point's own plan."""
    b, nl, ni, et, entry, q_std = CASES[name]
    if plan is not None and et == "fp32":
        raise ValueError(f"--plan applies to the 16-bit cases, not {name}")
    cu, _ = cw.device_info()
    rng = np.random.RandomState(0)
    q = (rng.randn(b, nl, D) * q_std).astype(np.float32)
    k = rng.randn(b, ni, D).astype(np.float32)
    v = rng.randn(b, ni, D).astype(np.float32)
    if et == "fp32":
        host = (q, k, v)
    else:
        host = cw._half_inputs(q, k, v, b, D, bf16=(et == "bf16"))
    bufs = [cw.DeviceBuffer.holding(a) for a in host]
    out = cw.DeviceBuffer(b * nl * D * 4).zero()
    extra = []
    stream = ctypes.c_void_p(0)
    fn = getattr(cw.lib, entry)
    note = {}
    if plan is not None:
        fn = cw.lib.launch_wmma_plan_kernel
        entry = "launch_wmma_plan_kernel"
        note["plan"] = list(plan)
        args = [int(et == "bf16")] + [p.ptr for p in bufs] + [out.f32, b, nl, ni, D, *plan, stream]
    elif entry == "launch_splitk_kernel":
        s = cw.plan_num_splits(nl, ni, b, cu)
        extra = [cw.DeviceBuffer(b * nl * s * D * 4), cw.DeviceBuffer(b * nl * s * 4),
                 cw.DeviceBuffer(b * nl * s * 4)]
        note["num_splits"] = s
        args = [p.f32 for p in bufs + [out] + extra] + [b, nl, ni, D, s, stream]
    elif et == "fp32":
        args = [p.f32 for p in bufs + [out]] + [b, nl, ni, D, stream]
    else:
        args = [p.ptr for p in bufs] + [out.f32, b, nl, ni, D, stream]
    wall, per = time_launches(cw, lambda: fn(*args), steps, warmup)
    for p in bufs + [out] + extra:
        p.close()
    bpe = 4 if et == "fp32" else 2
    kern_ms = float(np.mean(per))
    flop = algorithmic_flop(b, nl, ni, D)
    byt = algorithmic_bytes(b, nl, ni, D, bpe)
    peak = PEAK_FP32_MFMA_TFLOPS if et == "fp32" else 2516.6
    return {
        "case": name, "entry_point": entry, "dtype": et, "B": b, "NL": nl, "NI": ni, "D": D,
        "us_per_call": round(kern_ms * 1e3, 2),
        "tflops": round(flop / (kern_ms * 1e-3) / 1e12, 3),
        "pct_of_mfma_peak": round(100 * flop / (kern_ms * 1e-3) / 1e12 / peak, 2),
        "gbs_algorithmic": round(byt / (kern_ms * 1e-3) / 1e9, 1),
        "pct_of_hbm_peak": round(100 * byt / (kern_ms * 1e-3) / 8.0e12, 2),
        "ms_per_step_wall": round(wall * 1e3 / steps, 5),
        "launch_us": launch_stats(per), **note,
    }


def _phase_clock_fns(cw, et):
    """(clear, read) of the phase-clock library for element type `et`."""
    suffix = "f32" if et == "fp32" else "f16"
    read = getattr(cw.lib, "xattn_phase_clock_read_" + suffix, None)
    clear = getattr(cw.lib, "xattn_phase_clock_clear_" + suffix, None)
    if read is None or clear is None:
        raise RuntimeError("--phase-clock needs kernels_phaseclock.so (make phaseclock; "
                           "XATTN_KERNELS_SO=<path> python bench.py ...)")
    read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    read.restype = ctypes.c_int
    clear.argtypes = []
    clear.restype = ctypes.c_int
    return clear, read


def phase_clock_clear(cw, name):
    clear, _ = _phase_clock_fns(cw, CASES[name][3])
    if clear() != 0:
        raise RuntimeError("xattn_phase_clock_clear failed")


def phase_clock(cw, name):
    """Lifetime split of the flash kernel's workgroups in the last launch of
    case `name`, from a library built with `make phaseclock` (loaded through
    XATTN_KERNELS_SO; cleared before the case runs): per wavefront, cycles
    from start to the tile loop (prologue: Q block, first tiles), in the
    loop, and after it (epilogue: the O store); for the fp32 kernel also the
    loop's per-tile sums (waits at the tile barriers, the QK phase, the PV
    phase); the shader clock from the 100 MHz real-time stamps; and the
    workgroups' start times relative to the first (rounds show as
    clusters).  Workgroups and wavefronts that left no stamps (past the
    grid, or past the kernel's wavefronts) are not counted; a split launch's
    merge kernel is not instrumented."""
    _, read = _phase_clock_fns(cw, CASES[name][3])
    raw = np.zeros((4096, 8, 9), dtype=np.uint64)
    if read(raw.ctypes.data, raw.nbytes) != 0:
        raise RuntimeError("xattn_phase_clock_read failed")
    live = raw[..., 3] != 0
    nblk = int(live.any(axis=1).sum())
    nw = int(live[0].sum())
    if nblk == 0 or nw == 0:
        raise RuntimeError(f"no phase-clock stamps after case {name}")
    c = raw[:nblk, :nw].astype(np.int64)
    life = c[..., 3] - c[..., 0]
    cycles = {"lifetime": life, "prologue": c[..., 1] - c[..., 0],
              "tile_loop": c[..., 2] - c[..., 1], "epilogue": c[..., 3] - c[..., 2]}
    if c[..., 6:9].any():
        cycles.update({"loop_waits": c[..., 6], "loop_qk": c[..., 7], "loop_pv": c[..., 8]})
    rt = c[..., 5] - c[..., 4]
    start_us = (c[:, 0, 4] - c[:, 0, 4].min()) * 0.01
    return {
        "workgroups": nblk, "wavefronts": nw,
        "clock_ghz": round(float(life.sum() / rt.sum() * 0.1), 3),
        "cycles": {k: round(float(v.mean()), 0) for k, v in cycles.items()},
        "start_us_quantiles": [round(float(x), 2) for x in
                               np.quantile(start_us, [0, 0.25, 0.5, 0.75, 1.0])],
    }


def copy_calibration(cw, mib, reps=5):
    """Plain device-to-device copy of `mib` MiB, `reps` times: reads and writes
    exactly mib MiB per copy, the reference point for FETCH_SIZE/WRITE_SIZE."""
    n = mib * 1024 * 1024
    with cw.DeviceBuffer(n) as a, cw.DeviceBuffer(n) as b:
        cw.cudart.hipMemset(a.ptr, 1, n)
        cw.cudart.hipDeviceSynchronize()
        for _ in range(reps):
            if cw.cudart.hipMemcpy(b.ptr, a.ptr, n, 3) != 0:  # hipMemcpyDeviceToDevice
                raise RuntimeError("hipMemcpy D2D failed")
        cw.cudart.hipDeviceSynchronize()
    print(json.dumps({"copy_calibration_bytes_per_copy": n, "copies": reps}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--case", choices=sorted(CASES), action="append",
                    help="run a secondary workload instead of the headline")
    ap.add_argument("--copy-calibration", type=int, metavar="MIB")
    ap.add_argument("--phase-clock", action="store_true",
                    help="with --case and a `make phaseclock` library: add the flash "
                         "kernel's prologue / tile loop / epilogue cycles")
    ap.add_argument("--plan", type=parse_plan, metavar="LPW/CP/S",
                    help="with --case (16-bit cases): launch through launch_wmma_plan_kernel "
                         "with this plan (latents per workgroup / column parts / key splits)")
    ap.add_argument("--launch-log", metavar="PATH",
                    help="also write every timed launch's event time (µs) to PATH as JSON")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import cuda_wrappers as cw

    if args.copy_calibration:
        copy_calibration(cw, args.copy_calibration)
        return
    if args.case:
        for name in args.case:
            if args.phase_clock:
                phase_clock_clear(cw, name)
            rec = run_case(cw, name, args.steps, args.warmup, args.plan)
            if args.phase_clock:
                rec["phase_clock"] = phase_clock(cw, name)
            print(json.dumps(rec), flush=True)
        return

    cu, _ = cw.device_info()
    rng = np.random.RandomState(0)
    q = rng.randn(B, NL, D).astype(np.float32)
    k = rng.randn(B, NI, D).astype(np.float32)
    v = rng.randn(B, NI, D).astype(np.float32)
    bufs = [cw.DeviceBuffer.holding(a) for a in (q, k, v)]
    out = cw.DeviceBuffer(B * NL * D * 4).zero()
    qp, kp, vp = (p.f32 for p in bufs)
    op = out.f32
    stream = ctypes.c_void_p(0)

    def launch():
        cw.lib.launch_optimized_kernel(qp, kp, vp, op, B, NL, NI, D, stream)

    # Timed region: K back-to-back launches bracketed by a device sync; each
    # launch also bracketed by HIP events on the launch stream.
    wall, per = time_launches(cw, launch, args.steps, args.warmup)
    if args.launch_log:
        with open(args.launch_log, "w") as f:
            json.dump({"steps": args.steps, "warmup": args.warmup,
                       "launch_us": [round(x * 1e3, 3) for x in per]}, f)

    flop = algorithmic_flop(B, NL, NI, D)
    ms_per_step = wall * 1e3 / args.steps
    kern_ms = float(np.mean(per))
    achieved = flop / (kern_ms * 1e-3) / 1e12
    value = flop / (ms_per_step * 1e-3) / 1e12

    # spot-check the result of the timed launches against the float64 oracle
    # on a few rows (cheap; the full parity suite lives in tests/)
    res = out.download((B, NL, D))
    for p in bufs + [out]:
        p.close()
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import xattn_oracle
    rows = [0, 17, 31]
    ref = xattn_oracle.attention_f64(q[rows, :64], k[rows], v[rows])
    spot_err = xattn_oracle.max_abs(res[rows, :64], ref)

    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_call": round(kern_ms * 1e3, 2),
        "pct_of_mfma_peak": round(100.0 * achieved / PEAK_FP32_MFMA_TFLOPS, 2),
        "launch_us": launch_stats(per),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": f"fused cross-attention fp32 B={B} NL={NL} NI={NI} D={D}",
                   "batch": B, "n_latent": NL, "n_input": NI, "dim": D,
                   "entry_point": "launch_optimized_kernel", "compute_units": cu},
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
            "traffic": load_traffic(),
        },
        "spot_check_max_abs": spot_err,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
