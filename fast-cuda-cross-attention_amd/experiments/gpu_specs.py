"""
Hardware ceilings for the roofline columns, and detection of the device.

Peaks are AMD's published dense figures (no sparsity) for the two gfx950
parts the library is built for; FLOP/s and bytes/s, not T-units.  The fp32
figure is the MFMA (matrix) peak the fp32 kernel runs on.  The key names
(``sm_count`` = compute units, ``smem_per_sm_kb`` = LDS per CU) follow the
reference's table (experiments/gpu_specs.py:15-57) so the drivers and plots
read both.

    ridge_point = peak_flops / peak_bw   (FLOP per byte)

A point whose arithmetic intensity is above the ridge is compute-bound.
"""

import ctypes
import os
import re
import subprocess

TFLOP = 1.0e12
GBs = 1.0e9

GPU_SPECS = {
    # AMD Instinct MI355X (CDNA4, gfx950): 256 CUs in 8 XCDs, 2.4 GHz peak
    # engine clock, 160 KiB LDS per CU, 288 GB HBM3E.
    "MI355X": {
        "arch": "CDNA4",
        "gfx": "gfx950",
        "sm_count": 256,
        "smem_per_sm_kb": 160,
        "peak_fp32_flops": 157.3 * TFLOP,
        "peak_fp16_tc_flops": 2516.6 * TFLOP,
        "peak_bf16_tc_flops": 2516.6 * TFLOP,
        "peak_bw_bytes": 8000.0 * GBs,
    },
    # AMD Instinct MI350X: the same gfx950 silicon at a 2.2 GHz peak clock.
    "MI350X": {
        "arch": "CDNA4",
        "gfx": "gfx950",
        "sm_count": 256,
        "smem_per_sm_kb": 160,
        "peak_fp32_flops": 144.2 * TFLOP,
        "peak_fp16_tc_flops": 2306.9 * TFLOP,
        "peak_bf16_tc_flops": 2306.9 * TFLOP,
        "peak_bw_bytes": 8000.0 * GBs,
    },
}

# precision -> the peak a point of that precision is measured against
PRECISION_PEAK_KEY = {
    "fp32": "peak_fp32_flops",
    "fp16": "peak_fp16_tc_flops",
    "bf16": "peak_bf16_tc_flops",
}


def _hip_device_name(device=0):
    """Device name from the HIP runtime (hipDeviceGetName), or None."""
    for lib in ("libamdhip64.so", "libamdhip64.so.7", "libamdhip64.so.6",
                "/opt/rocm/lib/libamdhip64.so"):
        try:
            hip = ctypes.CDLL(lib)
            break
        except OSError:
            continue
    else:
        return None
    count = ctypes.c_int(0)
    if hip.hipGetDeviceCount(ctypes.byref(count)) != 0 or count.value <= device:
        return None
    buf = ctypes.create_string_buffer(256)
    if hip.hipDeviceGetName(buf, ctypes.c_int(len(buf)), ctypes.c_int(device)) != 0:
        return None
    name = buf.value.decode(errors="replace").strip()
    return name or None


def _smi_device_name():
    """Product name from amd-smi, then rocm-smi; None when neither answers."""
    probes = (
        (["amd-smi", "static", "--asic", "-g", "0"], r"MARKET_NAME:\s*(.+)"),
        (["rocm-smi", "--showproductname"], r"Card (?:Series|SKU)\s*:\s*(.+)"),
    )
    for cmd, pattern in probes:
        try:
            out = subprocess.run(cmd, capture_output=True, text=True, timeout=20)
        except (OSError, subprocess.SubprocessError):
            continue
        if out.returncode != 0:
            continue
        m = re.search(pattern, out.stdout)
        if m:
            return m.group(1).strip()
    return None


def raw_gpu_name(device=0):
    """The device's product name: HIP runtime, then amd-smi / rocm-smi, then
    torch; None off a GPU box."""
    name = _hip_device_name(device) or _smi_device_name()
    if name:
        return name
    try:
        import torch
        if torch.cuda.is_available():
            return torch.cuda.get_device_name(device)
    except Exception:
        pass
    return None


def gpu_key_for_name(name):
    """GPU_SPECS key for a product name, or None when it is not one of them."""
    if not name:
        return None
    upper = name.upper().replace(" ", "")
    for key in ("MI355X", "MI350X"):
        if key in upper:
            return key
    if "MI355" in upper:
        return "MI355X"
    if "MI350" in upper:
        return "MI350X"
    return None


def gpu_key_for_arch(arch, clock_khz):
    """GPU_SPECS key from the architecture name and peak engine clock: gfx950
    at 2.4 GHz is the MI355X, at 2.2 GHz the MI350X."""
    if not arch or not arch.split(":")[0] == "gfx950":
        return None
    return "MI355X" if clock_khz >= 2300000 else "MI350X"


def _library_arch(device=0):
    """(arch, clock_khz) through this library's kernels.so, or (None, 0)."""
    here = os.path.dirname(os.path.abspath(__file__))
    for so in (os.environ.get("XATTN_KERNELS_SO"),
               os.path.join(os.path.dirname(here), "kernels.so")):
        if not so or not os.path.exists(so):
            continue
        try:
            lib = ctypes.CDLL(so)
        except OSError:
            continue
        buf = ctypes.create_string_buffer(256)
        khz = ctypes.c_int(0)
        fn = lib.xattn_device_arch
        fn.argtypes = [ctypes.c_int, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]
        if fn(device, buf, len(buf), ctypes.byref(khz)) == 0:
            return buf.value.decode(errors="replace"), khz.value
    return None, 0


def detect_gpu_name(device=0):
    """GPU_SPECS key of the current device (XATTN_GPU_KEY overrides), or None
    for an unknown card or no GPU; callers then log the raw name.  The product
    name decides when it names the part; hosts without libdrm's ASIC table
    report a generic name, and then the architecture and clock decide."""
    forced = os.environ.get("XATTN_GPU_KEY")
    if forced:
        return forced if forced in GPU_SPECS else None
    key = gpu_key_for_name(raw_gpu_name(device))
    if key is None:
        key = gpu_key_for_arch(*_library_arch(device))
    return key


def ridge_point(gpu_key, precision="fp32"):
    """FLOP per HBM byte at which ``precision`` work on ``gpu_key`` turns
    compute-bound; None when the card has no such peak."""
    spec = GPU_SPECS[gpu_key]
    peak = spec.get(PRECISION_PEAK_KEY[precision])
    if peak is None:
        return None
    return peak / spec["peak_bw_bytes"]


if __name__ == "__main__":
    print(f"device: {raw_gpu_name() or '(none)'} -> key {detect_gpu_name()}")
    for key, spec in GPU_SPECS.items():
        for prec in ("fp32", "bf16"):
            peak = spec[PRECISION_PEAK_KEY[prec]]
            print(f"{key:7s} {prec:5s} ridge {ridge_point(key, prec):6.1f} FLOP/B  "
                  f"(peak {peak / TFLOP:7.1f} TFLOP/s, HBM {spec['peak_bw_bytes'] / GBs:.0f} GB/s, "
                  f"{spec['sm_count']} CUs)")
