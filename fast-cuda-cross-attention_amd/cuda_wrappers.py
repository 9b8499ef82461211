"""
Python wrappers for the MI355X (gfx950) cross-attention kernels, using ctypes
and the raw HIP runtime.  No PyTorch dependency.

Drop-in for the reference's ``cuda_wrappers.py``: every public name, argument
list and return tuple is kept (cuda_wrappers.py:177-691).  Differences a caller
can observe are additive:

* the runtime is ``libamdhip64.so``; the module global ``cudart`` exposes it
  under the CUDA names the reference calls (``cudart.cudaMalloc`` ...), so code
  written against the reference keeps working;
* ``kernels.so`` is loaded from this file's directory (or ``$XATTN_KERNELS_SO``),
  falling back to ``./kernels.so`` as the reference does (cuda_wrappers.py:79);
* argument errors the library refuses before launching (see include/xattn.h)
  raise ``RuntimeError`` with the library's message, and the shape limits of a
  kernel raise ``DesignLimited`` before anything is allocated;
* bf16 twins of the fp16 entry points (``benchmark_wmma_bf16_events``,
  ``benchmark_wmma_splitk_bf16_events``) and their ``HAS_*`` flags;
* the fp16/bf16 paths take any N_latent / N_input (the reference needed both
  to be multiples of 16).
"""

import contextlib
import ctypes
import math
import os
import statistics

import numpy as np

D_MODEL = 768

# ---------------------------------------------------------------------------
# HIP runtime
# ---------------------------------------------------------------------------

_HIP_PATHS = [
    os.environ.get("XATTN_HIP_RUNTIME", ""),
    "/opt/rocm/lib/libamdhip64.so",
    "libamdhip64.so",
    "libamdhip64.so.7",
]


def _load_hip():
    errs = []
    for path in _HIP_PATHS:
        if not path:
            continue
        try:
            return ctypes.CDLL(path)
        except OSError as e:  # try the next candidate
            errs.append(f"{path}: {e}")
    raise RuntimeError("libamdhip64.so (the HIP runtime of a ROCm install) did not load; "
                       "tried " + "; ".join(errs))


class _HipRuntime:
    """The HIP runtime, reachable under the CUDA runtime names the reference
    uses (cudaMalloc -> hipMalloc, ...), with ctypes signatures declared."""

    _SIGS = {
        # cuda name: (hip name, argtypes, restype)
        "cudaMalloc": ("hipMalloc", [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t],
                       ctypes.c_int),
        "cudaMemcpy": ("hipMemcpy", [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                     ctypes.c_int], ctypes.c_int),
        "cudaFree": ("hipFree", [ctypes.c_void_p], ctypes.c_int),
        "cudaDeviceSynchronize": ("hipDeviceSynchronize", [], ctypes.c_int),
        "cudaGetLastError": ("hipGetLastError", [], ctypes.c_int),
        "cudaMemset": ("hipMemset", [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t],
                       ctypes.c_int),
        "cudaDeviceGetAttribute": ("hipDeviceGetAttribute",
                                   [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int],
                                   ctypes.c_int),
        "cudaEventCreate": ("hipEventCreate", [ctypes.POINTER(ctypes.c_void_p)], ctypes.c_int),
        "cudaEventRecord": ("hipEventRecord", [ctypes.c_void_p, ctypes.c_void_p], ctypes.c_int),
        "cudaEventSynchronize": ("hipEventSynchronize", [ctypes.c_void_p], ctypes.c_int),
        "cudaEventElapsedTime": ("hipEventElapsedTime",
                                 [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                  ctypes.c_void_p], ctypes.c_int),
        "cudaEventDestroy": ("hipEventDestroy", [ctypes.c_void_p], ctypes.c_int),
        "cudaGetErrorString": ("hipGetErrorString", [ctypes.c_int], ctypes.c_char_p),
        "cudaSetDevice": ("hipSetDevice", [ctypes.c_int], ctypes.c_int),
        "cudaGetDeviceCount": ("hipGetDeviceCount", [ctypes.POINTER(ctypes.c_int)],
                               ctypes.c_int),
    }

    def __init__(self, dll):
        self._dll = dll
        for cuda_name, (hip_name, argtypes, restype) in self._SIGS.items():
            fn = getattr(dll, hip_name)
            fn.argtypes = argtypes
            fn.restype = restype
            setattr(self, cuda_name, fn)
            setattr(self, hip_name, fn)

    def __getattr__(self, name):
        return getattr(self._dll, name)


try:
    cudart = _HipRuntime(_load_hip())
    cudaMemcpyHostToDevice = 1   # hipMemcpyHostToDevice
    cudaMemcpyDeviceToHost = 2   # hipMemcpyDeviceToHost
except Exception as e:
    raise RuntimeError(f"HIP runtime unavailable: {e}")

# ---------------------------------------------------------------------------
# kernels.so
# ---------------------------------------------------------------------------

_HERE = os.path.dirname(os.path.abspath(__file__))
KERNELS_SO = os.environ.get("XATTN_KERNELS_SO") or os.path.join(_HERE, "kernels.so")
if not os.path.exists(KERNELS_SO) and os.path.exists("./kernels.so"):
    KERNELS_SO = os.path.abspath("./kernels.so")

try:
    lib = ctypes.CDLL(KERNELS_SO)
except OSError as e:
    raise RuntimeError(f"kernels.so did not load from {KERNELS_SO} ({e}); build it with "
                       f"'make -C {_HERE}'")

_F = ctypes.POINTER(ctypes.c_float)
_I = ctypes.c_int
_P = ctypes.c_void_p

for _name in ("launch_naive_kernel", "launch_parallel_kernel", "launch_tiled_kernel",
              "launch_optimized_kernel"):
    _fn = getattr(lib, _name)
    _fn.argtypes = [_F, _F, _F, _F, _I, _I, _I, _I, _P]
    _fn.restype = None

lib.xattn_get_last_error.argtypes = []
lib.xattn_get_last_error.restype = ctypes.c_int
lib.xattn_get_last_error_string.argtypes = []
lib.xattn_get_last_error_string.restype = ctypes.c_char_p
lib.xattn_device_info.argtypes = [_I, ctypes.POINTER(_I), ctypes.POINTER(_I)]
lib.xattn_device_info.restype = ctypes.c_int
lib.xattn_device_arch.argtypes = [_I, ctypes.c_char_p, _I, ctypes.POINTER(_I)]
lib.xattn_device_arch.restype = ctypes.c_int
lib.xattn_xcd_remap.argtypes = [_I, _I]
lib.xattn_xcd_remap.restype = ctypes.c_int
lib.xattn_optimized_num_splits.argtypes = [_I, _I, _I, _I]
lib.xattn_optimized_num_splits.restype = ctypes.c_int
lib.xattn_plan_splits.argtypes = [_I, _I, _I, _I, _I, _I]
lib.xattn_plan_splits.restype = ctypes.c_int
lib.xattn_wmma_plan.argtypes = [_I, _I, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_I)]
lib.xattn_wmma_plan.restype = None
lib.xattn_wmma_plan_ex.argtypes = [_I, _I, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_I),
                                  ctypes.POINTER(_I)]
lib.xattn_wmma_plan_ex.restype = None
lib.xattn_f32_plan.argtypes = [_I, _I, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_I)]
lib.xattn_f32_plan.restype = None
lib.xattn_f32_split_latents.argtypes = [_I, _I, _I, _I, _I]
lib.xattn_f32_split_latents.restype = ctypes.c_int
lib.xattn_wmma_split_latents.argtypes = [_I, _I, _I, _I, _I]
lib.xattn_wmma_split_latents.restype = ctypes.c_int

# Workgroup shape of the MFMA kernels (csrc/xattn_flash_*.hip): 64 latents per
# workgroup (the fp32 entry points drop to 32 or 16, the 16-bit ones to 32,
# when 64 cannot fill the device, see f32_plan and wmma_plan); 16-key tiles
# (fp32) and 32-key tiles (fp16/bf16).
LATENTS_PER_WORKGROUP = 64
KEYS_PER_TILE_F32 = 16
KEYS_PER_TILE_F16 = 32


def f32_plan(batch_size, N_latent, N_input, sm_count):
    """(latents per workgroup, key splits) of launch_optimized_kernel: 64, 32
    or 16 latents per workgroup and whole-tile key splits, chosen by the
    library's cost model (larger workgroups cost less per FLOP; smaller ones
    and splits fill ``sm_count`` compute units at small batch * N_latent)."""
    lpw, s = _I(0), _I(0)
    lib.xattn_f32_plan(batch_size, N_latent, N_input, int(sm_count), ctypes.byref(lpw),
                       ctypes.byref(s))
    return lpw.value, s.value


def wmma_plan(batch_size, N_latent, N_input, sm_count):
    """(latents per workgroup, key splits) of launch_wmma_kernel and its bf16
    twin: 64- or 32-latent workgroups and whole-tile key splits, chosen by
    the library's cost model."""
    lpw, s = _I(0), _I(0)
    lib.xattn_wmma_plan(batch_size, N_latent, N_input, int(sm_count), ctypes.byref(lpw),
                        ctypes.byref(s))
    return lpw.value, s.value


def wmma_plan_form(batch_size, N_latent, N_input, sm_count):
    """(latents per workgroup, column parts, key splits) of the same plan:
    column parts 2 runs each 64-latent row block as two workgroups, one per
    half of the output columns."""
    lpw, cp, s = _I(0), _I(0), _I(0)
    lib.xattn_wmma_plan_ex(batch_size, N_latent, N_input, int(sm_count), ctypes.byref(lpw),
                           ctypes.byref(cp), ctypes.byref(s))
    return lpw.value, cp.value, s.value


def plan_num_splits(N_latent, N_input, batch_size, sm_count, keys_per_tile=KEYS_PER_TILE_F32):
    """Default num_splits of the split-K drivers: the splits the library's
    own plan takes for the shape -- f32_plan's for fp32 (16-key tiles),
    wmma_plan's for the 16-bit kernels (32-key tiles) -- whose workgroup
    size launch_splitk_kernel / launch_wmma_splitk_kernel then pick again for
    that num_splits.  (The reference's ``choose_num_splits`` sizes for
    4-latent blocks and 4x oversubscription; it is kept unchanged for callers
    that use it directly.)"""
    if keys_per_tile == KEYS_PER_TILE_F32:
        return max(1, f32_plan(batch_size, N_latent, N_input, sm_count)[1])
    if keys_per_tile == KEYS_PER_TILE_F16:
        return max(1, wmma_plan(batch_size, N_latent, N_input, sm_count)[1])
    return max(1, lib.xattn_plan_splits(batch_size, N_latent, N_input, int(sm_count),
                                        LATENTS_PER_WORKGROUP, keys_per_tile))


def _bind_optional(name, argtypes):
    try:
        fn = getattr(lib, name)
    except AttributeError:
        return False
    fn.argtypes = argtypes
    fn.restype = None
    return True


_WMMA_ARGS = [_P, _P, _P, _F, _I, _I, _I, _I, _P]
_SPLITK_ARGS = [_F, _F, _F, _F, _F, _F, _F, _I, _I, _I, _I, _I, _P]
_WMMA_SPLITK_ARGS = [_P, _P, _P, _F, _F, _F, _F, _I, _I, _I, _I, _I, _P]

# Optional entry points: a kernels.so built without them loads, and the flag
# says which are there (the reference's convention, cuda_wrappers.py:136-175).
HAS_WMMA = _bind_optional("launch_wmma_kernel", _WMMA_ARGS)
HAS_SPLITK = _bind_optional("launch_splitk_kernel", _SPLITK_ARGS)
HAS_WMMA_SPLITK = _bind_optional("launch_wmma_splitk_kernel", _WMMA_SPLITK_ARGS)
HAS_WMMA_BF16 = _bind_optional("launch_wmma_bf16_kernel", _WMMA_ARGS)
HAS_WMMA_SPLITK_BF16 = _bind_optional("launch_wmma_splitk_bf16_kernel", _WMMA_SPLITK_ARGS)
# The 16-bit path with a caller-given plan (bf16 flag, Q, K, V, output, B, NL,
# NI, dim, latents per workgroup, column parts, key splits, stream; additive,
# for plan tuning).
HAS_WMMA_PLAN = _bind_optional("launch_wmma_plan_kernel", [_I] + _WMMA_ARGS[:-1] + [_I, _I, _I, _P])
# launch_optimized_kernel with a caller-given plan (Q, K, V, output, B, NL, NI,
# dim, latents per workgroup, key splits, stream; additive, for plan tuning).
HAS_OPTIMIZED_PLAN = _bind_optional("launch_optimized_plan_kernel",
                                    [_F, _F, _F, _F, _I, _I, _I, _I, _I, _I, _P])
# launch_optimized_kernel with its split partials in static device scratch:
# for callers that cannot allocate (additive, no reference counterpart).
HAS_NOALLOC = _bind_optional("launch_optimized_kernel_noalloc", [_F, _F, _F, _F, _I, _I, _I, _I,
                                                                 _P])
if HAS_NOALLOC:
    lib.xattn_noalloc_prepare.argtypes = [_I]
    lib.xattn_noalloc_prepare.restype = ctypes.c_int
# The LSE merge pass on its own (po, pm, pl, output, rows, splits, column
# parts, stream; additive: the second launch of launch_splitk_kernel).
HAS_LSE_COMBINE = _bind_optional("xattn_lse_combine", [_F, _F, _F, _F, _I, _I, _I, _P])
if HAS_LSE_COMBINE:
    lib.xattn_lse_combine_parts.argtypes = [_I, _I, _I]
    lib.xattn_lse_combine_parts.restype = ctypes.c_int


class DesignLimited(RuntimeError):
    """A shape this build's kernel does not take, as a matter of design.

    Two cases: the wave-per-latent rung keeps a whole score row (4 bytes per
    key) in one workgroup's LDS, so N_input has a device-dependent ceiling;
    and the MFMA kernels are compiled for D = 768 only.  Sweeps catch it and
    log the point as 'design-limited' instead of failed.
    """


def _lib_error_check(what):
    """Raise RuntimeError if the library refused the last launch."""
    code = lib.xattn_get_last_error()
    if code != 0:
        msg = lib.xattn_get_last_error_string().decode(errors="replace")
        raise RuntimeError(f"{what}: kernels.so refused the launch (code {code}): {msg}")


def device_info(device=0):
    """(compute-unit count, max LDS bytes per workgroup) of ``device``."""
    cu = ctypes.c_int(0)
    lds = ctypes.c_int(0)
    err = lib.xattn_device_info(device, ctypes.byref(cu), ctypes.byref(lds))
    if err != 0:
        raise RuntimeError(f"xattn_device_info failed with HIP error {err}")
    return cu.value, lds.value


def device_arch(device=0):
    """(architecture name, e.g. 'gfx950:sramecc+:xnack-', peak clock in kHz)
    of ``device``."""
    buf = ctypes.create_string_buffer(256)
    khz = ctypes.c_int(0)
    err = lib.xattn_device_arch(device, buf, len(buf), ctypes.byref(khz))
    if err != 0:
        raise RuntimeError(f"xattn_device_arch failed with HIP error {err}")
    return buf.value.decode(errors="replace"), khz.value


def _max_smem_optin(device=0):
    """LDS bytes one workgroup of ``device`` may use (160 KiB on MI355X),
    queried through kernels.so rather than by attribute ordinal; 48 KiB if
    the query fails."""
    try:
        return device_info(device)[1] or 48 * 1024
    except RuntimeError:
        return 48 * 1024


def warp_smem_bytes(N_input):
    """LDS the warp kernel needs for a given N_input."""
    return (4 * N_input + 4) * 4


def _require_dim(D, what):
    if D != D_MODEL:
        raise DesignLimited(f"{what} is built for D={D_MODEL} (got D={D})")


def _require_warp_lds(N_input):
    """The wave-per-latent rung's LDS ceiling, checked before any allocation."""
    need, have = warp_smem_bytes(N_input), _max_smem_optin()
    if need > have:
        raise DesignLimited(
            f"wave-per-latent rung: a {N_input}-key score row takes {need} B of LDS, "
            f"over the {have} B a workgroup may use here (the tiled and MFMA kernels "
            f"stream keys instead)")


def _hip_check(err, what):
    if err != 0:
        name = cudart.hipGetErrorString(err)
        name = name.decode(errors="replace") if name else "?"
        raise RuntimeError(f"{what}: HIP error {err} ({name})")


# ---------------------------------------------------------------------------
# Device memory
# ---------------------------------------------------------------------------

class DeviceBuffer:
    """A block of device memory from hipMalloc, released by ``close()`` or on
    leaving a ``with`` block.  ``ptr`` is the ``void*`` the 16-bit launchers
    take, ``f32`` the ``float*`` view the fp32 ones take."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = ctypes.c_void_p()
        _hip_check(cudart.hipMalloc(ctypes.byref(self.ptr), max(self.nbytes, 1)),
                   f"hipMalloc({self.nbytes})")

    @classmethod
    def holding(cls, host):
        """A new buffer with a copy of the contiguous host array ``host``."""
        buf = cls(host.nbytes)
        try:
            buf.upload(host)
        except Exception:
            buf.close()
            raise
        return buf

    @property
    def f32(self):
        return ctypes.cast(self.ptr, _F)

    def upload(self, host):
        host = np.ascontiguousarray(host)
        if host.nbytes > self.nbytes:
            raise ValueError(f"{host.nbytes} B do not fit a {self.nbytes} B buffer")
        if host.nbytes:
            _hip_check(cudart.hipMemcpy(self.ptr, host.ctypes.data_as(_P), host.nbytes,
                                        cudaMemcpyHostToDevice), "host -> device copy")

    def download(self, shape, dtype=np.float32):
        """A fresh host array of ``shape`` filled from the start of the buffer."""
        host = np.empty(shape, dtype)
        if host.nbytes > self.nbytes:
            raise ValueError(f"{host.nbytes} B exceed the {self.nbytes} B buffer")
        if host.nbytes:
            _hip_check(cudart.hipMemcpy(host.ctypes.data_as(_P), self.ptr, host.nbytes,
                                        cudaMemcpyDeviceToHost), "device -> host copy")
        return host

    def zero(self):
        _hip_check(cudart.hipMemset(self.ptr, 0, max(self.nbytes, 1)), "hipMemset")
        return self

    def close(self):
        if self.ptr:
            cudart.hipFree(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


_NULL_STREAM = ctypes.c_void_p(0)


def _raise_launch_errors(what):
    """Refusals recorded by kernels.so, then the runtime's own launch error."""
    _lib_error_check(what)
    err = cudart.hipGetLastError()
    if err != 0:
        _hip_check(err, f"{what}: launch")


def _run_kernel(kernel_func, Q, K, V, batch_size, N_latent, N_input, D):
    """One self-contained call of an fp32 launcher, in the manner of the
    reference's legacy drivers (cuda_wrappers.py:228-289): device buffers are
    made and filled, the launch runs on the null stream and is waited for,
    and the output comes back as a new [batch_size, N_latent, D] array.
    Every step's cost (allocation, PCIe copies) is part of the call."""
    name = getattr(kernel_func, "__name__", "launch")
    host = [np.ascontiguousarray(a, dtype=np.float32) for a in (Q, K, V)]
    with contextlib.ExitStack() as owned:
        q, k, v = (owned.enter_context(DeviceBuffer.holding(a)) for a in host)
        out = owned.enter_context(DeviceBuffer(batch_size * N_latent * D * 4)).zero()
        kernel_func(q.f32, k.f32, v.f32, out.f32, batch_size, N_latent, N_input, D,
                    _NULL_STREAM)
        _raise_launch_errors(name)
        _hip_check(cudart.hipDeviceSynchronize(), f"{name}: waiting for the kernel")
        return out.download((batch_size, N_latent, D))


def _batchify(Q, K, V):
    if len(Q.shape) == 3:
        return Q.shape[0], Q, K, V
    return (1, np.expand_dims(Q, axis=0).astype(np.float32),
            np.expand_dims(K, axis=0).astype(np.float32),
            np.expand_dims(V, axis=0).astype(np.float32))


def run_naive_kernel(Q, K, V, N_latent, N_input, D):
    """Thread-per-output rung; 2-D or batched 3-D inputs."""
    batch_size, Q, K, V = _batchify(Q, K, V)
    return _run_kernel(lib.launch_naive_kernel, Q, K, V, batch_size, N_latent, N_input, D)


def run_warp_parallel_kernel(Q, K, V, N_latent, N_input, D):
    """Wave-per-latent rung (score row in LDS); DesignLimited past its LDS
    ceiling."""
    _require_warp_lds(N_input)
    batch_size, Q, K, V = _batchify(Q, K, V)
    return _run_kernel(lib.launch_parallel_kernel, Q, K, V, batch_size, N_latent, N_input, D)


def run_tiled_kernel(Q, K, V, N_latent, N_input, D):
    """LDS-tiled online-softmax rung."""
    batch_size, Q, K, V = _batchify(Q, K, V)
    return _run_kernel(lib.launch_tiled_kernel, Q, K, V, batch_size, N_latent, N_input, D)


def run_vectorized_kernel(Q, K, V, N_latent, N_input, D):
    """The fp32 MFMA kernel behind launch_optimized_kernel."""
    _require_dim(D, "the MFMA kernel")
    batch_size, Q, K, V = _batchify(Q, K, V)
    return _run_kernel(lib.launch_optimized_kernel, Q, K, V, batch_size, N_latent, N_input, D)


LAUNCHERS = {
    'naive': lib.launch_naive_kernel,
    'warp': lib.launch_parallel_kernel,
    'tiled': lib.launch_tiled_kernel,
    'vectorized': lib.launch_optimized_kernel,
}


def _prep(arr, batch_size):
    """``arr`` as a C-contiguous float32 [batch_size, rows, D] array: a 2-D
    matrix gains a batch axis, and a batch of one is copied out to
    ``batch_size`` identical batch elements."""
    a = np.asarray(arr, dtype=np.float32)
    if a.ndim == 2:
        a = a.reshape((1,) + a.shape)
    if a.shape[0] == 1 and batch_size > 1:
        a = np.broadcast_to(a, (batch_size,) + a.shape[1:])
    return np.ascontiguousarray(a)


# ---------------------------------------------------------------------------
# Event timing of resident data
# ---------------------------------------------------------------------------

def _time_resident(launch, warmup, iters, label, stream=_NULL_STREAM):
    """Warm up, then time ``iters`` launches one by one with a pair of HIP
    events around each (record, launch, record, wait): the protocol of the
    reference's event drivers (cuda_wrappers.py:422-446).  The first launch
    is checked for a library refusal before any timing.  Returns the
    per-launch times in ms."""
    launch()
    _lib_error_check(label)
    for _ in range(max(warmup - 1, 0)):
        launch()
    err = cudart.hipDeviceSynchronize()
    if err != 0:
        _hip_check(cudart.hipGetLastError() or err, f"{label}: warmup")
    start, stop = ctypes.c_void_p(), ctypes.c_void_p()
    _hip_check(cudart.hipEventCreate(ctypes.byref(start)), "hipEventCreate")
    _hip_check(cudart.hipEventCreate(ctypes.byref(stop)), "hipEventCreate")
    try:
        out, ms = [], ctypes.c_float(0.0)
        for _ in range(iters):
            cudart.hipEventRecord(start, stream)
            launch()
            cudart.hipEventRecord(stop, stream)
            cudart.hipEventSynchronize(stop)
            cudart.hipEventElapsedTime(ctypes.byref(ms), start, stop)
            out.append(ms.value)
        return out
    finally:
        cudart.hipEventDestroy(start)
        cudart.hipEventDestroy(stop)


def _mean_pstdev(times):
    if not times:
        return 0.0, 0.0
    return statistics.mean(times), (statistics.pstdev(times) if len(times) > 1 else 0.0)


def _resident_run(launch_fn, inputs, out_shape, warmup, iters, label, scratch=(),
                  keep_scratch=False):
    """Shared body of the event drivers.  ``inputs`` are host arrays in the
    launcher's element type; ``scratch`` lists the shapes of extra float32
    device buffers (split partials).  ``launch_fn(bufs, out, scratch_bufs)``
    issues one launch.  Returns (output, mean_ms, std_ms, host copies of the
    scratch buffers after the last launch, or None)."""
    with contextlib.ExitStack() as owned:
        bufs = [owned.enter_context(DeviceBuffer.holding(a)) for a in inputs]
        out = owned.enter_context(DeviceBuffer(int(np.prod(out_shape)) * 4)).zero()
        sc = [owned.enter_context(DeviceBuffer(int(np.prod(s)) * 4)) for s in scratch]
        times = _time_resident(lambda: launch_fn(bufs, out, sc), warmup, iters, label)
        mean_ms, std_ms = _mean_pstdev(times)
        kept = [b.download(s) for b, s in zip(sc, scratch)] if keep_scratch else None
        return out.download(out_shape), mean_ms, std_ms, kept


def benchmark_kernel_events(impl, Q, K, V, batch_size, N_latent, N_input, D,
                            warmup=20, iters=100):
    """Time launcher ``impl`` (a LAUNCHERS key) with Q/K/V already in HBM.

    Inputs are copied to the device once; only the launches are timed, with
    HIP events.  Returns (output [batch_size, N_latent, D], mean_ms, std_ms).
    DesignLimited: the wave-per-latent rung past its LDS ceiling, or D != 768
    for the MFMA kernel -- raised before anything is allocated.
    """
    if impl == 'warp':
        _require_warp_lds(N_input)
    if impl == 'vectorized':
        _require_dim(D, "the MFMA kernel")
    launch_fn = LAUNCHERS[impl]
    inputs = [_prep(a, batch_size) for a in (Q, K, V)]

    def one(bufs, out, _):
        launch_fn(bufs[0].f32, bufs[1].f32, bufs[2].f32, out.f32, batch_size, N_latent,
                  N_input, D, _NULL_STREAM)

    out, mean_ms, std_ms, _ = _resident_run(
        one, inputs, (batch_size, N_latent, D), warmup, iters,
        f"kernel '{impl}' (N_latent={N_latent}, N_input={N_input})")
    return out, mean_ms, std_ms


def choose_num_splits(N_latent, N_input, batch_size, sm_count=142,
                      latents_per_block=4):
    """The reference's split heuristic, unchanged (cuda_wrappers.py:456-467):
    enough splits for about four workgroups of ``latents_per_block`` latents
    per compute unit, with at least 16 keys per split.  The reference's
    split-K drivers use it with latents_per_block = 4 (fp32) and 16 (fp16)
    when num_splits is None; ``sm_count`` 142 is its L40S default (MI355X
    has 256 compute units, see ``device_info``).
    """
    base = math.ceil(N_latent / latents_per_block) * batch_size
    target = max(1, (4 * sm_count) // max(1, base))
    return max(1, min(N_input // 16, target)) or 1


def _default_splits(num_splits, N_latent, N_input, batch_size, sm_count, latents_per_block,
                    keys_per_tile):
    """num_splits of a split-K driver: None -> the reference's default,
    choose_num_splits (cuda_wrappers.py:480-481, 553-555); "plan" -> the
    library's cost-model plan (plan_num_splits); an int is used as given."""
    if num_splits is None:
        return choose_num_splits(N_latent, N_input, batch_size, sm_count, latents_per_block)
    if isinstance(num_splits, str):
        if num_splits != "plan":
            raise ValueError(f"num_splits must be an int, None or 'plan' (got {num_splits!r})")
        return plan_num_splits(N_latent, N_input, batch_size, sm_count, keys_per_tile)
    return int(num_splits)


def _splitk_run(launch, inputs, batch_size, N_latent, N_input, D, num_splits, warmup, iters,
                what, keep_partials=False):
    """Event-time a split-K launcher whose caller-owned scratch (po, pm, pl)
    is allocated once.  ``launch`` takes the launcher's argument list with
    Q, K, V as DeviceBuffers.  Returns (output, mean_ms, std_ms) and, with
    ``keep_partials``, host copies of the (po, pm, pl) the last launch wrote."""
    rows = (batch_size, N_latent, num_splits)

    def one(bufs, out, sc):
        launch(bufs[0], bufs[1], bufs[2], out.f32, sc[0].f32, sc[1].f32, sc[2].f32,
               batch_size, N_latent, N_input, D, num_splits, _NULL_STREAM)

    out, mean_ms, std_ms, kept = _resident_run(
        one, inputs, (batch_size, N_latent, D), warmup, iters,
        f"{what} (N_latent={N_latent} N_input={N_input} splits={num_splits})",
        scratch=(rows + (D,), rows, rows), keep_scratch=keep_partials)
    if not keep_partials:
        return out, mean_ms, std_ms
    return out, mean_ms, std_ms, tuple(kept)


def benchmark_splitk_events(Q, K, V, batch_size, N_latent, N_input, D,
                            warmup=20, iters=100, num_splits=None, sm_count=142):
    """Event timing of launch_splitk_kernel (partials + LSE merge).

    The split scratch is allocated once with the inputs.  num_splits: None
    takes the reference's choose_num_splits(..., sm_count) with 4-latent
    blocks, "plan" the library's plan for ``sm_count`` compute units.
    Returns (output, mean_ms, std_ms, num_splits).
    """
    if not HAS_SPLITK:
        raise RuntimeError("this kernels.so does not export launch_splitk_kernel")
    _require_dim(D, "split-K")
    num_splits = _default_splits(num_splits, N_latent, N_input, batch_size, sm_count, 4,
                                 KEYS_PER_TILE_F32)
    inputs = [_prep(a, batch_size) for a in (Q, K, V)]
    launch = lambda q, k, v, *rest: lib.launch_splitk_kernel(  # noqa: E731
        q.f32, k.f32, v.f32, *rest)
    out, mean_ms, std_ms = _splitk_run(launch, inputs, batch_size, N_latent, N_input, D,
                                       num_splits, warmup, iters, "split-K")
    return out, mean_ms, std_ms, num_splits


def lse_combine(po, pm, pl, column_parts=0):
    """Merge host split partials on the GPU (xattn_lse_combine): po [rows, S,
    768], pm and pl [rows, S] -> output [rows, 768] fp32.  column_parts 0
    takes the library's choice; 1, 2 and 4 force that many workgroups per
    row (the output is the same bit for bit)."""
    if not HAS_LSE_COMBINE:
        raise RuntimeError("this kernels.so does not export xattn_lse_combine")
    po = np.ascontiguousarray(po, dtype=np.float32)
    pm = np.ascontiguousarray(pm, dtype=np.float32)
    pl = np.ascontiguousarray(pl, dtype=np.float32)
    rows, S, D = po.shape
    if D != 768 or pm.shape != (rows, S) or pl.shape != (rows, S):
        raise ValueError(f"partials of shapes {po.shape}, {pm.shape}, {pl.shape}: expected "
                         f"[rows, S, 768], [rows, S], [rows, S]")
    with DeviceBuffer.holding(po) as dpo, DeviceBuffer.holding(pm) as dpm, \
            DeviceBuffer.holding(pl) as dpl, DeviceBuffer(rows * D * 4) as out:
        lib.xattn_lse_combine(dpo.f32, dpm.f32, dpl.f32, out.f32, rows, S, int(column_parts),
                              _NULL_STREAM)
        _raise_launch_errors("xattn_lse_combine")
        _hip_check(cudart.hipDeviceSynchronize(), "xattn_lse_combine: waiting for the kernel")
        return out.download((rows, D))


def splitk_partials(Q, K, V, batch_size, N_latent, N_input, D, num_splits):
    """One launch_splitk_kernel call; returns (output, (po, pm, pl)), the
    caller-visible scratch in the reference's layout."""
    _require_dim(D, "split-K")
    inputs = [_prep(a, batch_size) for a in (Q, K, V)]
    launch = lambda q, k, v, *rest: lib.launch_splitk_kernel(  # noqa: E731
        q.f32, k.f32, v.f32, *rest)
    out, _, _, parts = _splitk_run(launch, inputs, batch_size, N_latent, N_input, D,
                                   num_splits, 1, 0, "split-K", keep_partials=True)
    return out, parts


# ---------------------------------------------------------------------------
# fp16 / bf16 MFMA paths
# ---------------------------------------------------------------------------

def _to_bf16_bits(x):
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return np.where(nan, (u >> 16) | 0x40, rounded).astype(np.uint16)


def _half_inputs(Q, K, V, batch_size, D, bf16):
    """Host side of the 16-bit paths: Q pre-scaled by 1/sqrt(D) in fp32, then
    Q, K, V rounded to fp16 or bf16 (cuda_wrappers.py:635-640)."""
    Q = _prep(Q, batch_size).astype(np.float32) / np.sqrt(D).astype(np.float32)
    K = _prep(K, batch_size)
    V = _prep(V, batch_size)
    if bf16:
        return tuple(np.ascontiguousarray(_to_bf16_bits(a)) for a in (Q, K, V))
    return tuple(np.ascontiguousarray(a, dtype=np.float16) for a in (Q, K, V))


def _wmma_events(launch_fn, what, Q, K, V, batch_size, N_latent, N_input, D, warmup, iters,
                 bf16):
    _require_dim(D, what)
    inputs = _half_inputs(Q, K, V, batch_size, D, bf16)

    def one(bufs, out, _):
        launch_fn(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, out.f32, batch_size, N_latent,
                  N_input, D, _NULL_STREAM)

    out, mean_ms, std_ms, _ = _resident_run(
        one, inputs, (batch_size, N_latent, D), warmup, iters,
        f"{what} (N_latent={N_latent} N_input={N_input})")
    return out, mean_ms, std_ms


def benchmark_wmma_events(Q, K, V, batch_size, N_latent, N_input, D,
                          warmup=20, iters=100):
    """Event timing of launch_wmma_kernel (fp16 MFMA, fp32 accumulate).

    fp32 Q/K/V in, as for the other drivers; Q is scaled by 1/sqrt(D) and all
    three are rounded to fp16 on the host.  Returns (fp32 output, mean_ms,
    std_ms).
    """
    if not HAS_WMMA:
        raise RuntimeError("this kernels.so does not export launch_wmma_kernel")
    return _wmma_events(lib.launch_wmma_kernel, "fp16 MFMA kernel", Q, K, V, batch_size,
                        N_latent, N_input, D, warmup, iters, bf16=False)


def benchmark_wmma_bf16_events(Q, K, V, batch_size, N_latent, N_input, D,
                               warmup=20, iters=100):
    """bf16 twin of ``benchmark_wmma_events`` (additive)."""
    if not HAS_WMMA_BF16:
        raise RuntimeError("this kernels.so does not export launch_wmma_bf16_kernel")
    return _wmma_events(lib.launch_wmma_bf16_kernel, "bf16 MFMA kernel", Q, K, V, batch_size,
                        N_latent, N_input, D, warmup, iters, bf16=True)


def _wmma_splitk(launch_fn, what, Q, K, V, batch_size, N_latent, N_input, D, warmup, iters,
                 num_splits, sm_count, bf16, keep_partials=False):
    _require_dim(D, what)
    num_splits = _default_splits(num_splits, N_latent, N_input, batch_size, sm_count, 16,
                                 KEYS_PER_TILE_F16)
    inputs = _half_inputs(Q, K, V, batch_size, D, bf16)
    launch = lambda q, k, v, *rest: launch_fn(q.ptr, k.ptr, v.ptr, *rest)  # noqa: E731
    res = _splitk_run(launch, inputs, batch_size, N_latent, N_input, D, num_splits,
                      warmup, iters, what, keep_partials=keep_partials)
    return res, num_splits


def benchmark_wmma_splitk_events(Q, K, V, batch_size, N_latent, N_input, D,
                                 warmup=20, iters=100, num_splits=None,
                                 sm_count=142):
    """Event timing of launch_wmma_splitk_kernel (fp16, key-parallel).

    Inputs prepared as for ``benchmark_wmma_events``; fp32 scratch and
    output.  num_splits: None takes the reference's choose_num_splits with
    16-latent blocks, "plan" the library's plan.  Returns (fp32 output,
    mean_ms, std_ms, num_splits).
    """
    if not HAS_WMMA_SPLITK:
        raise RuntimeError("this kernels.so does not export launch_wmma_splitk_kernel")
    (out, mean_ms, std_ms), s = _wmma_splitk(
        lib.launch_wmma_splitk_kernel, "fp16 split-K", Q, K, V, batch_size, N_latent,
        N_input, D, warmup, iters, num_splits, sm_count, bf16=False)
    return out, mean_ms, std_ms, s


def benchmark_wmma_splitk_bf16_events(Q, K, V, batch_size, N_latent, N_input, D,
                                      warmup=20, iters=100, num_splits=None,
                                      sm_count=142):
    """bf16 twin of ``benchmark_wmma_splitk_events`` (additive)."""
    if not HAS_WMMA_SPLITK_BF16:
        raise RuntimeError("this kernels.so does not export launch_wmma_splitk_bf16_kernel")
    (out, mean_ms, std_ms), s = _wmma_splitk(
        lib.launch_wmma_splitk_bf16_kernel, "bf16 split-K", Q, K, V, batch_size, N_latent,
        N_input, D, warmup, iters, num_splits, sm_count, bf16=True)
    return out, mean_ms, std_ms, s


def benchmark_plan_events(Q, K, V, batch_size, N_latent, N_input, D, latents_per_workgroup,
                          num_splits, column_parts=1, precision="fp32", warmup=20, iters=100):
    """Event timing of the fused path under a given launch plan instead of
    the library's (additive, for plan tuning): launch_optimized_plan_kernel
    for precision "fp32" (64, 32 or 16 latents per workgroup), else
    launch_wmma_plan_kernel ("fp16" or "bf16"; 64 latents in one or two
    column parts, or 32).  Returns (output, mean_ms, std_ms); a plan the
    library refuses raises RuntimeError before anything is timed."""
    _require_dim(D, "the MFMA kernels")
    what = (f"{precision} plan {latents_per_workgroup}/{column_parts}/{num_splits} "
            f"(N_latent={N_latent} N_input={N_input})")
    if precision == "fp32":
        if not HAS_OPTIMIZED_PLAN:
            raise RuntimeError("this kernels.so does not export launch_optimized_plan_kernel")
        inputs = tuple(_prep(a, batch_size) for a in (Q, K, V))

        def one(bufs, out, _):
            lib.launch_optimized_plan_kernel(bufs[0].f32, bufs[1].f32, bufs[2].f32, out.f32,
                                             batch_size, N_latent, N_input, D,
                                             latents_per_workgroup, num_splits, _NULL_STREAM)
    elif precision in ("fp16", "bf16"):
        if not HAS_WMMA_PLAN:
            raise RuntimeError("this kernels.so does not export launch_wmma_plan_kernel")
        bf16 = precision == "bf16"
        inputs = _half_inputs(Q, K, V, batch_size, D, bf16)

        def one(bufs, out, _):
            lib.launch_wmma_plan_kernel(int(bf16), bufs[0].ptr, bufs[1].ptr, bufs[2].ptr,
                                        out.f32, batch_size, N_latent, N_input, D,
                                        latents_per_workgroup, column_parts, num_splits,
                                        _NULL_STREAM)
    else:
        raise ValueError(f"precision {precision!r} is not fp32, fp16 or bf16")
    out, mean_ms, std_ms, _ = _resident_run(one, inputs, (batch_size, N_latent, D), warmup,
                                            iters, what)
    return out, mean_ms, std_ms


def wmma_splitk_partials(Q, K, V, batch_size, N_latent, N_input, D, num_splits, bf16=False):
    """Run the 16-bit split-K once; return (output, (po, pm, pl))."""
    fn = lib.launch_wmma_splitk_bf16_kernel if bf16 else lib.launch_wmma_splitk_kernel
    (out, _, _, parts), _ = _wmma_splitk(fn, "16-bit split-K", Q, K, V, batch_size, N_latent,
                                         N_input, D, 1, 0, num_splits, 142, bf16,
                                         keep_partials=True)
    return out, parts
