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
    raise RuntimeError("Could not find the HIP runtime library (libamdhip64.so). "
                       "Please ensure ROCm is installed. Tried: " + "; ".join(errs))


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
    raise RuntimeError(f"Failed to load HIP runtime: {e}")

# ---------------------------------------------------------------------------
# kernels.so
# ---------------------------------------------------------------------------

_HERE = os.path.dirname(os.path.abspath(__file__))
KERNELS_SO = os.environ.get("XATTN_KERNELS_SO") or os.path.join(_HERE, "kernels.so")
if not os.path.exists(KERNELS_SO) and os.path.exists("./kernels.so"):
    KERNELS_SO = os.path.abspath("./kernels.so")

try:
    lib = ctypes.CDLL(KERNELS_SO)
except OSError:
    raise RuntimeError(f"Failed to load kernels.so ({KERNELS_SO}). Please compile the HIP "
                       f"kernels first using 'make' in {_HERE}.")

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

# fp16 MFMA kernel: half* Q/K/V (passed as void*), float* output.
HAS_WMMA = _bind_optional("launch_wmma_kernel", _WMMA_ARGS)
# Split-K (key-parallel) kernel: Q/K/V/out + po/pm/pl scratch + num_splits.
HAS_SPLITK = _bind_optional("launch_splitk_kernel", _SPLITK_ARGS)
# fp16 MFMA split-K: half Q/K/V (void*) + float out/po/pm/pl + num_splits.
HAS_WMMA_SPLITK = _bind_optional("launch_wmma_splitk_kernel", _WMMA_SPLITK_ARGS)
# bf16 twins (additive)
HAS_WMMA_BF16 = _bind_optional("launch_wmma_bf16_kernel", _WMMA_ARGS)
HAS_WMMA_SPLITK_BF16 = _bind_optional("launch_wmma_splitk_bf16_kernel", _WMMA_SPLITK_ARGS)


class DesignLimited(RuntimeError):
    """Raised when a kernel cannot run a config by design (not a bug).

    Used by the warp-parallel kernel: it materializes the full score row in
    LDS, so N_input is capped by the device's per-workgroup LDS limit.  Beyond
    that we skip cleanly and the benchmark records the config as
    'design-limited'.  Also raised for a dim the MFMA kernels are not built
    for (they are built for D = 768).
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
    """Device max LDS per workgroup, in bytes (the reference's opt-in shared
    memory limit, cuda_wrappers.py:187-194)."""
    try:
        _, lds = device_info(device)
    except RuntimeError:
        return 48 * 1024  # conservative default, as the reference
    return lds if lds > 0 else 48 * 1024


def warp_smem_bytes(N_input):
    """LDS the warp kernel needs for a given N_input."""
    return (4 * N_input + 4) * 4


def _require_dim(D, what):
    if D != D_MODEL:
        raise DesignLimited(f"{what} is built for D={D_MODEL} (got D={D})")


def _allocate_gpu_memory(size_bytes):
    """Allocate GPU memory."""
    ptr = ctypes.c_void_p()
    err = cudart.cudaMalloc(ctypes.byref(ptr), max(int(size_bytes), 1))
    if err != 0:
        raise RuntimeError(f"hipMalloc failed with error {err}")
    return ptr


def _copy_to_gpu(host_data, gpu_ptr, size_bytes):
    """Copy data from host to GPU."""
    if size_bytes == 0:
        return
    host_ptr = host_data.ctypes.data_as(ctypes.c_void_p)
    err = cudart.cudaMemcpy(gpu_ptr, host_ptr, size_bytes, cudaMemcpyHostToDevice)
    if err != 0:
        raise RuntimeError(f"hipMemcpy H2D failed with error {err}")


def _copy_from_gpu(gpu_ptr, host_data, size_bytes):
    """Copy data from GPU to host."""
    if size_bytes == 0:
        return
    host_ptr = host_data.ctypes.data_as(ctypes.c_void_p)
    err = cudart.cudaMemcpy(host_ptr, gpu_ptr, size_bytes, cudaMemcpyDeviceToHost)
    if err != 0:
        raise RuntimeError(f"hipMemcpy D2H failed with error {err}")


def _free_gpu_memory(ptr):
    """Free GPU memory."""
    cudart.cudaFree(ptr)


def _fptr(p):
    return ctypes.cast(p, ctypes.POINTER(ctypes.c_float))


def _check_after_launch(what):
    _lib_error_check(what)
    err = cudart.cudaGetLastError()
    if err != 0:
        raise RuntimeError(f"Kernel launch failed with HIP error {err}. "
                           f"This usually indicates a kernel configuration problem, "
                           f"invalid memory access, or architecture incompatibility.")


def _run_kernel(kernel_func, Q, K, V, batch_size, N_latent, N_input, D):
    """Helper function to run a kernel with batch support (alloc, copy,
    launch, sync, copy back, free; cuda_wrappers.py:228-289)."""

    Q = np.ascontiguousarray(Q, dtype=np.float32)
    K = np.ascontiguousarray(K, dtype=np.float32)
    V = np.ascontiguousarray(V, dtype=np.float32)

    Q_size = Q.size * 4
    K_size = K.size * 4
    V_size = V.size * 4
    output_size = batch_size * N_latent * D * 4

    Q_gpu = _allocate_gpu_memory(Q_size)
    K_gpu = _allocate_gpu_memory(K_size)
    V_gpu = _allocate_gpu_memory(V_size)
    output_gpu = _allocate_gpu_memory(output_size)

    try:
        err = cudart.cudaMemset(output_gpu, 0, max(output_size, 1))
        if err != 0:
            raise RuntimeError(f"hipMemset failed with error {err}")

        _copy_to_gpu(Q, Q_gpu, Q_size)
        _copy_to_gpu(K, K_gpu, K_size)
        _copy_to_gpu(V, V_gpu, V_size)

        kernel_func(_fptr(Q_gpu), _fptr(K_gpu), _fptr(V_gpu), _fptr(output_gpu),
                    batch_size, N_latent, N_input, D, ctypes.c_void_p(0))

        _check_after_launch(getattr(kernel_func, "__name__", "kernel"))

        err = cudart.cudaDeviceSynchronize()
        if err != 0:
            err_detail = cudart.cudaGetLastError()
            raise RuntimeError(f"[ERROR] hipDeviceSynchronize failed with error {err}, "
                               f"last HIP error: {err_detail}. "
                               f"This usually indicates a kernel execution error, "
                               f"such as invalid memory access or illegal instruction.")

        output = np.zeros((batch_size, N_latent, D), dtype=np.float32)
        _copy_from_gpu(output_gpu, output, output_size)
        return output
    finally:
        _free_gpu_memory(Q_gpu)
        _free_gpu_memory(K_gpu)
        _free_gpu_memory(V_gpu)
        _free_gpu_memory(output_gpu)


def _batchify(Q, K, V):
    if len(Q.shape) == 3:
        return Q.shape[0], Q, K, V
    return (1, np.expand_dims(Q, axis=0).astype(np.float32),
            np.expand_dims(K, axis=0).astype(np.float32),
            np.expand_dims(V, axis=0).astype(np.float32))


def run_naive_kernel(Q, K, V, N_latent, N_input, D):
    """Run the naive kernel (baseline - one thread per output element)."""
    batch_size, Q, K, V = _batchify(Q, K, V)
    return _run_kernel(lib.launch_naive_kernel, Q, K, V, batch_size, N_latent, N_input, D)


def run_warp_parallel_kernel(Q, K, V, N_latent, N_input, D):
    """Run the wave-per-latent kernel.

    Raises DesignLimited when N_input exceeds what fits in the device's
    per-workgroup LDS -- the kernel materializes the full score row, so this
    is a hard design limit, not a failure.
    """
    needed = warp_smem_bytes(N_input)
    avail = _max_smem_optin()
    if needed > avail:
        raise DesignLimited(
            f"warp kernel needs {needed/1024:.1f} KB LDS for "
            f"N_input={N_input} but device allows {avail/1024:.1f} KB/block "
            f"(materializes full score row; use tiled/vectorized instead)")
    batch_size, Q, K, V = _batchify(Q, K, V)
    return _run_kernel(lib.launch_parallel_kernel, Q, K, V, batch_size, N_latent, N_input, D)


def run_tiled_kernel(Q, K, V, N_latent, N_input, D):
    """Run the tiled kernel (LDS tiling + online softmax)."""
    batch_size, Q, K, V = _batchify(Q, K, V)
    return _run_kernel(lib.launch_tiled_kernel, Q, K, V, batch_size, N_latent, N_input, D)


def run_vectorized_kernel(Q, K, V, N_latent, N_input, D):
    """Run the fast fp32 kernel (fp32 MFMA, online softmax)."""
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
    """Normalize Q/K/V to a contiguous fp32 [batch_size, n, D] array."""
    arr = np.ascontiguousarray(arr, dtype=np.float32)
    if arr.ndim == 2:
        arr = arr[None]
    if arr.shape[0] == 1 and batch_size > 1:
        arr = np.repeat(arr, batch_size, axis=0)
    return np.ascontiguousarray(arr, dtype=np.float32)


class _Events:
    def __init__(self):
        self.start = ctypes.c_void_p()
        self.stop = ctypes.c_void_p()
        cudart.cudaEventCreate(ctypes.byref(self.start))
        cudart.cudaEventCreate(ctypes.byref(self.stop))

    def time(self, launch, iters, stream=None):
        stream = stream if stream is not None else ctypes.c_void_p(0)
        times = []
        ms = ctypes.c_float(0.0)
        for _ in range(iters):
            cudart.cudaEventRecord(self.start, stream)
            launch()
            cudart.cudaEventRecord(self.stop, stream)
            cudart.cudaEventSynchronize(self.stop)
            cudart.cudaEventElapsedTime(ctypes.byref(ms), self.start, self.stop)
            times.append(ms.value)
        return times

    def destroy(self):
        cudart.cudaEventDestroy(self.start)
        cudart.cudaEventDestroy(self.stop)


def _stats(times):
    if not times:
        return 0.0, 0.0
    return statistics.mean(times), (statistics.pstdev(times) if len(times) > 1 else 0.0)


def _warmup(launch, warmup, what):
    launch()
    _lib_error_check(what)
    for _ in range(max(warmup - 1, 0)):
        launch()
    if cudart.cudaDeviceSynchronize() != 0:
        raise RuntimeError(f"{what} failed during warmup (HIP error "
                           f"{cudart.cudaGetLastError()})")


def benchmark_kernel_events(impl, Q, K, V, batch_size, N_latent, N_input, D,
                            warmup=20, iters=100):
    """Kernel-only GPU timing via HIP events.

    Allocates device buffers and copies Q/K/V to the GPU ONCE, then times only
    the kernel launches with the data resident.  Returns (output, mean_ms,
    std_ms).  Raises DesignLimited for the warp kernel when N_input exceeds
    the device's per-workgroup LDS, and for the MFMA kernel when D != 768.
    """
    if impl == 'warp':
        needed = warp_smem_bytes(N_input)
        avail = _max_smem_optin()
        if needed > avail:
            raise DesignLimited(
                f"warp needs {needed/1024:.1f} KB LDS for "
                f"N_input={N_input}, device allows {avail/1024:.1f} KB/block")
    if impl == 'vectorized':
        _require_dim(D, "the MFMA kernel")
    launch_fn = LAUNCHERS[impl]

    Q = _prep(Q, batch_size)
    K = _prep(K, batch_size)
    V = _prep(V, batch_size)

    Q_size, K_size, V_size = Q.size * 4, K.size * 4, V.size * 4
    out_size = batch_size * N_latent * D * 4

    Q_gpu = _allocate_gpu_memory(Q_size)
    K_gpu = _allocate_gpu_memory(K_size)
    V_gpu = _allocate_gpu_memory(V_size)
    out_gpu = _allocate_gpu_memory(out_size)
    ev = _Events()

    try:
        cudart.cudaMemset(out_gpu, 0, max(out_size, 1))
        _copy_to_gpu(Q, Q_gpu, Q_size)
        _copy_to_gpu(K, K_gpu, K_size)
        _copy_to_gpu(V, V_gpu, V_size)

        qp, kp, vp, op = _fptr(Q_gpu), _fptr(K_gpu), _fptr(V_gpu), _fptr(out_gpu)
        null_stream = ctypes.c_void_p(0)

        def _launch():
            launch_fn(qp, kp, vp, op, batch_size, N_latent, N_input, D, null_stream)

        _warmup(_launch, warmup, f"kernel '{impl}' (N_input={N_input}, N_latent={N_latent})")
        times = ev.time(_launch, iters, null_stream)

        output = np.zeros((batch_size, N_latent, D), dtype=np.float32)
        _copy_from_gpu(out_gpu, output, out_size)
        mean_ms, std_ms = _stats(times)
        return output, mean_ms, std_ms
    finally:
        ev.destroy()
        _free_gpu_memory(Q_gpu)
        _free_gpu_memory(K_gpu)
        _free_gpu_memory(V_gpu)
        _free_gpu_memory(out_gpu)


def choose_num_splits(N_latent, N_input, batch_size, sm_count=142,
                      latents_per_block=4):
    """Pick num_splits so the partial-kernel grid oversubscribes the GPU.

    Base workgroups (no split) = ceil(Nl/latents_per_block)*batch.  Aim for
    ~4x sm_count workgroups, capped so each split still holds >= ~16 keys
    (cuda_wrappers.py:456-467).  On MI355X pass sm_count=256 (compute units;
    see ``device_info``).
    """
    base = math.ceil(N_latent / latents_per_block) * batch_size
    target = max(1, (4 * sm_count) // max(1, base))
    return max(1, min(N_input // 16, target)) or 1


def _splitk_run(launch, Qd, Kd, Vd, batch_size, N_latent, N_input, D, num_splits,
                warmup, iters, what, keep_partials=False):
    """Shared body of the split-K event drivers: Qd/Kd/Vd are host arrays in
    the element type the launcher takes; scratch po/pm/pl is allocated once."""
    out_size = batch_size * N_latent * D * 4
    po_size = batch_size * N_latent * num_splits * D * 4
    pml_size = batch_size * N_latent * num_splits * 4

    Q_gpu = _allocate_gpu_memory(Qd.nbytes)
    K_gpu = _allocate_gpu_memory(Kd.nbytes)
    V_gpu = _allocate_gpu_memory(Vd.nbytes)
    out_gpu = _allocate_gpu_memory(out_size)
    po_gpu = _allocate_gpu_memory(po_size)
    pm_gpu = _allocate_gpu_memory(pml_size)
    pl_gpu = _allocate_gpu_memory(pml_size)
    ev = _Events()
    try:
        cudart.cudaMemset(out_gpu, 0, max(out_size, 1))
        _copy_to_gpu(Qd, Q_gpu, Qd.nbytes)
        _copy_to_gpu(Kd, K_gpu, Kd.nbytes)
        _copy_to_gpu(Vd, V_gpu, Vd.nbytes)
        null_stream = ctypes.c_void_p(0)

        def _launch():
            launch(Q_gpu, K_gpu, V_gpu, _fptr(out_gpu), _fptr(po_gpu), _fptr(pm_gpu),
                   _fptr(pl_gpu), batch_size, N_latent, N_input, D, num_splits, null_stream)

        _warmup(_launch, warmup,
                f"{what} (Nl={N_latent} Ni={N_input} splits={num_splits})")
        times = ev.time(_launch, iters, null_stream)

        output = np.zeros((batch_size, N_latent, D), dtype=np.float32)
        _copy_from_gpu(out_gpu, output, out_size)
        mean_ms, std_ms = _stats(times)
        if keep_partials:
            po = np.zeros((batch_size, N_latent, num_splits, D), np.float32)
            pm = np.zeros((batch_size, N_latent, num_splits), np.float32)
            pl = np.zeros((batch_size, N_latent, num_splits), np.float32)
            _copy_from_gpu(po_gpu, po, po_size)
            _copy_from_gpu(pm_gpu, pm, pml_size)
            _copy_from_gpu(pl_gpu, pl, pml_size)
            return output, mean_ms, std_ms, (po, pm, pl)
        return output, mean_ms, std_ms
    finally:
        ev.destroy()
        for p in (Q_gpu, K_gpu, V_gpu, out_gpu, po_gpu, pm_gpu, pl_gpu):
            _free_gpu_memory(p)


def benchmark_splitk_events(Q, K, V, batch_size, N_latent, N_input, D,
                            warmup=20, iters=100, num_splits=None, sm_count=142):
    """HIP-event timing for the split-K (key-parallel) kernel.

    Allocates Q/K/V/out AND the partial scratch (po/pm/pl) once, then times the
    partial+combine launches.  Returns (output, mean_ms, std_ms, num_splits).
    """
    if not HAS_SPLITK:
        raise RuntimeError("kernels.so has no launch_splitk_kernel (rebuild "
                           "with csrc/xattn_flash_f32.hip).")
    _require_dim(D, "split-K")
    if num_splits is None:
        num_splits = plan_num_splits(N_latent, N_input, batch_size, sm_count)
    Q = _prep(Q, batch_size)
    K = _prep(K, batch_size)
    V = _prep(V, batch_size)
    launch = lambda q, k, v, *rest: lib.launch_splitk_kernel(  # noqa: E731
        _fptr(q), _fptr(k), _fptr(v), *rest)
    out, mean_ms, std_ms = _splitk_run(launch, Q, K, V, batch_size, N_latent, N_input, D,
                                       num_splits, warmup, iters, "split-K")
    return out, mean_ms, std_ms, num_splits


def splitk_partials(Q, K, V, batch_size, N_latent, N_input, D, num_splits):
    """Run launch_splitk_kernel once; return (output, (po, pm, pl)) -- the
    caller-visible scratch the reference's split-K writes."""
    _require_dim(D, "split-K")
    Q = _prep(Q, batch_size)
    K = _prep(K, batch_size)
    V = _prep(V, batch_size)
    launch = lambda q, k, v, *rest: lib.launch_splitk_kernel(  # noqa: E731
        _fptr(q), _fptr(k), _fptr(v), *rest)
    out, _, _, parts = _splitk_run(launch, Q, K, V, batch_size, N_latent, N_input, D,
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
    Qh, Kh, Vh = _half_inputs(Q, K, V, batch_size, D, bf16)
    out_size = batch_size * N_latent * D * 4
    Q_gpu = _allocate_gpu_memory(Qh.nbytes)
    K_gpu = _allocate_gpu_memory(Kh.nbytes)
    V_gpu = _allocate_gpu_memory(Vh.nbytes)
    out_gpu = _allocate_gpu_memory(out_size)
    ev = _Events()
    try:
        cudart.cudaMemset(out_gpu, 0, max(out_size, 1))
        _copy_to_gpu(Qh, Q_gpu, Qh.nbytes)
        _copy_to_gpu(Kh, K_gpu, Kh.nbytes)
        _copy_to_gpu(Vh, V_gpu, Vh.nbytes)
        op = _fptr(out_gpu)
        null_stream = ctypes.c_void_p(0)

        def _launch():
            launch_fn(Q_gpu, K_gpu, V_gpu, op, batch_size, N_latent, N_input, D, null_stream)

        _warmup(_launch, warmup, f"{what} (Nl={N_latent} Ni={N_input})")
        times = ev.time(_launch, iters, null_stream)
        output = np.zeros((batch_size, N_latent, D), dtype=np.float32)
        _copy_from_gpu(out_gpu, output, out_size)
        mean_ms, std_ms = _stats(times)
        return output, mean_ms, std_ms
    finally:
        ev.destroy()
        for p in (Q_gpu, K_gpu, V_gpu, out_gpu):
            _free_gpu_memory(p)


def benchmark_wmma_events(Q, K, V, batch_size, N_latent, N_input, D,
                          warmup=20, iters=100):
    """HIP-event timing for the fp16 MFMA kernel.

    Takes fp32 Q/K/V (same references the other kernels use), pre-scales Q by
    1/sqrt(D), casts to fp16, runs the MFMA kernel, and returns (fp32 output,
    mean_ms, std_ms).
    """
    if not HAS_WMMA:
        raise RuntimeError("kernels.so has no launch_wmma_kernel (rebuild with "
                           "csrc/xattn_flash_f16.hip).")
    return _wmma_events(lib.launch_wmma_kernel, "fp16 MFMA kernel", Q, K, V, batch_size,
                        N_latent, N_input, D, warmup, iters, bf16=False)


def benchmark_wmma_bf16_events(Q, K, V, batch_size, N_latent, N_input, D,
                               warmup=20, iters=100):
    """bf16 twin of ``benchmark_wmma_events`` (additive)."""
    if not HAS_WMMA_BF16:
        raise RuntimeError("kernels.so has no launch_wmma_bf16_kernel.")
    return _wmma_events(lib.launch_wmma_bf16_kernel, "bf16 MFMA kernel", Q, K, V, batch_size,
                        N_latent, N_input, D, warmup, iters, bf16=True)


def _wmma_splitk(launch_fn, what, Q, K, V, batch_size, N_latent, N_input, D, warmup, iters,
                 num_splits, sm_count, bf16, keep_partials=False):
    _require_dim(D, what)
    if num_splits is None:
        num_splits = plan_num_splits(N_latent, N_input, batch_size, sm_count,
                                     KEYS_PER_TILE_F16)
    Qh, Kh, Vh = _half_inputs(Q, K, V, batch_size, D, bf16)
    launch = lambda q, k, v, *rest: launch_fn(q, k, v, *rest)  # noqa: E731
    res = _splitk_run(launch, Qh, Kh, Vh, batch_size, N_latent, N_input, D, num_splits,
                      warmup, iters, what, keep_partials=keep_partials)
    return res, num_splits


def benchmark_wmma_splitk_events(Q, K, V, batch_size, N_latent, N_input, D,
                                 warmup=20, iters=100, num_splits=None,
                                 sm_count=142):
    """HIP-event timing for the fp16 MFMA split-K kernel (fp16 + key-split).

    fp16 Q/K/V (Q pre-scaled by 1/sqrt(D)), fp32 scratch + output.  Returns
    (fp32 output, mean_ms, std_ms, num_splits).
    """
    if not HAS_WMMA_SPLITK:
        raise RuntimeError("kernels.so has no launch_wmma_splitk_kernel "
                           "(rebuild with csrc/xattn_flash_f16.hip).")
    (out, mean_ms, std_ms), s = _wmma_splitk(
        lib.launch_wmma_splitk_kernel, "fp16 split-K", Q, K, V, batch_size, N_latent,
        N_input, D, warmup, iters, num_splits, sm_count, bf16=False)
    return out, mean_ms, std_ms, s


def benchmark_wmma_splitk_bf16_events(Q, K, V, batch_size, N_latent, N_input, D,
                                      warmup=20, iters=100, num_splits=None,
                                      sm_count=142):
    """bf16 twin of ``benchmark_wmma_splitk_events`` (additive)."""
    if not HAS_WMMA_SPLITK_BF16:
        raise RuntimeError("kernels.so has no launch_wmma_splitk_bf16_kernel.")
    (out, mean_ms, std_ms), s = _wmma_splitk(
        lib.launch_wmma_splitk_bf16_kernel, "bf16 split-K", Q, K, V, batch_size, N_latent,
        N_input, D, warmup, iters, num_splits, sm_count, bf16=True)
    return out, mean_ms, std_ms, s


def wmma_splitk_partials(Q, K, V, batch_size, N_latent, N_input, D, num_splits, bf16=False):
    """Run the 16-bit split-K once; return (output, (po, pm, pl))."""
    fn = lib.launch_wmma_splitk_bf16_kernel if bf16 else lib.launch_wmma_splitk_kernel
    (out, _, _, parts), _ = _wmma_splitk(fn, "16-bit split-K", Q, K, V, batch_size, N_latent,
                                         N_input, D, 1, 0, num_splits, 142, bf16,
                                         keep_partials=True)
    return out, parts
