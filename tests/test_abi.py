"""CPU tests of the C ABI and the host logic of the drop-in wrapper.

No kernel runs here: these cover that kernels.so loads and exports every
symbol include/xattn.h declares, the launch-planning helpers, argument
validation (refused before any HIP call), and the wrapper's pure-Python
policy (choose_num_splits, DesignLimited thresholds, _prep broadcasting).
"""

import ctypes
import os
import re

import numpy as np
import pytest

from conftest import PKG, ROOT


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "xattn.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:launch|xattn)_\w+)\s*\(", text)))


def test_header_declares_reference_entry_points():
    names = _declared_symbols()
    # the seven launchers of the reference's kernels.so (cuda_wrappers.py:83-175)
    for n in ("launch_naive_kernel", "launch_parallel_kernel", "launch_tiled_kernel",
              "launch_optimized_kernel", "launch_wmma_kernel", "launch_splitk_kernel",
              "launch_wmma_splitk_kernel"):
        assert n in names


def test_library_exports_every_declared_symbol(cw):
    lib = ctypes.CDLL(os.path.join(PKG, "kernels.so"))
    missing = [n for n in _declared_symbols() if not hasattr(lib, n)]
    assert not missing, f"kernels.so lacks {missing}"


def test_wrapper_flags(cw):
    assert cw.HAS_SPLITK
    assert set(cw.LAUNCHERS) == {"naive", "warp", "tiled", "vectorized"}
    assert cw.cudart.cudaMalloc is cw.cudart.hipMalloc


def test_xcd_remap_is_bijection(cw):
    for n in (1, 7, 8, 9, 64, 255, 256, 257, 512, 1000):
        got = sorted(cw.lib.xattn_xcd_remap(b, n) for b in range(n))
        assert got == list(range(n)), n
    # blocks dealt to one XCD (b % 8 == x) get consecutive logical ids
    n = 512
    for x in range(8):
        ids = [cw.lib.xattn_xcd_remap(b, n) for b in range(x, n, 8)]
        assert ids == list(range(ids[0], ids[0] + len(ids)))


def test_optimized_num_splits(cw):
    f = cw.lib.xattn_optimized_num_splits
    assert f(32, 1024, 784, 256) == 1      # 512 workgroups already fill 256 CUs
    assert f(1, 64, 784, 256) == 25        # 4 x 16-latent blocks, two 16-key tiles per split
    assert f(4, 1024, 784, 256) == 1       # 256 x 16-latent blocks, unsplit
    assert f(1, 256, 50176, 256) == 64     # 4 x 64-latent blocks x 64 splits of 49 tiles
    assert f(1, 64, 0, 256) == 1
    for b, nl, ni in [(1, 1, 1), (2, 100, 33), (1, 64, 17), (3, 7, 5000)]:
        s = f(b, nl, ni, 256)
        tiles = (ni + 15) // 16
        assert 1 <= s <= tiles
        chunk_tiles = -(-tiles // s)
        assert -(-tiles // chunk_tiles) == s  # tile-aligned chunks leave no empty split


def test_f32_plan(cw):
    # (latents per workgroup, key splits) of launch_optimized_kernel on 256
    # CUs, against the workgroup sizes and split counts timed on an MI355X at
    # that shape (HIP events around each of 300 launches); repeated timings
    # of one plan spread by a few per cent.
    assert cw.f32_plan(32, 1024, 784, 256) == (64, 1)    # 512 x 64-latent blocks
    assert cw.f32_plan(16, 512, 784, 256) == (32, 1)     # 256 x 32-latent blocks: one round
    assert cw.f32_plan(8, 1024, 784, 256) == (32, 1)
    assert cw.f32_plan(12, 1024, 784, 256) == (16, 1)    # 0.8 % ahead of (32, 2)
    assert cw.f32_plan(4, 1024, 784, 256) == (16, 1)     # 3.5 % ahead of (32, 2)
    assert cw.f32_plan(1, 1024, 784, 256) == (16, 4)     # 3.6 % ahead of (32, 7)
    assert cw.f32_plan(1, 256, 784, 256) == (16, 13)
    assert cw.f32_plan(1, 64, 784, 256) == (16, 25)
    assert cw.f32_plan(1, 256, 4096, 256) == (16, 16)    # 0.9 % ahead of (32, 32)
    assert cw.f32_plan(1, 256, 16384, 256) == (32, 32)
    assert cw.f32_plan(1, 256, 50176, 256) == (64, 64)
    assert cw.f32_plan(1, 64, 0, 256) == (64, 1)
    split = cw.lib.xattn_f32_split_latents
    assert split(1, 256, 50176, 64, 256) == 64           # 4 x 64 splits fill the device
    assert split(1, 256, 4096, 32, 256) == 32
    assert split(1, 256, 4096, 16, 256) == 16
    assert split(1, 1, 1, 1, 256) == 16                  # one tile: four wavefronts share it
    for b, nl, ni in [(1, 1, 1), (2, 100, 33), (3, 7, 5000), (64, 64, 784), (5, 300, 784),
                      (2, 70, 300), (1, 40, 200)]:
        lpw, s = cw.f32_plan(b, nl, ni, 256)
        tiles = -(-ni // 16)
        assert lpw in (16, 32, 64) and 1 <= s <= tiles
        assert s == cw.lib.xattn_optimized_num_splits(b, nl, ni, 256)
        ct = -(-tiles // s)
        assert -(-tiles // ct) == s  # whole-tile chunks leave no empty split
        # launch_splitk_kernel with the planned splits and the same chunks
        # picks the same workgroup size
        if -(-(-(-ni // s)) // 16) == ct:
            assert split(b, nl, ni, s, 256) == lpw


def test_wmma_plan(cw):
    # (latents per workgroup, column parts, key splits) of launch_wmma_kernel
    # on 256 CUs, against every form and split count timed at that shape on
    # an MI355X (through launch_wmma_plan_kernel, bf16 and fp16); repeated
    # timings of one plan spread by a few per cent.
    form = cw.wmma_plan_form
    assert form(32, 1024, 784, 256) == (64, 1, 1)    # measured best
    assert form(16, 512, 784, 256) == (32, 1, 1)     # measured best
    assert form(8, 1024, 784, 256) == (32, 1, 1)     # measured best
    assert form(8, 512, 784, 256) == (64, 2, 1)      # measured best
    assert form(4, 1024, 784, 256) == (64, 2, 1)     # measured best
    assert form(1, 1024, 16384, 256) == (64, 1, 16)  # measured best
    assert form(16, 256, 784, 256) == (64, 2, 1)     # fp16 best; bf16 2.7 % behind (64, 1, 3)
    assert form(16, 512, 1568, 256) == (64, 1, 2)    # 1 % behind (32, 1, 1)
    assert form(1, 64, 784, 256) == (64, 2, 25)      # 1 % behind (64, 2, 13)
    assert form(1, 256, 4096, 256) == (64, 2, 26)    # within 1 % of (64, 2, 22)
    assert form(1, 256, 784, 256) == (64, 2, 13)     # 3.5 % behind (64, 2, 7)
    assert form(2, 256, 50176, 256) == (64, 1, 32)   # 9 % ahead of the best timed, (64, 1, 25)
    assert form(1, 64, 20, 256) == (64, 2, 1)       # one tile: nothing to split
    for b, nl, ni in [(32, 1024, 784), (1, 256, 4096), (1, 64, 20)]:
        assert cw.wmma_plan(b, nl, ni, 256) == (form(b, nl, ni, 256)[0], form(b, nl, ni, 256)[2])
    split = cw.lib.xattn_wmma_split_latents
    assert split(1, 256, 50176, 64, 256) == 64
    assert split(16, 512, 784, 1, 256) == 32
    for b, nl, ni in [(1, 1, 1), (2, 100, 33), (3, 7, 5000), (64, 64, 784), (1, 256, 4096),
                      (16, 512, 784)]:
        lpw, cp, s = form(b, nl, ni, 256)
        tiles = -(-ni // 32)
        assert (lpw, cp) in ((64, 1), (64, 2), (32, 1)) and 1 <= s <= tiles
        ct = -(-tiles // s)
        assert -(-tiles // ct) == s  # whole-tile chunks leave no empty split
        # the split-K entry with the planned splits and the same chunk picks
        # the same workgroup size
        chunk = -(-(-(-ni // s)) // 16) * 16
        if -(-min(chunk, ni) // 32) == ct:
            assert split(b, nl, ni, s, 256) == lpw


def test_wmma_plan_launch_refuses_other_plans(cw):
    """launch_wmma_plan_kernel takes the three forms only and whole-tile
    split counts 1..ceil(N_input / 32); anything else is refused before any
    HIP call (so no GPU is needed to see it)."""
    P = ctypes.c_void_p
    F = ctypes.POINTER(ctypes.c_float)
    dummy = ctypes.cast(P(0x1000), F)
    q = P(0x1000)
    s0 = P(0)
    for lpw, cp, s in [(16, 1, 1), (32, 2, 1), (64, 3, 1), (64, 1, 0), (64, 2, 26), (32, 1, -1)]:
        code, msg = _call(cw, "launch_wmma_plan_kernel", 1, q, q, q, dummy, 1, 64, 784, 768,
                          lpw, cp, s, s0)
        assert code == 1, (lpw, cp, s, msg)
        assert ("column parts" in msg) if s >= 1 and s <= 25 else ("num_splits" in msg), msg
    code, msg = _call(cw, "launch_wmma_plan_kernel", 0, q, q, q, dummy, 1, 64, 784, 100,
                      64, 1, 1, s0)
    assert code == 2 and "dim=100" in msg
    # an empty problem is a no-op, whatever the (valid) plan
    code, _ = _call(cw, "launch_wmma_plan_kernel", 0, q, q, q, dummy, 0, 64, 784, 768, 64, 2, 3,
                    s0)
    assert code == 0


def test_split_drivers_default_to_the_reference_heuristic(cw):
    """num_splits=None in the split-K drivers means what it means in the
    reference (cuda_wrappers.py:480-481, 553-555): choose_num_splits with
    4-latent blocks for fp32 and 16-latent blocks for fp16, at the caller's
    sm_count (default 142).  "plan" asks for the library's own plan."""
    d = cw._default_splits
    f32, f16 = cw.KEYS_PER_TILE_F32, cw.KEYS_PER_TILE_F16
    assert d(None, 256, 4096, 1, 142, 4, f32) == 8
    assert d(None, 256, 4096, 1, 256, 4, f32) == 16
    assert d(None, 256, 4096, 1, 142, 16, f16) == 35
    assert d(None, 256, 4096, 1, 256, 16, f16) == 64
    assert d(None, 1024, 784, 32, 142, 4, f32) == 1
    assert d(7, 256, 4096, 1, 142, 4, f32) == 7
    assert d("plan", 256, 4096, 1, 256, 4, f32) == cw.f32_plan(1, 256, 4096, 256)[1]
    assert d("plan", 256, 4096, 1, 256, 16, f16) == cw.wmma_plan(1, 256, 4096, 256)[1]
    with pytest.raises(ValueError):
        d("auto", 256, 4096, 1, 256, 4, f32)


def test_choose_num_splits_known_values(cw):
    # values worked out by hand from cuda_wrappers.py:456-467
    assert cw.choose_num_splits(256, 4096, 1) == 8            # sm 142, lpb 4
    assert cw.choose_num_splits(256, 4096, 1, sm_count=256) == 16
    assert cw.choose_num_splits(256, 4096, 1, latents_per_block=16) == 35
    assert cw.choose_num_splits(256, 4096, 1, sm_count=256, latents_per_block=16) == 64
    assert cw.choose_num_splits(1024, 784, 32) == 1            # headline
    assert cw.choose_num_splits(64, 8, 1) == 1                 # N_input // 16 == 0 -> 1


def test_warp_design_limit(cw, monkeypatch):
    monkeypatch.setattr(cw, "_max_smem_optin", lambda device=0: 160 * 1024)
    assert cw.warp_smem_bytes(10239) <= 160 * 1024 < cw.warp_smem_bytes(10240)
    q = np.zeros((1, 4, 768), np.float32)
    k = np.zeros((1, 10240, 768), np.float32)
    with pytest.raises(cw.DesignLimited):
        cw.run_warp_parallel_kernel(q, k, k, 4, 10240, 768)
    with pytest.raises(cw.DesignLimited):
        cw.benchmark_kernel_events("warp", q, k, k, 1, 4, 10240, 768)


def test_mfma_paths_refuse_other_dims(cw):
    q = np.zeros((1, 4, 64), np.float32)
    with pytest.raises(cw.DesignLimited):
        cw.run_vectorized_kernel(q, q, q, 4, 4, 64)
    with pytest.raises(cw.DesignLimited):
        cw.benchmark_splitk_events(q, q, q, 1, 4, 4, 64)


def test_prep_broadcasting(cw):
    a = np.arange(2 * 3, dtype=np.float64).reshape(2, 3)
    got = cw._prep(a, 4)
    assert got.dtype == np.float32 and got.flags.c_contiguous and got.shape == (4, 2, 3)
    assert np.array_equal(got, np.repeat(a[None].astype(np.float32), 4, axis=0))
    b3 = np.ones((3, 2, 3))
    assert cw._prep(b3, 3).shape == (3, 2, 3)


def _call(cw, name, *args):
    fn = getattr(cw.lib, name)
    fn(*args)
    return cw.lib.xattn_get_last_error(), cw.lib.xattn_get_last_error_string().decode()


def test_optimized_plan_launch_refuses_other_plans(cw):
    """launch_optimized_plan_kernel takes 64, 32 or 16 latents per workgroup
    and whole-tile split counts 1..ceil(N_input / 16) only, refused before
    any HIP call."""
    F = ctypes.POINTER(ctypes.c_float)
    dummy = ctypes.cast(ctypes.c_void_p(0x1000), F)
    s0 = ctypes.c_void_p(0)
    for lpw, s, what in [(8, 1, "latents"), (48, 1, "latents"), (64, 0, "num_splits"),
                         (16, 50, "num_splits"), (32, -2, "num_splits")]:
        code, msg = _call(cw, "launch_optimized_plan_kernel", dummy, dummy, dummy, dummy, 1, 64,
                          784, 768, lpw, s, s0)
        assert code == 1 and what in msg, (lpw, s, msg)
    # an empty problem is a no-op, whatever the (valid) plan
    code, _ = _call(cw, "launch_optimized_plan_kernel", dummy, dummy, dummy, dummy, 1, 0, 784,
                    768, 16, 49, s0)
    assert code == 0


def test_noalloc_refuses_plans_past_its_scratch(cw):
    """launch_optimized_kernel_noalloc takes launch_optimized_kernel's plan;
    when that plan's split partials exceed the 64 MiB static scratch it is
    refused before any HIP call (so no GPU is needed to see it)."""
    F = ctypes.POINTER(ctypes.c_float)
    dummy = ctypes.cast(ctypes.c_void_p(0x1000), F)
    b, nl, ni = 28, 1792, 50176
    lpw, s = cw.f32_plan(b, nl, ni, 256)
    assert s > 1 and b * nl * s * 770 * 4 > (64 << 20)
    code, msg = _call(cw, "launch_optimized_kernel_noalloc", dummy, dummy, dummy, dummy, b, nl,
                      ni, 768, ctypes.c_void_p(0))
    assert code == 2 and "static scratch" in msg and f"{s} key splits" in msg, msg
    code, msg = _call(cw, "launch_optimized_kernel_noalloc", dummy, dummy, dummy, dummy, 1, 64,
                      784, 100, ctypes.c_void_p(0))
    assert code == 2 and "dim=100" in msg


def test_validation_refuses_before_launch(cw):
    """Refused arguments never reach the HIP runtime (no GPU is needed)."""
    F = ctypes.POINTER(ctypes.c_float)
    dummy = ctypes.cast(ctypes.c_void_p(0x1000), F)
    null = ctypes.cast(ctypes.c_void_p(0), F)
    s0 = ctypes.c_void_p(0)
    code, msg = _call(cw, "launch_optimized_kernel", dummy, dummy, dummy, dummy, 1, 64, 784,
                      100, s0)
    assert code == 2 and "dim=100" in msg
    code, msg = _call(cw, "launch_optimized_kernel", dummy, dummy, dummy, dummy, -1, 64, 784,
                      768, s0)
    assert code == 1 and "negative" in msg
    code, msg = _call(cw, "launch_optimized_kernel", null, dummy, dummy, dummy, 1, 64, 784,
                      768, s0)
    assert code == 1 and "NULL" in msg
    code, msg = _call(cw, "launch_splitk_kernel", dummy, dummy, dummy, dummy, dummy, dummy,
                      dummy, 1, 64, 784, 768, 0, s0)
    assert code == 1 and "num_splits" in msg
    code, msg = _call(cw, "launch_tiled_kernel", dummy, dummy, dummy, dummy, 1, 4, 4, 769, s0)
    assert code == 2
    # the MFMA paths move rows in 16-byte vectors: every operand must be aligned
    odd = ctypes.cast(ctypes.c_void_p(0x1004), F)
    code, msg = _call(cw, "launch_optimized_kernel", dummy, odd, dummy, dummy, 1, 64, 784, 768,
                      s0)
    assert code == 1 and "K pointer" in msg and "16-byte" in msg
    P = ctypes.c_void_p
    code, msg = _call(cw, "launch_wmma_splitk_bf16_kernel", P(0x1000), P(0x1000), P(0x1000),
                      dummy, odd, dummy, dummy, 1, 64, 784, 768, 2, s0)
    assert code == 1 and "partial output" in msg
    code, msg = _call(cw, "launch_wmma_kernel", P(0x1002), P(0x1000), P(0x1000), dummy, 1, 64,
                      784, 768, s0)
    assert code == 1 and "Q pointer" in msg
    # the scalar rungs take any float pointer
    code, _ = _call(cw, "launch_tiled_kernel", dummy, dummy, dummy, dummy, 0, 4, 4, 768, s0)
    assert code == 0
    # the error is cleared once read
    assert cw.lib.xattn_get_last_error() == 0
    # empty problems are a no-op, not an error
    code, _ = _call(cw, "launch_optimized_kernel", null, null, null, null, 0, 0, 0, 768, s0)
    assert code == 0


def test_unread_errors_keep_the_first(cw):
    """Two refusals with no read between them: the code and the message are
    both the first one's, like hipGetLastError; once read, the next refusal
    is recorded afresh."""
    F = ctypes.POINTER(ctypes.c_float)
    dummy = ctypes.cast(ctypes.c_void_p(0x1000), F)
    s0 = ctypes.c_void_p(0)
    cw.lib.launch_optimized_kernel(dummy, dummy, dummy, dummy, 1, 64, 784, 100, s0)
    cw.lib.launch_optimized_kernel(dummy, dummy, dummy, dummy, -1, 64, 784, 768, s0)
    code, msg = cw.lib.xattn_get_last_error(), cw.lib.xattn_get_last_error_string().decode()
    assert code == 2 and "dim=100" in msg and "negative" not in msg, msg
    # the message stays readable after the code was read
    assert "dim=100" in cw.lib.xattn_get_last_error_string().decode()
    code, msg = _call(cw, "launch_optimized_kernel", dummy, dummy, dummy, dummy, -1, 64, 784,
                      768, s0)
    assert code == 1 and "negative" in msg, msg


def test_merge_column_parts_choice(cw):
    """Workgroups per row of the LSE merge: the most of 1, 2 or 4 that leave
    at most one workgroup per CU (one for a single split)."""
    parts = cw.lib.xattn_lse_combine_parts
    assert parts(64, 25, 256) == 4     # configuration 1: 64 rows, 25 splits
    assert parts(65, 8, 256) == 2
    assert parts(128, 8, 256) == 2
    assert parts(129, 8, 256) == 1
    assert parts(256, 8, 256) == 1     # configuration 4: 256 rows
    assert parts(512, 8, 256) == 1
    assert parts(64, 1, 256) == 1
    assert parts(0, 4, 256) == 1


def test_merge_refuses_bad_arguments(cw):
    """xattn_lse_combine refuses other column parts, num_splits < 1 and NULL
    partials before any HIP call."""
    F = ctypes.POINTER(ctypes.c_float)
    dummy = ctypes.cast(ctypes.c_void_p(0x1000), F)
    null = ctypes.cast(ctypes.c_void_p(0), F)
    s0 = ctypes.c_void_p(0)
    for parts in (3, 8, -1):
        code, msg = _call(cw, "xattn_lse_combine", dummy, dummy, dummy, dummy, 64, 25, parts, s0)
        assert code == 1 and "column_parts" in msg, msg
    code, msg = _call(cw, "xattn_lse_combine", dummy, dummy, dummy, dummy, 64, 0, 0, s0)
    assert code == 1 and "num_splits" in msg, msg
    code, msg = _call(cw, "xattn_lse_combine", null, dummy, dummy, dummy, 64, 4, 0, s0)
    assert code == 1 and "NULL" in msg, msg
    code, msg = _call(cw, "xattn_lse_combine", dummy, dummy, dummy, dummy, -1, 4, 0, s0)
    assert code == 1 and "negative" in msg, msg
