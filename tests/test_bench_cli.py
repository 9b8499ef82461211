"""bench.py's command-line contract that needs no GPU: more than one GPU is
refused with a message before anything is loaded, and the algorithmic work
figures match the headline workload's closed forms."""

import os
import subprocess
import sys

from conftest import ROOT


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=60, cwd=ROOT)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)
    assert not r.stdout.lstrip().startswith("{")  # no JSON line for a refused run


def test_algorithmic_work_of_the_headline():
    sys.path.insert(0, ROOT)
    import bench
    # 4 * B * NL * NI * D and the fused byte model with fp32 output
    assert bench.algorithmic_flop(32, 1024, 784, 768) == 4 * 32 * 1024 * 784 * 768
    assert round(bench.algorithmic_flop(32, 1024, 784, 768) / 1e9, 2) == 78.92
    assert bench.algorithmic_bytes(32, 1024, 784, 768) == 32 * (1024 + 2 * 784 + 1024) * 768 * 4
    assert bench.algorithmic_bytes(16, 512, 784, 768, 2) == 16 * ((512 + 2 * 784) * 2 + 512 * 4) * 768


class _FakeLib:
    """Stands in for kernels_phaseclock.so: xattn_phase_clock_read fills the
    [4096][8][6] stamp array with a chosen pattern."""

    def __init__(self, fill):
        self.fill = fill

        def read(dst, nbytes):
            import ctypes

            import numpy as np
            arr = np.ctypeslib.as_array((ctypes.c_uint64 * (nbytes // 8)).from_address(dst))
            self.fill(arr.reshape(4096, 8, 6))
            return 0

        self.xattn_phase_clock_read = read


class _FakeCw:
    def __init__(self, fill, lpw, splits):
        self.lib = _FakeLib(fill)
        self.lpw, self.splits = lpw, splits

    def device_info(self):
        return 256, 160 * 1024

    def wmma_plan(self, b, nl, ni, cu):
        return self.lpw, self.splits


def test_phase_clock_split_from_stamps():
    """phase_clock() turns the per-wavefront stamps (start, loop start, loop
    end, end; real-time start and end) into the prologue / loop / epilogue
    means, the clock, and the workgroups' start-time quantiles; only the
    launch's own workgroups and wavefronts count."""
    sys.path.insert(0, ROOT)
    import bench

    def fill(c):
        c[:] = 0
        blocks = 32 * 16  # headline: B=32, NL=1024 in 64-latent workgroups
        for b in range(blocks):
            base = 1000 * b
            c[b, :, 0] = base
            c[b, :, 1] = base + 100      # prologue 100 cycles
            c[b, :, 2] = base + 1100     # loop 1000
            c[b, :, 3] = base + 1300     # epilogue 200; lifetime 1300
            c[b, :, 4] = 5000 + (0 if b < 256 else 2600)  # two rounds, 26 us apart
            c[b, :, 5] = c[b, :, 4] + 65  # 1300 cycles in 0.65 us: 2.0 GHz
        c[blocks:, :, :] = 7  # stale stamps past the grid must not count

    rec = bench.phase_clock(_FakeCw(fill, 64, 1), "headline-bf16")
    assert rec["workgroups"] == 512 and rec["wavefronts"] == 8
    assert rec["cycles"] == {"lifetime": 1300.0, "prologue": 100.0, "tile_loop": 1000.0,
                             "epilogue": 200.0}
    assert rec["clock_ghz"] == 2.0
    assert rec["start_us_quantiles"][0] == 0.0 and rec["start_us_quantiles"][-1] == 26.0


def test_phase_clock_refuses_fp32_and_product_library():
    sys.path.insert(0, ROOT)
    import bench
    import pytest

    cw = _FakeCw(lambda c: None, 64, 1)
    with pytest.raises(ValueError):
        bench.phase_clock(cw, "cfg1")

    class NoClock:
        lib = object()
    with pytest.raises(RuntimeError, match="phaseclock"):
        bench.phase_clock(NoClock(), "headline-bf16")
