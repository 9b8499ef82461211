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
    """Stands in for kernels_phaseclock.so: xattn_phase_clock_read_* fills
    the [4096][8][9] stamp array with a chosen pattern."""

    def __init__(self, fill):
        self.cleared = 0

        def read(dst, nbytes):
            import ctypes

            import numpy as np
            arr = np.ctypeslib.as_array((ctypes.c_uint64 * (nbytes // 8)).from_address(dst))
            fill(arr.reshape(4096, 8, 9))
            return 0

        def clear():
            self.cleared += 1
            return 0

        self.xattn_phase_clock_read_f16 = self.xattn_phase_clock_read_f32 = read
        self.xattn_phase_clock_clear_f16 = self.xattn_phase_clock_clear_f32 = clear


class _FakeCw:
    def __init__(self, fill):
        self.lib = _FakeLib(fill)


def _fill_rounds(c, blocks, waves, tiles=False):
    c[:] = 0
    for b in range(blocks):
        base = 1000 * b
        c[b, :waves, 0] = base
        c[b, :waves, 1] = base + 100      # prologue 100 cycles
        c[b, :waves, 2] = base + 1100     # loop 1000
        c[b, :waves, 3] = base + 1300     # epilogue 200; lifetime 1300
        c[b, :waves, 4] = 5000 + (0 if b < blocks // 2 else 2600)  # two rounds, 26 us apart
        c[b, :waves, 5] = c[b, :waves, 4] + 65  # 1300 cycles in 0.65 us: 2.0 GHz
        if tiles:
            c[b, :waves, 6], c[b, :waves, 7], c[b, :waves, 8] = 100, 450, 450


def test_phase_clock_split_from_stamps():
    """phase_clock() turns the per-wavefront stamps (start, loop start, loop
    end, end; real-time start and end) into the prologue / loop / epilogue
    means, the clock, and the workgroups' start-time quantiles; workgroups
    and wavefronts that left no stamps do not count."""
    sys.path.insert(0, ROOT)
    import bench

    cw = _FakeCw(lambda c: _fill_rounds(c, 512, 8))
    bench.phase_clock_clear(cw, "headline-bf16")
    assert cw.lib.cleared == 1
    rec = bench.phase_clock(cw, "headline-bf16")
    assert rec["workgroups"] == 512 and rec["wavefronts"] == 8
    assert rec["cycles"] == {"lifetime": 1300.0, "prologue": 100.0, "tile_loop": 1000.0,
                             "epilogue": 200.0}
    assert rec["clock_ghz"] == 2.0
    assert rec["start_us_quantiles"][0] == 0.0 and rec["start_us_quantiles"][-1] == 26.0

    # the fp32 kernel: four wavefronts, and the loop's per-tile sums
    rec = bench.phase_clock(_FakeCw(lambda c: _fill_rounds(c, 512, 4, tiles=True)),
                            "headline-fp32")
    assert rec["wavefronts"] == 4
    assert rec["cycles"]["loop_waits"] == 100.0 and rec["cycles"]["loop_qk"] == 450.0


def test_phase_clock_needs_the_instrumented_library():
    sys.path.insert(0, ROOT)
    import bench
    import pytest

    class NoClock:
        lib = object()
    with pytest.raises(RuntimeError, match="phaseclock"):
        bench.phase_clock(NoClock(), "headline-bf16")
    with pytest.raises(RuntimeError, match="no phase-clock stamps"):
        bench.phase_clock(_FakeCw(lambda c: c.fill(0)), "cfg1")


def test_plan_option():
    """--plan LPW/CP/S parses into the three numbers, and an fp32 case
    refuses it before touching the device."""
    import argparse

    import pytest

    sys.path.insert(0, ROOT)
    import bench
    assert bench.parse_plan("64/2/1") == (64, 2, 1)
    assert bench.parse_plan("32/1/13") == (32, 1, 13)
    for bad in ("64/2", "a/b/c", "64-2-1"):
        with pytest.raises(argparse.ArgumentTypeError):
            bench.parse_plan(bad)
    with pytest.raises(ValueError, match="16-bit"):
        bench.run_case(None, "cfg1", 1, 1, plan=(64, 1, 1))


def test_exactly_warmup_then_steps_launches():
    """time_launches makes exactly `warmup` untimed launches and then `steps`
    timed ones, each timed launch between its own pair of events; the error
    state is read after the first launch and after the timed region."""
    import ctypes

    sys.path.insert(0, ROOT)
    import bench

    class Rt:
        def __init__(self):
            self.log = []

        def cudaDeviceSynchronize(self):
            self.log.append("sync")
            return 0

        def cudaEventCreate(self, p):
            return 0

        def cudaEventRecord(self, ev, stream):
            self.log.append("event")
            return 0

        def cudaEventElapsedTime(self, out, a, b):
            ctypes.cast(out, ctypes.POINTER(ctypes.c_float)).contents.value = 0.5
            return 0

        def cudaEventDestroy(self, ev):
            return 0

    class Cw:
        def __init__(self):
            self.cudart = Rt()
            self.checks = 0

        def _lib_error_check(self, what):
            self.checks += 1
            self.cudart.log.append("check")

    for warmup, steps in ((5, 20), (0, 3), (1, 1)):
        cw = Cw()
        wall, per = bench.time_launches(
            cw, lambda: cw.cudart.log.append("launch"), steps, warmup)
        log = cw.cudart.log
        assert log.count("launch") == warmup + steps and len(per) == steps
        assert all(x == 0.5 for x in per)
        timed = log[log.index("event"):]
        assert timed.count("launch") == steps and timed.count("event") == 2 * steps
        assert log[:log.index("event")].count("launch") == warmup
        assert cw.checks == (2 if warmup else 1)
