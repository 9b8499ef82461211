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
