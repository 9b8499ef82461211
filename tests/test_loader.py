"""How cuda_wrappers.py loads kernels.so, on the CPU (no kernel runs): a
missing library is a RuntimeError at import (reference cuda_wrappers.py:
77-81), and a library without the optional entry points still loads with
their HAS_* flags False (reference cuda_wrappers.py:136-175)."""

import json
import os
import shutil
import subprocess
import sys

import pytest

from conftest import PKG, ROOT

FLAGS = ["HAS_WMMA", "HAS_SPLITK", "HAS_WMMA_SPLITK", "HAS_WMMA_BF16",
         "HAS_WMMA_SPLITK_BF16", "HAS_NOALLOC", "HAS_WMMA_PLAN", "HAS_OPTIMIZED_PLAN"]


def _import_in_child(env_so, cwd):
    code = ("import json, sys; sys.path.insert(0, %r); import cuda_wrappers as cw; "
            "print(json.dumps({f: getattr(cw, f, None) for f in %r}))" % (PKG, FLAGS))
    env = dict(os.environ, XATTN_KERNELS_SO=env_so)
    return subprocess.run([sys.executable, "-c", code], cwd=cwd, env=env,
                          capture_output=True, text=True, timeout=120)


def test_missing_library_raises_runtime_error(tmp_path):
    r = _import_in_child(str(tmp_path / "no_such_dir" / "kernels.so"), str(tmp_path))
    assert r.returncode != 0
    assert "RuntimeError" in r.stderr and "kernels.so" in r.stderr, r.stderr[-2000:]


def test_library_without_optional_entry_points(tmp_path):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not on PATH")
    so = str(tmp_path / "kernels.so")
    src = os.path.join(ROOT, "tests", "c", "stub_kernels.c")
    b = subprocess.run(["gcc", "-shared", "-fPIC", "-O1", src, "-o", so],
                       capture_output=True, text=True, timeout=120)
    assert b.returncode == 0, b.stderr
    r = _import_in_child(so, str(tmp_path))
    assert r.returncode == 0, r.stderr[-2000:]
    flags = json.loads(r.stdout.strip().splitlines()[-1])
    assert flags == {f: False for f in FLAGS}


def test_in_tree_library_has_every_entry_point(cw):
    for f in FLAGS:
        assert getattr(cw, f) is True, f
