"""The C ABI used from C: tests/c/abi_client.c compiles with gcc against
include/xattn.h and links kernels.so (CPU); on a GPU it runs the fp32,
split-K and bf16 entry points and checks them against its own
double-precision reference."""

import os
import shutil
import subprocess

import pytest

from conftest import PKG, ROOT

SRC = os.path.join(ROOT, "tests", "c", "abi_client.c")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def _build(tmp_path):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not on PATH")
    exe = str(tmp_path / "abi_client")
    cmd = ["gcc", "-std=c11", "-O1", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
           f"-I{ROCM}/include", f"-I{os.path.join(ROOT, 'include')}", SRC,
           f"-L{PKG}", "-l:kernels.so", f"-Wl,-rpath,{PKG}", f"-L{ROCM}/lib", "-lamdhip64",
           f"-Wl,-rpath,{ROCM}/lib", "-lm", "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return exe


def test_c_client_builds_against_the_header(tmp_path):
    assert os.path.exists(os.path.join(PKG, "kernels.so")), "build kernels.so first"
    assert os.access(_build(tmp_path), os.X_OK)


@pytest.mark.gpu
def test_c_client_runs(tmp_path):
    exe = _build(tmp_path)
    print("running", exe, flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr
