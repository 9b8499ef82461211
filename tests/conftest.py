import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "fast-cuda-cross-attention_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests"),
          os.path.join(ROOT, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: long-running case")


@pytest.fixture(scope="session")
def cw():
    """cuda_wrappers over the in-tree kernels.so; fails loudly if it is absent."""
    so = os.path.join(PKG, "kernels.so")
    if not os.path.exists(so):
        raise RuntimeError(f"{so} is missing: run `make -C '{PKG}'` (or __graft_entry__.build())")
    import cuda_wrappers
    return cuda_wrappers


@pytest.fixture(scope="session")
def oracle():
    import xattn_oracle
    return xattn_oracle


def fp32_gate(out, ref, atol=1e-4, rtol=1e-3):
    """fp32 gate: max-abs <= 1e-4 and rel = max-abs / (max|ref| + 1e-6) <= 1e-3."""
    import xattn_oracle as o
    ma = o.max_abs(out, ref)
    rel = o.rel_err(out, ref)
    assert np.all(np.isfinite(out)), "non-finite output"
    assert ma <= atol and rel <= rtol, f"max_abs={ma:.3e} rel={rel:.3e}"
    return ma, rel
