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


# 16-bit gates: rel <= 2e-2 against the fp32 oracle on the unrounded inputs
# (the reduced-precision contract), and, against the oracle evaluated on the
# rounded inputs the kernel sees, the kernel's own error bound TIGHT16 (P
# rounded to 16 bits, fp32 accumulation), times a margin where the shapes
# are many and ragged.
GATE16 = 2e-2
TIGHT16 = {False: 1e-3, True: 4e-3}


def gate16(out, ref_unrounded, ref_rounded, bf16, margin=2.0):
    """Both 16-bit gates; returns (rel vs unrounded, rel vs rounded)."""
    import xattn_oracle as o
    assert np.all(np.isfinite(out)), "non-finite output"
    rel = o.rel_err(out, ref_unrounded)
    tight = o.rel_err(out, ref_rounded)
    assert rel <= GATE16, f"rel vs fp32 oracle {rel:.3e} > {GATE16}"
    assert tight <= margin * TIGHT16[bf16], \
        f"rel vs rounded-input oracle {tight:.3e} > {margin * TIGHT16[bf16]:.1e}"
    return rel, tight
