"""The gfx950 code objects inside the built kernels.so: every flash and merge
kernel runs without a private (scratch) segment and fits the CU's LDS.

A register spill in these kernels is a performance defect that no parity
test sees: the 64-latent 16-bit form once reloaded a Q fragment from scratch
in every tile, behind a wait for all global->LDS DMA in flight.  This test
reads the kernel descriptors' metadata from the library itself (LLVM's
offload bundler and readelf, from the ROCm toolchain), so it needs no GPU.
"""

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SO = os.path.join(ROOT, "fast-cuda-cross-attention_amd", "kernels.so")
LLVM = "/opt/rocm/llvm/bin"
TOOLS = [os.path.join(LLVM, t) for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-readelf")]
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
LDS_BYTES = 160 * 1024


def _kernels(tmp_path):
    """{kernel symbol: metadata fields} over every gfx950 code object of kernels.so."""
    objcopy, bundler, readelf = TOOLS
    fatbin = tmp_path / "fatbin.bin"
    subprocess.run([objcopy, f"--dump-section=.hip_fatbin={fatbin}", SO, str(tmp_path / "so")],
                   check=True, capture_output=True)
    data = fatbin.read_bytes()
    # one offload bundle per translation unit, concatenated by the linker
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    assert starts, "no offload bundle in .hip_fatbin"
    out = {}
    for i, s in enumerate(starts):
        e = starts[i + 1] if i + 1 < len(starts) else len(data)
        bundle, co = tmp_path / f"b{i}.bin", tmp_path / f"co{i}.o"
        bundle.write_bytes(data[s:e])
        subprocess.run([bundler, "--unbundle", "--type=o", f"--targets={TARGET}",
                        f"--input={bundle}", f"--output={co}"], check=True, capture_output=True)
        notes = subprocess.run([readelf, "--notes", str(co)], check=True, capture_output=True,
                               text=True).stdout
        # Within a kernel's entry the keys are sorted: its arguments' .name
        # fields come first, then the kernel's own .name, then
        # .private_segment_fixed_size; .group_segment_fixed_size precedes both.
        name, group = None, None
        for line in notes.splitlines():
            m = re.match(r"\s*-?\s*\.(\w+):\s+(\S+)", line)
            if not m:
                continue
            key, val = m.groups()
            if key == "group_segment_fixed_size":
                group = int(val)
            elif key == "name":
                name = val
            elif key == "private_segment_fixed_size" and name is not None:
                out[name] = {"private": int(val), "group": group}
                name, group = None, None
    return out


@pytest.fixture(scope="module")
def kernels(tmp_path_factory):
    if not os.path.exists(SO):
        raise RuntimeError(f"{SO} is missing: run `make -C fast-cuda-cross-attention_amd`")
    missing = [t for t in TOOLS if not shutil.which(t)]
    if missing:
        pytest.skip(f"ROCm LLVM tools not found: {missing}")
    return _kernels(tmp_path_factory.mktemp("code_objects"))


def test_every_instantiation_is_present(kernels):
    names = list(kernels)
    assert sum("flash_f32_kernel" in n for n in names) == 6   # {split, full} x DS {1, 2, 4}
    assert sum("flash16_kernel" in n for n in names) == 12    # {fp16, bf16} x split x 3 forms
    assert sum("lse_combine_kernel" in n for n in names) == 4
    assert any("naive_kernel" in n for n in names)


def test_hot_kernels_do_not_spill(kernels):
    hot = {n: k for n, k in kernels.items()
           if any(s in n for s in ("flash_f32_kernel", "flash16_kernel", "lse_combine_kernel"))}
    spilled = {n: k["private"] for n, k in hot.items() if k["private"] != 0}
    assert not spilled, f"kernels with a scratch segment (bytes per lane): {spilled}"


def test_lds_fits_one_cu(kernels):
    over = {n: k["group"] for n, k in kernels.items() if (k["group"] or 0) > LDS_BYTES}
    assert not over, f"LDS over {LDS_BYTES} bytes: {over}"
