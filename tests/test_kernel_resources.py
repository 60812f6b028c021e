"""Resources of the built gfx950 kernels, read from the code object's own
metadata (no GPU): no kernel uses scratch memory or spills registers.

A kernel with a private segment writes that memory per lane on every launch
(12 bytes per lane in the token-major kernels once cost the 32-token mixed
layer a sixth of its routed gate/up time and most of its write traffic), so
the build keeps every kernel at zero."""
import os
import re
import subprocess

import pytest

LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


def kernel_metadata(tmp_path):
    from sabah.runtime import rt
    lib = rt.library_path()
    if not os.path.exists(lib):
        pytest.skip("libsabah_rt.so is not built")
    tools = {t: os.path.join(LLVM, t) for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-readelf")}
    if not all(os.access(p, os.X_OK) for p in tools.values()):
        pytest.skip("ROCm LLVM tools absent")
    fat, co = tmp_path / "fat.bin", tmp_path / "co.o"
    # objcopy writes a copy (an output path keeps the library itself untouched)
    subprocess.run([tools["llvm-objcopy"], "--dump-section", ".hip_fatbin=%s" % fat, lib, str(tmp_path / "copy.so")],
                   check=True, capture_output=True)
    subprocess.run([tools["clang-offload-bundler"], "--unbundle", "--type=o", "--input=%s" % fat,
                    "--targets=" + TARGET, "--output=%s" % co], check=True, capture_output=True)
    notes = subprocess.run([tools["llvm-readelf"], "--notes", str(co)], check=True, capture_output=True,
                           text=True).stdout
    kernels = []
    for block in re.split(r"\n\s+- \.agpr_count:", notes)[1:]:
        fields = dict(re.findall(r"^\s+\.(\w+):\s+(\S+)\s*$", block, flags=re.M))
        if "symbol" in fields:
            kernels.append(fields)
    return kernels


def test_no_kernel_uses_scratch_or_spills(tmp_path):
    kernels = kernel_metadata(tmp_path)
    assert len(kernels) >= 100, len(kernels)
    bad = [(k["name"], k.get("private_segment_fixed_size"), k.get("vgpr_spill_count"), k.get("sgpr_spill_count"))
           for k in kernels
           if int(k.get("private_segment_fixed_size", 0)) or int(k.get("vgpr_spill_count", 0))
           or int(k.get("sgpr_spill_count", 0))]
    assert not bad, bad
