"""CPU: the build's kernel-resource guard.  `build.resource_usage` reads
clang's kernel-resource-usage remarks; the build fails when any kernel uses
scratch memory (a register-indexed private array or argument block costs
every launch)."""
from __future__ import annotations

from pathlib import Path

import pytest

from cubic_serve_amd import build

REMARKS = """\
x.hip:35:1: remark: Function Name: _ZN5cubic4kernAEv [-Rpass-analysis=kernel-resource-usage]
   35 | __global__ void kernA() {
x.hip:35:1: remark:     TotalSGPRs: 57 [-Rpass-analysis=kernel-resource-usage]
x.hip:35:1: remark:     VGPRs: 134 [-Rpass-analysis=kernel-resource-usage]
x.hip:35:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:35:1: remark:     Occupancy [waves/SIMD]: 3 [-Rpass-analysis=kernel-resource-usage]
x.hip:35:1: remark:     SGPRs Spill: 84 [-Rpass-analysis=kernel-resource-usage]
x.hip:35:1: remark:     LDS Size [bytes/block]: 38920 [-Rpass-analysis=kernel-resource-usage]
x.hip:90:1: remark: Function Name: _ZN5cubic4kernBEv [-Rpass-analysis=kernel-resource-usage]
x.hip:90:1: remark:     VGPRs: 211 [-Rpass-analysis=kernel-resource-usage]
x.hip:90:1: remark:     ScratchSize [bytes/lane]: 312 [-Rpass-analysis=kernel-resource-usage]
x.hip:90:1: remark:     Dynamic Stack: False [-Rpass-analysis=kernel-resource-usage]
"""


def test_resource_remarks_parse_per_kernel():
    u = build.resource_usage(REMARKS)
    assert set(u) == {"_ZN5cubic4kernAEv", "_ZN5cubic4kernBEv"}
    a, b = u["_ZN5cubic4kernAEv"], u["_ZN5cubic4kernBEv"]
    assert a["VGPRs"] == 134 and a["ScratchSize [bytes/lane]"] == 0 and a["Occupancy [waves/SIMD]"] == 3
    assert a["SGPRs Spill"] == 84 and a["LDS Size [bytes/block]"] == 38920 and a["TotalSGPRs"] == 57
    assert b["ScratchSize [bytes/lane]"] == 312 and "Dynamic Stack" not in b  # non-numeric values skipped


def test_built_library_has_no_scratch_kernels():
    """When the library has been built here, its resource summary lists every
    kernel and none uses scratch (the build refuses otherwise)."""
    summary = Path(build.LIB_DIR) / "resources.txt"
    if not summary.exists():
        pytest.skip("library not built in this tree")
    lines = summary.read_text().splitlines()
    assert len(lines) > 100
    assert all(" scratch=0 " in ln for ln in lines), [ln for ln in lines if " scratch=0 " not in ln][:3]
