"""Register budgets of the gfx950 kernels, checked on the CPU from the compiler's own metadata.

The attention kernels' throughput depends on keeping every live value in registers: a launch
bound that the compiler can only meet by spilling VGPRs to scratch memory costs several percent
(a two-tile decode kernel that spilled 8-10 VGPRs measured 10 % slower on the MTP-verify
batch), and nothing else in the test suite would notice.  This compiles attention.hip for gfx950
(device code only, to assembly) and requires that no kernel spills VGPRs."""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_attention_kernels_do_not_spill_vgprs():
    src = os.path.join(ROOT, "lia.rs_amd", "csrc", "attention.hip")
    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "attention.s")
        subprocess.run([HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature",
                        "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S", src, "-o", out],
                       check=True, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
        text = open(out).read()
    kernels = {}
    for block in text.split("  - .agpr_count:")[1:]:
        name = re.search(r"\.name:\s+(\S+)", block)
        spill = re.search(r"\.vgpr_spill_count:\s+(\d+)", block)
        if name and spill:
            kernels[name.group(1)] = int(spill.group(1))
    assert any("attention_kernel" in k for k in kernels) and any("wide_kernel" in k for k in kernels)
    spilled = {k: v for k, v in kernels.items() if v > 0}
    assert not spilled, spilled
