"""The 4x4x4 skinny kernel issues its weight loads as explicit instructions whose destination
registers stay in flight until a later wait; the compiler takes them as written at
issue, so a kernel that spilled (or reused a spilled register) before the wait would have the
load's data land in a register that by then holds something else.  Every instantiation must
therefore use no scratch.  This compiles each source for gfx950 with the library's own flags
(device code only, to assembly) and checks each kernel's private segment size.  CPU only."""
import os
import re
import subprocess
import tempfile

import pytest

from nemotron_infer_amd import build

HIPCC = build.HIPCC


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
@pytest.mark.parametrize("source,min_kernels", [("skinny4_fp8.hip", 10)])
def test_skinny_kernels_use_no_scratch(source, min_kernels):
    src = os.path.join(build.CSRC, source)
    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "kernels.s")
        subprocess.run([HIPCC, *build.HIP_FLAGS, "--cuda-device-only", "-S", src, "-o", out], check=True,
                       capture_output=True)
        asm = open(out).read()
    kernels = re.findall(r"\.amdhsa_kernel (\S+)(.*?)\.end_amdhsa_kernel", asm, re.S)
    assert len(kernels) >= min_kernels, "kernel descriptors not found in the assembly"
    spilled = []
    for name, body in kernels:
        m = re.search(r"\.amdhsa_private_segment_fixed_size\s+(\d+)", body)
        assert m, name
        if int(m.group(1)) != 0:
            spilled.append((name, int(m.group(1))))
    assert not spilled, spilled
