"""Every kernel instantiation of the library compiles for gfx950 without scratch memory.

A register spill shows up as scratch stores on the HBM write path (the pipelined ReLU
forward once wrote 8 bytes per lane per wavefront, 2 MiB per north-star launch, that
way) and as reloads inside the tile loop.  The compiler's resource remarks
(-Rpass-analysis=kernel-resource-usage) give each kernel's ScratchSize; this test
compiles every HIP source of the library, device side only, and requires 0 for all,
and no VGPR spills.
"""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

from chia_proj_amd import _build

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
KERNEL_SOURCES = [s for s in _build.SOURCES if s != "attn_api.hip"]


def _resources(src: str) -> dict[str, dict[str, int]]:
    cmd = [HIPCC, *_build.HIPCC_FLAGS, f"-I{_build.INCLUDE}", f"-I{_build.CSRC}", "-c", "--cuda-device-only",
           "-Rpass-analysis=kernel-resource-usage", str(_build.CSRC / src), "-o", "/dev/null"]
    out = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=600)
    assert out.returncode == 0, out.stdout[-2000:]
    kernels: dict[str, dict[str, int]] = {}
    name = None
    for line in out.stdout.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            kernels[name] = {}
            continue
        m = re.search(r"remark:\s+(ScratchSize \[bytes/lane\]|VGPRs Spill|SGPRs Spill): (\d+)", line)
        if m and name:
            kernels[name][m.group(1).split()[0]] = int(m.group(2))
    return kernels


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc (ROCm) is not installed")
@pytest.mark.parametrize("src", KERNEL_SOURCES)
def test_no_scratch(src):
    kernels = _resources(src)
    assert kernels, f"no kernels reported for {src}"
    # (SGPR spills go to VGPR lanes, not to memory, and are allowed)
    bad = {k: v for k, v in kernels.items() if v.get("ScratchSize", 0) or v.get("VGPRs", 0)}
    assert not bad, f"{src}: kernels with scratch or spills: {bad}"
