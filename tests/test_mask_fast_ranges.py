"""CPU check of the kernel's unclassified fast paths: fast_ranges
(chia_proj_amd/csrc/mask.h) against classify_tile by brute force over masks,
residues, row blocks and key tiles (tests/cpp/check_fast_ranges.cpp)."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_fast_ranges_agree_with_classification(tmp_path):
    exe = tmp_path / "check_fast_ranges"
    subprocess.run(["g++", "-std=c++17", "-O1", f"-I{ROOT / 'chia_proj_amd' / 'csrc'}",
                    str(ROOT / "tests" / "cpp" / "check_fast_ranges.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "on a fast path" in out.stdout
