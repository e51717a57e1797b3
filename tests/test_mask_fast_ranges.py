"""CPU checks of chia_proj_amd/csrc/mask.h by brute force: the kernel's
unclassified fast paths (fast_ranges, wide_range_all) and per-block class bounds
(KeyRanges) against classify_tile over
masks, residues, row blocks and key tiles (tests/cpp/check_fast_ranges.cpp), and
the multiply-high divider against plain division (tests/cpp/check_udiv.cpp),
the LDS tile layout against a bank model (tests/cpp/check_lds_banks.cpp),
the paired core's DMA / barrier schedule (tests/cpp/check_schedule.cpp) and the
one-block core's stepped tile keys (tests/cpp/check_tile_keys.cpp), all
built with AddressSanitizer and UndefinedBehaviorSanitizer."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
SANITIZE = ["-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all"]


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_fast_ranges_agree_with_classification(tmp_path):
    exe = tmp_path / "check_fast_ranges"
    subprocess.run(["g++", "-std=c++17", "-O1", *SANITIZE, f"-I{ROOT / 'chia_proj_amd' / 'csrc'}",
                    str(ROOT / "tests" / "cpp" / "check_fast_ranges.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "on a fast path" in out.stdout and "key-range classes" in out.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_udiv_matches_division(tmp_path):
    exe = tmp_path / "check_udiv"
    subprocess.run(["g++", "-std=c++17", "-O1", *SANITIZE, f"-I{ROOT / 'chia_proj_amd' / 'csrc'}",
                    str(ROOT / "tests" / "cpp" / "check_udiv.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "pairs" in out.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_lds_layout_is_bank_conflict_free(tmp_path):
    """The LDS chunk placement (csrc/lds_layout.h) against a 64-bank model that
    reproduces the conflict counters measured on the layout it replaced."""
    exe = tmp_path / "check_lds_banks"
    subprocess.run(["g++", "-std=c++17", "-O1", *SANITIZE, f"-I{ROOT / 'chia_proj_amd' / 'csrc'}",
                    str(ROOT / "tests" / "cpp" / "check_lds_banks.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "0 failures" in out.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_tile_schedule_is_safe(tmp_path):
    """The paired core's tile schedule (prologue, WIDE2 steps, pipelined run,
    vmcnt waits, stage reuse) over every workgroup of a mask and shape sweep:
    equal barriers in every wavefront, every read tile landed, no stage reused
    while read; and each of four planted schedule mistakes is caught."""
    exe = tmp_path / "check_schedule"
    subprocess.run(["g++", "-std=c++17", "-O1", *SANITIZE, f"-I{ROOT / 'chia_proj_amd' / 'csrc'}",
                    str(ROOT / "tests" / "cpp" / "check_schedule.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "0 violations" in out.stdout
    planted = subprocess.run([str(exe), "planted"], capture_output=True, text=True)
    assert planted.returncode == 0, planted.stdout + planted.stderr
    assert planted.stdout.count("planted mistake") == 4


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_one_block_split_schedule_is_safe(tmp_path):
    """The one-block core with two groups per workgroup (a zigzag pair's steps split
    between them, the shared block merged through LDS): every step computed once,
    equal barrier counts and roles in both groups, each group's two-stage DMA safe,
    the merge buffer inside the LDS; and each of four planted mistakes is caught."""
    exe = tmp_path / "check_q1_split"
    subprocess.run(["g++", "-std=c++17", "-O1", *SANITIZE, f"-I{ROOT / 'chia_proj_amd' / 'csrc'}",
                    str(ROOT / "tests" / "cpp" / "check_q1_split.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "0 violations" in out.stdout
    planted = subprocess.run([str(exe), "planted"], capture_output=True, text=True)
    assert planted.returncode == 0, planted.stdout + planted.stderr
    assert planted.stdout.count("planted mistake") == 4


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_stepped_tile_keys(tmp_path):
    """The one-block core's stepped tile keys (the full key only at a block's start, the
    prefix/band seam and the rotation's wrap) against the full formula, over random tile
    ranges, walk directions and group starts; each of two planted break mistakes is caught."""
    exe = tmp_path / "check_tile_keys"
    subprocess.run(["g++", "-std=c++17", "-O1", *SANITIZE, f"-I{ROOT / 'chia_proj_amd' / 'csrc'}",
                    str(ROOT / "tests" / "cpp" / "check_tile_keys.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "0 stepped keys differ" in out.stdout
    planted = subprocess.run([str(exe), "planted"], capture_output=True, text=True)
    assert planted.returncode == 0, planted.stdout + planted.stderr
    assert planted.stdout.count("planted mistake") == 2
