"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

chia_proj_amd/csrc/attn_api.hip is compiled with the sanitizers on its host
side only (hipcc's -Xarch_host; the device code is built as usual and never
launched) and linked into tests/cpp/check_abi_host.cpp, which drives every
entry point that runs on the host alone: argument validation of the
forward, backward, allocation-free backward and FP8 entries, the
scratch-size refusal, planning (pair counts against a brute force over the
mask definition and against closed forms past 2^32 pairs), tile maps, query
intervals and their buffer-length checks.  No GPU is needed."""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = ROCM / "bin" / "hipcc"
CLANG = ROCM / "llvm" / "bin" / "clang++"
NO_PACKED_FP32 = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
HOST_SANITIZE = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                 "-Xarch_host", "-fno-sanitize-recover=all"]


@pytest.mark.skipif(not (HIPCC.exists() and CLANG.exists()), reason="ROCm compilers not available")
def test_abi_host_code_under_sanitizers(tmp_path):
    api = tmp_path / "attn_api.o"
    drv = tmp_path / "check_abi_host.o"
    exe = tmp_path / "check_abi_host"
    csrc = ROOT / "chia_proj_amd" / "csrc"
    inc = ROOT / "include"
    subprocess.run([str(HIPCC), "--offload-arch=gfx950", "-std=c++17", "-O1", "-g", "-fPIC", *NO_PACKED_FP32,
                    *HOST_SANITIZE, f"-I{inc}", f"-I{csrc}", "-c", str(csrc / "attn_api.hip"), "-o", str(api)],
                   check=True, capture_output=True)
    subprocess.run([str(CLANG), "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
                    "-fno-sanitize-recover=all", f"-I{inc}", "-c", str(ROOT / "tests" / "cpp" / "check_abi_host.cpp"),
                    "-o", str(drv)], check=True)
    subprocess.run([str(CLANG), "-fsanitize=address,undefined", str(drv), str(api), "-o", str(exe),
                    f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}"], check=True)
    # the HIP runtime keeps process-lifetime allocations: leak reports are off
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1")
    out = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "0 failures" in out.stdout
    assert "ERROR: AddressSanitizer" not in out.stderr and "runtime error" not in out.stderr
