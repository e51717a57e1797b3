"""Build recipe for the gfx950 shared library ``libchia_attn.so`` (in-tree).

The library is compiled with ``hipcc`` for gfx950 only and linked into the
package directory, where :mod:`chia_proj_amd._lib` loads it with ctypes.  The
three translation units compile in parallel (the two head-dim halves of the
kernel instantiations and the C-ABI file).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_NAME = "libchia_attn.so"
LIB_PATH = PKG_DIR / LIB_NAME
BUILD_DIR = REPO_DIR / "_build"

SOURCES = ["attn_fwd_d64.hip", "attn_fwd_d128.hip", "attn_fwd_q1_d64.hip", "attn_fwd_q1_d128.hip", "attn_bwd_d64.hip", "attn_bwd_d128.hip", "attn_fp8.hip", "attn_api.hip"]
HEADERS = ["attn_fwd_kernel.h", "attn_fwd_q1_kernel.h", "lds_layout.h", "mask.h"]

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    # Packed fp32 VALU forms are disabled for every HIP file of this library.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libchia_attn.so")
    return path


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line and line.strip()
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out:
        print(out, file=sys.stderr)


def build(verbose: bool = True, extra_flags: list[str] | None = None) -> Path:
    """Compile every HIP source for gfx950 and link ``libchia_attn.so``."""
    BUILD_DIR.mkdir(exist_ok=True)
    cc = hipcc()
    flags = HIPCC_FLAGS + [f"-I{INCLUDE}", f"-I{CSRC}"] + list(extra_flags or [])
    objs = []
    cmds = []
    for src in SOURCES:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([cc, *flags, "-c", str(CSRC / src), "-o", str(obj)])
    if verbose:
        print(f"[chia_proj_amd] compiling {len(cmds)} HIP sources for {ARCH}", file=sys.stderr)
    with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1)) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[chia_proj_amd] built {LIB_PATH}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
