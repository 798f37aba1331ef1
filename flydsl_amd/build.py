"""Build recipe for libpa_fp8.so (hand-written gfx950 HIP kernels + C ABI).

``python flydsl_amd/build.py`` compiles the library in-tree next to this file (run it
by path: importing the package first would try to load the library).
hipcc cross-compiles for gfx950 without a GPU, so this runs anywhere the ROCm
toolchain is installed.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
LIB_PATH = HERE / "libpa_fp8.so"
SOURCES = [HERE / "csrc" / "pa_decode.hip", HERE / "csrc" / "pa_metadata.hip", HERE / "csrc" / "rope_cache.hip"]
HEADERS = [HERE / "csrc" / "pa_common.h", REPO / "include" / "pa_fp8.h"]
OFFLOAD_ARCH = "gfx950"


def hipcc() -> str:
    return os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def compile_command(out: Path, extra=()) -> list:
    return [
        hipcc(),
        f"--offload-arch={OFFLOAD_ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-I",
        str(REPO / "include"),
        # packed fp32 VALU forms are kept out of the device code
        "-Xclang",
        "-target-feature",
        "-Xclang",
        "-packed-fp32-ops",
        *extra,
        *[str(s) for s in SOURCES],
        "-o",
        str(out),
    ]


def build(verbose: bool = False, extra=()) -> Path:
    """Compile every HIP source into ``flydsl_amd/libpa_fp8.so`` (always rebuilds)."""
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = compile_command(tmp, extra)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose=True, extra=tuple(sys.argv[1:]))
    print(path)
