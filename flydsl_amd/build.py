"""Build recipe for libpa_fp8.so (hand-written gfx950 HIP kernels + C ABI).

``python flydsl_amd/build.py`` compiles the library in-tree next to this file (run it
by path: importing the package first would try to load the library).
hipcc cross-compiles for gfx950 without a GPU, so this runs anywhere the ROCm
toolchain is installed.  Every source becomes an object in ``flydsl_amd/_build``
(the per-head-dim decode kernels once per head dim), compiled in parallel, and the
objects are linked into the library.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
LIB_PATH = HERE / "libpa_fp8.so"
OBJ_DIR = HERE / "_build"
HEAD_DIMS = (64, 128, 192, 256)  # decode kernels (pa_decode_hd.hip) are built once per head dim
# (object name, source, extra defines)
UNITS = [("pa_decode", CSRC / "pa_decode.hip", ())] + [
    (f"pa_decode_hd{d}", CSRC / "pa_decode_hd.hip", (f"-DPA_HEAD_DIM={d}",)) for d in HEAD_DIMS
] + [("pa_metadata", CSRC / "pa_metadata.hip", ()), ("rope_cache", CSRC / "rope_cache.hip", ())]
SOURCES = sorted({src for _, src, _ in UNITS})
HEADERS = [CSRC / "pa_common.h", CSRC / "pa_decode_params.h", CSRC / "pa_decode_kernels.h", REPO / "include" / "pa_fp8.h"]
OFFLOAD_ARCH = "gfx950"


def hipcc() -> str:
    return os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def compile_command(src: Path, obj: Path, defines=(), extra=()) -> list:
    return [
        hipcc(),
        f"--offload-arch={OFFLOAD_ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-c",
        "-I",
        str(REPO / "include"),
        # packed fp32 VALU forms are kept out of the device code
        "-Xclang",
        "-target-feature",
        "-Xclang",
        "-packed-fp32-ops",
        *defines,
        *extra,
        str(src),
        "-o",
        str(obj),
    ]


def link_command(objs, out: Path) -> list:
    return [hipcc(), f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *[str(o) for o in objs], "-o", str(out)]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")


def build(verbose: bool = False, extra=()) -> Path:
    """Compile every HIP source into ``flydsl_amd/libpa_fp8.so`` (always rebuilds)."""
    OBJ_DIR.mkdir(exist_ok=True)
    jobs = []
    for name, src, defines in UNITS:
        obj = OBJ_DIR / f"{name}.o"
        jobs.append((compile_command(src, obj, defines, extra), obj))
    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        for f in [pool.submit(_run, cmd, verbose) for cmd, _ in jobs]:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run(link_command([obj for _, obj in jobs], tmp), verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose=True, extra=tuple(sys.argv[1:]))
    print(path)
