"""Build the C-ABI library ``libgen_worker_amd.so`` for gfx950 with hipcc.

The library is built in-tree (next to this file) so that it travels with the
source tree; nothing is installed. ``python -m gen_worker_amd.build`` or
``__graft_entry__.build()`` runs it.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR.parent / "csrc"
INCLUDE = PKG_DIR.parent.parent / "include"
BUILD_DIR = PKG_DIR.parent / "_build"
LIB_NAME = "libgen_worker_amd.so"
LIB_PATH = PKG_DIR / LIB_NAME
DEBUG_LIB_NAME = "libgen_worker_amd_debug.so"
DEBUG_LIB_PATH = PKG_DIR / DEBUG_LIB_NAME
ARCH = "gfx950"

SOURCES = ("gwa_runtime.hip", "act_quant.hip", "w4a4_gemm.hip", "w4a4_gemm_fp6.hip", "w4a4_gemm_fp6_pipe.hip",
           "w4a4_linear.hip", "w8a8_gemm.hip", "awq_w4a16.hip", "nvfp4.hip", "dit_block.hip",
           "w4a4_gemv.hip", "dit_attention.hip")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # hipcc -O3 otherwise forms v_pk_{add,mul,fma}_f32 from scalar fp32 code;
    # this build never emits packed-fp32 arithmetic.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(src: Path, obj: Path, extra: list[str]) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, f"-I{INCLUDE}", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr[-6000:]}")


def _build_one(debug: bool, ex: cf.Executor) -> Path:
    """Compile every source (GWA_DEBUG: the bounds-checked debug build) and link; returns the library path."""
    out_dir = BUILD_DIR / ("debug" if debug else "release")
    out_dir.mkdir(parents=True, exist_ok=True)
    lib_path = DEBUG_LIB_PATH if debug else LIB_PATH
    extra = [f'-DGWA_BUILD_DESC="archs={ARCH}{" debug" if debug else ""}"'] + (["-DGWA_DEBUG=1"] if debug else [])
    objs = [out_dir / (Path(s).stem + ".o") for s in SOURCES]
    for f in [ex.submit(_compile, CSRC / s, o, extra) for s, o in zip(SOURCES, objs)]:
        f.result()
    tmp = lib_path.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, lib_path)
    return lib_path


def build(verbose: bool = False, jobs: int | None = None, debug: bool = True) -> Path:
    """Compile every HIP source for gfx950 and link the shared library; returns its path. With ``debug`` the
    same sources are also built with GWA_DEBUG (device-side bounds checks that record violations, read with
    ``gwa_debug_violations``) into ``libgen_worker_amd_debug.so``."""
    jobs = jobs or max(1, (os.cpu_count() or 2) - 1)
    # the two builds wait on compile jobs of a pool of their own, so neither can starve the other
    with cf.ThreadPoolExecutor(max_workers=jobs) as cex, cf.ThreadPoolExecutor(max_workers=2) as bex:
        rel = bex.submit(_build_one, False, cex)
        dbg = bex.submit(_build_one, True, cex) if debug else None
        path = rel.result()
        if dbg is not None:
            dpath = dbg.result()
            if verbose:
                print(f"built {dpath}", file=sys.stderr)
    if verbose:
        print(f"built {path}", file=sys.stderr)
    return path


if __name__ == "__main__":
    build(verbose=True)
