"""Builds the gfx950 kernel library ``trainscale_amd/lib/libtrainscale_amd.so``.

The library is a plain C-ABI shared object (see ``include/trainscale_amd.h``):
every ``csrc/*.hip`` file is compiled by hipcc for gfx950 only and linked with
``hipcc -shared``. No torch headers are involved; the Python side binds the
entry points with ctypes.

Usage: ``python -m trainscale_amd.build`` (or ``build()`` from Python).
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC_DIR = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "lib"
LIB_PATH = LIB_DIR / "libtrainscale_amd.so"
OBJ_DIR = PKG_DIR.parent / "_build" / "trainscale_amd"
INCLUDE_DIR = PKG_DIR.parent / "include"

OFFLOAD_ARCH = "gfx950"

# Packed-FP32 instructions are disabled for all device code: hipcc would
# otherwise form v_pk_{add,mul,fma}_f32 from ordinary float code.
HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={OFFLOAD_ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE_DIR}",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = True, jobs: int | None = None) -> Path:
    """Compiles every kernel source and links the shared library. Always rebuilds."""
    sources = sorted(CSRC_DIR.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[trainscale_amd] built {LIB_PATH} from {len(sources)} sources", flush=True)
    return LIB_PATH


if __name__ == "__main__":
    build()
    sys.exit(0)
