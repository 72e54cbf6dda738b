"""Builds libfe_paged.so (the C-ABI HIP library) in-tree for gfx950.

Usage: python -m flexengine_amd.build   (or flexengine_amd.build.build())

Each csrc/*.hip file is compiled to an object with hipcc, in parallel, then
linked into flexengine_amd/libfe_paged.so.  The library is always rebuilt:
this is the "does it build" check as well as the build.

`python -m flexengine_amd.build --timeline` builds the diagnostic variant
libfe_paged_timeline.so instead (FE_TIMELINE: per-workgroup phase stamps of the
decode kernel, read by flexengine_amd/timeline_c2.py); the product library is
not touched.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC_DIR = PKG_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
LIB_NAME = "libfe_paged.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = os.environ.get("FE_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: keep the compiler from emitting v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libfe_paged.so")
    return exe


TIMELINE_LIB_PATH = PKG_DIR / "libfe_paged_timeline.so"


def _compile(src: Path, obj: Path, verbose: bool, defines: tuple = ()) -> None:
    cmd = [hipcc(), *HIP_FLAGS, *defines, "-I", str(INCLUDE_DIR), "-I", str(CSRC_DIR), "-c",
           str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msg = "\n".join(line for line in (res.stderr or "").splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{msg}")
    if msg.strip() and verbose:
        print(msg, file=sys.stderr)


def build(verbose: bool = False, timeline: bool = False) -> Path:
    sources = sorted(CSRC_DIR.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    target = TIMELINE_LIB_PATH if timeline else LIB_PATH
    defines = ("-DFE_TIMELINE",) if timeline else ()
    with tempfile.TemporaryDirectory(prefix="fe_build_") as tmp:
        objs = [Path(tmp) / (s.stem + ".o") for s in sources]
        workers = min(len(sources), max(1, (os.cpu_count() or 2) // 2), 8)
        with ThreadPoolExecutor(max_workers=workers) as pool:
            list(pool.map(lambda so: _compile(so[0], so[1], verbose, defines), zip(sources, objs)))
        tmp_lib = PKG_DIR / (target.name + ".tmp")
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp_lib)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link of {target.name} failed:\n{res.stderr}")
        os.replace(tmp_lib, target)
    return target


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv, timeline="--timeline" in sys.argv)
    print(path)
