"""Build the gfx950 C-ABI library ``libmlora.so`` in-tree with hipcc.

Usage: ``python dmd-system_amd/build.py`` (or ``build()`` from Python).
Each ``csrc/*.hip`` is compiled for gfx950 only, then linked into one shared
library next to this file. hipcc cross-compiles, so no GPU is needed.
"""
from __future__ import annotations

import concurrent.futures
import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_PATH = PKG_DIR / "libmlora.so"
INCLUDE = PKG_DIR.parent / "include"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # Packed fp32 VALU forms stay disabled for every device pass.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def source_files() -> list[Path]:
    """Every file the library is compiled from: the HIP sources, their headers and the C ABI."""
    return sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.h"), *INCLUDE.glob("*.h")])


def source_hash() -> str:
    """SHA-256 over the sources (name and bytes of each, in name order); the library
    returns the value it was built with from mlora_source_hash()."""
    h = hashlib.sha256()
    root = PKG_DIR.parent
    for f in source_files():
        h.update(str(f.relative_to(root)).encode())
        h.update(b"\0")
        h.update(f.read_bytes())
        h.update(b"\0")
    return h.hexdigest()


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libmlora.so")
    return exe


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link ``libmlora.so``; returns its path."""
    hipcc = _hipcc()
    obj_dir = PKG_DIR / "_build"
    obj_dir.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")

    digest = source_hash()

    def compile_one(src: Path) -> Path:
        obj = obj_dir / (src.stem + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", f'-DMLORA_SOURCE_HASH="{digest}"', "-c", str(src), "-o", str(obj)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        out = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines()
                        if "packed-fp32-ops" not in line)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{out}")
        if verbose and out.strip():
            print(out)
        return obj

    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objs = list(pool.map(compile_one, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
