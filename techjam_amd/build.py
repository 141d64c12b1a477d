"""Build the gfx950 attention library ``techjam_amd/lib/libtechjam_attn.so``.

Every ``csrc/*.hip`` file is compiled for gfx950 only and linked into one
shared library exposing the C ABI of ``include/techjam_attn.h``. Run as
``python -m techjam_amd.build``; ``__graft_entry__.build()`` calls ``build()``.
"""

from __future__ import annotations

import hashlib
import json
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIBDIR = PKG / "lib"
LIBNAME = "libtechjam_attn.so"
OBJDIR = PKG / "_build"
# Written next to the library: the commit and sources it was built from, so
# that a run on a machine without the repository's history can still name them.
BUILD_INFO = LIBDIR / "build_info.json"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed-FP32 VALU instructions are switched off for all device code.
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
    "-Wno-unused-command-line-argument",
]


# Per-file additions. The exact-attention kernel never needs IEEE NaN
# semantics in its row maxima (scores are finite or -inf), and without them
# fmaxf chains compile to v_max3 with no canonicalising moves. Its split-score
# instance with two query blocks per wave is scheduled by LLVM's max-ILP
# strategy (faster for it; the default scheduler is faster for the others).
FILE_FLAGS = {
    "attn_exact.hip": ["-fno-honor-nans"],
    "attn_exact_split.hip": ["-fno-honor-nans", "-mllvm", "-amdgpu-sched-strategy=max-ilp"],
}


def sources():
    return sorted(CSRC.glob("*.hip"))


def library_source_digest() -> str:
    """sha256 (16 hex digits) of everything the library is compiled from:
    ``csrc/*`` (kernels and the shared header) and ``include/*.h``."""
    h = hashlib.sha256()
    for f in sorted(CSRC.glob("*")) + sorted(INCLUDE.glob("*.h")):
        h.update(f.name.encode())
        h.update(f.read_bytes())
    return h.hexdigest()[:16]


def _git(*args: str):
    try:
        res = subprocess.run(["git", "-C", str(ROOT), *args], capture_output=True, text=True, timeout=10)
    except (OSError, subprocess.SubprocessError):
        return None
    return res.stdout.strip() if res.returncode == 0 else None


def write_build_info() -> dict:
    commit = _git("rev-parse", "HEAD")
    status = _git("status", "--short", "--", "techjam_amd/csrc", "include") if commit else None
    info = {"commit": commit, "library_sources_dirty": bool(status), "library_source_digest": library_source_digest()}
    BUILD_INFO.write_text(json.dumps(info, indent=1) + "\n")
    return info


def _compile(src: Path) -> Path:
    obj = OBJDIR / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    OBJDIR.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(_compile, srcs))
    out = LIBDIR / LIBNAME
    tmp = LIBDIR / (LIBNAME + ".tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    write_build_info()
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
