"""Build libtriune_hip.so (gfx950) in-tree from triune_amd/csrc/*.hip.

Each source compiles to an object in parallel; the objects link into one shared library next
to this file, which triune_amd._lib loads with ctypes.  Usage: python -m triune_amd.build
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libtriune_hip.so"
ARCH = os.environ.get("TRIUNE_HIP_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # keep the compiler from emitting packed fp32 VALU ops
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    for line in res.stderr.splitlines():
        if "packed-fp32-ops" in line:  # host pass does not know the feature; harmless
            continue
        if line.strip():
            print(line, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every csrc/*.hip and link libtriune_hip.so.  Always recompiles."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = min(len(sources), max(1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} ({LIB.stat().st_size} bytes) from {len(sources)} sources")
    return LIB


if __name__ == "__main__":
    build()
