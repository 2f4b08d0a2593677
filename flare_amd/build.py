"""Build ``libflare_amd.so`` (the C-ABI library) in-tree with hipcc for gfx950.

Usage: ``python -m flare_amd.build`` (also called by ``__graft_entry__.build``).
Objects go to ``flare_amd/_build/``; the library to ``flare_amd/libflare_amd.so``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "libflare_amd.so"
ARCH = "gfx950"

# -ffp-contract=off keeps every multiply and add separately rounded, so sums
# and optimizer arithmetic follow the order the code states (and the oracle).
# -packed-fp32-ops keeps v_pk_*_f32 out of the generated code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build flare_amd")
    return path


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd = [hipcc(), "-O2", "-std=c++17", "-fPIC", f"-I{ROOT / 'include'}", f"-I{CSRC}",
               "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compiling {src.name} failed:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every source for gfx950 and link the shared library."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    with ThreadPoolExecutor(max_workers=max(1, workers)) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"linking libflare_amd.so failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(sources)} sources", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build()
