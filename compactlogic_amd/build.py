"""Build libcompactlogic_hip.so (gfx950) in-tree with hipcc.

Usage: ``python -m compactlogic_amd.build`` (or ``build()`` from Python).  Every source in
``csrc/*.hip`` is compiled to an object in ``_build/`` in parallel and linked into
``compactlogic_amd/libcompactlogic_hip.so``.  The package loads that file only; nothing is
compiled at import time.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libcompactlogic_hip.so"
ARCH = os.environ.get("CL_OFFLOAD_ARCH", "gfx950")

# -Xclang -target-feature -Xclang -packed-fp32-ops keeps the compiler from emitting packed
# fp32 arithmetic (v_pk_*_f32), which is avoided on these boxes.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the HIP extension cannot be built")


def _compile(src: Path, hipcc: str) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every csrc/*.hip for gfx950 and link the shared library. Returns its path."""
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), max(1, (os.cpu_count() or 2) // 2), 8)
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, hipcc), sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
