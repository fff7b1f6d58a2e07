"""Build recipe for libnsmoe.so, the gfx950 HIP library behind nanospeaker_amd.

Every `.hip` file under csrc/ is compiled by hipcc for gfx950 only and linked into one
shared library that sits next to this file (nanospeaker_amd/libnsmoe.so), so it travels
with the source tree.  Run `python -m nanospeaker_amd.build`.
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
LIB = PKG / "libnsmoe.so"
OBJ_DIR = PKG / "_build"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# packed-fp32 instructions are switched off for all device code (they have returned
# wrong results on these boxes); hipcc's host pass warns that it does not know the
# feature, which is harmless.
COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        noise = "is not a recognized feature for this target"
        err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip for gfx950 and link nanospeaker_amd/libnsmoe.so."""
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    OBJ_DIR.mkdir(exist_ok=True)
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 16)

    def compile_one(src: Path) -> Path:
        obj = OBJ_DIR / (src.stem + ".o")
        cmd = [HIPCC, *COMMON, "-I", str(CSRC), "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        _run(cmd)
        return obj

    with cf.ThreadPoolExecutor(jobs) as pool:
        objs = list(pool.map(compile_one, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    _run(cmd)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
