"""Build recipe of ``libiris_hip.so``: hipcc for gfx950, one object per source, then a link.

Run as ``python -m iris_mi355x.build`` (from ``iris-3b-metal_amd/``) or through
``__graft_entry__.build()``. Objects go to ``csrc/_build/`` and the library lands beside
this file, where ``iris_mi355x._lib`` loads it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIBRARY = HERE / "libiris_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed FP32 instructions are kept out of every kernel on this target
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found (ROCm is required to build libiris_hip.so)")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every ``csrc/*.hip`` for gfx950 and link ``libiris_hip.so``; returns its path."""
    out_dir = CSRC / "_build"
    out_dir.mkdir(exist_ok=True)
    cc = hipcc()
    srcs = sources()
    headers = list(CSRC.glob("*.hpp")) + list((HERE.parents[1] / "include").glob("*.h"))

    def compile_one(src: Path) -> Path:
        obj = out_dir / (src.stem + ".o")
        cmd = [cc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")
        if verbose:
            print(f"compiled {src.name}", flush=True)
        return obj

    del headers  # every build recompiles all sources: the inputs are small and a stale object is worse
    workers = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(compile_one, srcs))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of libiris_hip.so failed:\n{res.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
