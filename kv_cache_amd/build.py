"""Builds libqkv.so (all HIP sources under csrc/) for gfx950 with hipcc.

The library is built in-tree next to this file so that it travels with the
repository snapshot; objects go to ``kv_cache_amd/_build/`` (git-ignored).
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
OBJ = PKG / "_build"
LIB = PKG / "libqkv.so"
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-mcode-object-version=5",
    # Every fp32 multiply and add is rounded on its own unless the source
    # asks for a fused multiply-add; the int4 keys and the reference-order
    # fp32 loops rely on this to match the CPU oracle bit for bit.
    "-ffp-contract=off",
    # Packed fp32 ops stay disabled (they have given silently wrong results
    # on these boxes); hipcc's host pass warns that it ignores the feature.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; libqkv needs ROCm's hipcc to build")
    return path


def _compile(src: Path, extra: list[str]) -> Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")
    return obj


def build(extra_flags: list[str] | None = None, out: Path | None = None, jobs: int = 8) -> Path:
    """Compile every csrc/*.hip and link libqkv.so; returns the library path."""
    extra = list(extra_flags or [])
    OBJ.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(sources)))) as ex:
        objs = list(ex.map(lambda s: _compile(s, extra), sources))
    target = Path(out) if out else LIB
    tmp = target.with_name(target.name + f".tmp{os.getpid()}")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, target)
    return target


if __name__ == "__main__":
    print(build(sys.argv[1:]))
