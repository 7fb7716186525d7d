"""Builds libcign_amd.so (gfx950 HIP kernels + C-ABI) in-tree with hipcc.

Run as ``python -m cign_amd._build`` or through ``__graft_entry__.build()``.
Object files go to ``cign_amd/_build/`` and the library to
``cign_amd/libcign_amd.so``; both are git-ignored build products.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
SRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libcign_amd.so"

ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 VALU forms are kept out of generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def sources() -> list[Path]:
    return sorted(list(SRC.glob("*.hip")) + list(SRC.glob("*.cpp")))


def _deps(src: Path) -> set[Path]:
    """src and the local headers it includes, transitively."""
    seen, todo = set(), [src]
    while todo:
        f = todo.pop()
        if f in seen or not f.exists():
            continue
        seen.add(f)
        for line in f.read_text().splitlines():
            line = line.strip()
            if line.startswith("#include \""):
                todo.append(SRC / line.split('"')[1])
    return seen


def _compile(hipcc: str, src: Path, force: bool) -> Path:
    obj = OBJ / (src.stem + ".o")
    if not force and obj.exists():
        newest = max([*(d.stat().st_mtime for d in _deps(src)), Path(__file__).stat().st_mtime])
        if obj.stat().st_mtime >= newest:
            return obj
    cmd = [hipcc, *HIP_FLAGS, "-x", "hip", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr[-6000:]}")
    return obj


def build(verbose: bool = False, jobs: int | None = None, force: bool = True) -> Path:
    """Compiles every HIP source for gfx950 and links libcign_amd.so.

    ``force=False`` reuses object files that are newer than their source,
    every header and this script (incremental developer builds)."""
    hipcc = _hipcc()
    OBJ.mkdir(parents=True, exist_ok=True)
    # Slowest translation units first so the parallel build finishes early.
    srcs = sorted(sources(), key=lambda p: ("hp32" not in p.name, p.name))
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)), 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(hipcc, s, force), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    # The library links the HIP runtime only; inside a torch process its
    # soname resolves to the copy torch has already loaded.
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-6000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources", flush=True)
    return LIB


if __name__ == "__main__":
    build(verbose=True, force="--force" in sys.argv)
    sys.exit(0)
