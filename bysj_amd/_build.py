"""Build recipe of libdpa4k.so: hipcc for gfx950, one object per source.

The library is built in-tree (``bysj_amd/libdpa4k.so``) so that it travels
with the source tree; objects go to ``bysj_amd/_build/``.  No torch headers
are involved: the library exports a plain C ABI (``include/dpa4k.h``).
"""
from __future__ import annotations

import concurrent.futures
import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
SOURCES = PACKAGE / "csrc"
OBJECTS = PACKAGE / "_build"
LIBRARY = PACKAGE / "libdpa4k.so"
ARCH = "gfx950"

# -ffp-contract=off keeps every product rounded before its add, which the
# sequential segment kernels rely on to reproduce the CPU chain bit for bit.
# The packed-FP32 feature is disabled: the compiler would otherwise pair
# independent fp32 adds/muls into v_pk_* instructions.
HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-ffp-contract=off",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found: a ROCm toolchain is required to build libdpa4k")
    return found


def _sources() -> list[Path]:
    return sorted(SOURCES.glob("*.hip"))


def _digest(path: Path) -> str:
    hasher = hashlib.sha256()
    for dependency in [path, *sorted(SOURCES.glob("*.h")), ROOT / "include" / "dpa4k.h"]:
        hasher.update(dependency.read_bytes())
    hasher.update(" ".join(HIP_FLAGS).encode())
    return hasher.hexdigest()[:16]


def _compile(source: Path, incremental: bool) -> Path:
    obj = OBJECTS / f"{source.stem}.o"
    stamp = OBJECTS / f"{source.stem}.stamp"
    digest = _digest(source)
    if incremental and obj.exists() and stamp.exists() and stamp.read_text() == digest:
        return obj
    command = [hipcc(), *HIP_FLAGS, "-c", str(source), "-o", str(obj)]
    result = subprocess.run(command, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    messages = "\n".join(
        line for line in (result.stdout + result.stderr).splitlines() if noise not in line
    ).strip()
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source.name}:\n{messages}")
    if messages:
        print(f"[build] {source.name}:\n{messages}", file=sys.stderr)
    stamp.write_text(digest)
    return obj


def build(*, incremental: bool = False, jobs: int | None = None, verbose: bool = True) -> Path:
    """Compile every HIP source for gfx950 and link ``libdpa4k.so``."""
    OBJECTS.mkdir(exist_ok=True)
    sources = _sources()
    workers = jobs or min(len(sources), max(1, (os.cpu_count() or 2)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(lambda source: _compile(source, incremental), sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    command = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
               *map(str, objects)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link of libdpa4k.so failed:\n{result.stdout}{result.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"[build] {LIBRARY.relative_to(ROOT)} from {len(objects)} sources", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build(incremental="--incremental" in sys.argv)
