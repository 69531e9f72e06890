"""Compile the HIP sources in ``csrc/`` into ``libsbda_amd.so`` (gfx950).

Each ``.hip`` file is compiled to an object with ``hipcc`` (in parallel),
then linked into one shared library next to this file.  The library is
rebuilt when forced (every source recompiled) or when a source or header is
newer than it (only the stale objects recompiled).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
INCLUDE = ROOT / "include"
OBJDIR = HERE / "_build"
LIB = HERE / "libsbda_amd.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed-FP32 VALU forms are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the SBDA library needs ROCm's hipcc")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _stale() -> bool:
    if not LIB.exists():
        return True
    stamp = LIB.stat().st_mtime
    deps = list(CSRC.glob("*")) + list(INCLUDE.glob("*.h")) + [Path(__file__)]
    return any(p.stat().st_mtime > stamp for p in deps)


def _object(src: Path) -> Path:
    return OBJDIR / (src.stem + ".o")


def _object_stale(src: Path) -> bool:
    """An object is rebuilt when it is missing or older than its source, a
    header or this script (headers are shared, so any header change counts)."""
    obj = _object(src)
    if not obj.exists():
        return True
    stamp = obj.stat().st_mtime
    deps = [src, Path(__file__), *CSRC.glob("*.h"), *INCLUDE.glob("*.h")]
    return any(p.stat().st_mtime > stamp for p in deps)


def _compile(src: Path, hipcc: str) -> Path:
    obj = _object(src)
    cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build_library(force: bool = False, verbose: bool = False) -> Path:
    if not force and not _stale():
        return LIB
    hipcc = _hipcc()
    OBJDIR.mkdir(exist_ok=True)
    srcs = sources()
    todo = srcs if force else [s for s in srcs if _object_stale(s)]
    jobs = max(1, min(len(todo), int(os.environ.get("MAX_JOBS", "8")) or 1))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda s: _compile(s, hipcc), todo))
    objs = [_object(s) for s in srcs]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} HIP sources for {ARCH}")
    return LIB


if __name__ == "__main__":
    build_library(force="--force" in sys.argv, verbose=True)
