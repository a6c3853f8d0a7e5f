"""Build the kquant_amd HIP library (gfx950) and the CPU oracle library.

``build_native()`` compiles every ``csrc/*.hip`` source to an object under
``kquant_amd/_build/`` (one hipcc process per source, in parallel) and links
them into one in-tree shared library, ``kquant_amd/libkquant_amd.so``.  The
library's C ABI is declared in ``include/kquant_amd.h``.  With
``force=False`` an object is reused when it is newer than its source and every
local header the source includes.  ``build_oracle()`` compiles the test-only C oracle
(``oracle/*.c``) with gcc into ``oracle/libmx_oracle.so``.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
OBJ_DIR = PACKAGE_DIR / "_build"
LIB_PATH = PACKAGE_DIR / "libkquant_amd.so"
ORACLE_DIR = REPO_ROOT / "oracle"
ORACLE_LIB = ORACLE_DIR / "libmx_oracle.so"

OFFLOAD_ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 VALU ops are kept out of every kernel
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def hip_sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


_INCLUDE = re.compile(r'^\s*#\s*include\s+"([^"]+)"', re.M)


def _deps_mtime(src: Path) -> float:
    """Newest modification time of ``src`` and the local headers it includes (transitively)."""

    seen: set[Path] = set()
    todo = [src]
    newest = 0.0
    while todo:
        f = todo.pop()
        if f in seen or not f.exists():
            continue
        seen.add(f)
        newest = max(newest, f.stat().st_mtime)
        for name in _INCLUDE.findall(f.read_text(errors="replace")):
            for base in (f.parent, REPO_ROOT / "include"):
                cand = (base / name).resolve()
                if cand.exists():
                    todo.append(cand)
                    break
    return newest


def _run(cmd: list[str]) -> subprocess.CompletedProcess:
    return subprocess.run(cmd, capture_output=True, text=True)


def build_native(verbose: bool = False, force: bool = True, jobs: int | None = None) -> Path:
    """Compile the HIP sources (all of them unless ``force`` is False) and link the library."""

    hipcc = _hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    todo = []
    objects = []
    for src in hip_sources():
        obj = OBJ_DIR / (src.stem + ".o")
        objects.append(obj)
        stale = force or not obj.exists() or obj.stat().st_mtime < _deps_mtime(src)
        if stale:
            todo.append((src, obj))
    cmds = [[hipcc, *HIP_FLAGS, f"-I{REPO_ROOT / 'include'}", "-c", str(src), "-o", str(obj) + ".tmp"]
            for src, obj in todo]
    workers = jobs or max(1, min(len(cmds), os.cpu_count() or 1, 16))
    with ThreadPoolExecutor(max_workers=max(1, workers)) as pool:
        results = list(pool.map(_run, cmds))
    for (src, obj), cmd, proc in zip(todo, cmds, results):
        if proc.returncode != 0:
            raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + proc.stdout + proc.stderr)
        if verbose and proc.stderr.strip():
            print(proc.stderr)
        os.replace(str(obj) + ".tmp", obj)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    link = [hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *[str(o) for o in objects], "-o", str(tmp)]
    proc = _run(link)
    if proc.returncode != 0:
        raise RuntimeError("link failed:\n" + " ".join(link) + "\n" + proc.stdout + proc.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def build_oracle() -> Path:
    """Compile the test-only C oracle with gcc (always rebuilds)."""

    sources = sorted(ORACLE_DIR.glob("*.c"))
    tmp = ORACLE_LIB.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-fopenmp",
           *[str(s) for s in sources], "-lm", "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("gcc failed:\n" + " ".join(cmd) + "\n" + proc.stdout + proc.stderr)
    os.replace(tmp, ORACLE_LIB)
    return ORACLE_LIB


if __name__ == "__main__":
    import sys

    print(build_native(verbose=True, force="--incremental" not in sys.argv))
    print(build_oracle())
