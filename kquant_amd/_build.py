"""Build the kquant_amd HIP library (gfx950) and the CPU oracle library.

``build_native()`` compiles every ``csrc/*.hip`` source into one in-tree
shared library, ``kquant_amd/libkquant_amd.so``, with hipcc.  The library's
C ABI is declared in ``include/kquant_amd.h``.  ``build_oracle()`` compiles the
test-only C oracle (``oracle/*.c``) with gcc into ``oracle/libmx_oracle.so``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
LIB_PATH = PACKAGE_DIR / "libkquant_amd.so"
ORACLE_DIR = REPO_ROOT / "oracle"
ORACLE_LIB = ORACLE_DIR / "libmx_oracle.so"

OFFLOAD_ARCH = "gfx950"


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def hip_sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build_native(verbose: bool = False) -> Path:
    """Compile all HIP sources into ``libkquant_amd.so`` (always rebuilds)."""

    sources = hip_sources()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [
        _hipcc(),
        f"--offload-arch={OFFLOAD_ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        # packed fp32 VALU ops are kept out of every kernel
        "-Xclang",
        "-target-feature",
        "-Xclang",
        "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
        f"-I{REPO_ROOT / 'include'}",
        *[str(s) for s in sources],
        "-o",
        str(tmp),
    ]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            "hipcc failed:\n" + " ".join(cmd) + "\n" + proc.stdout + proc.stderr
        )
    if verbose and proc.stderr.strip():
        print(proc.stderr)
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
    print(build_native(verbose=True))
    print(build_oracle())
