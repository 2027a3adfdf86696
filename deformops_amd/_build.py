"""Ahead-of-time build of the HIP library for gfx950.

libdeformops_amd.so is the MSDA library (the C ABI of include/deformops_amd.h),
built in-tree (``deformops_amd/lib/``) with hipcc and loaded with ctypes; nothing is
compiled at import or call time.

    python -m deformops_amd._build
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

__all__ = ["ARCH", "HIPCC_FLAGS", "LIBRARY", "SOURCES", "build", "compile_library"]

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
SOURCES = [PACKAGE_DIR / "csrc" / "msda.hip"]
INCLUDE_DIR = REPO_DIR / "include"
LIBRARY = PACKAGE_DIR / "lib" / "libdeformops_amd.so"
ARCH = os.environ.get("DEFORMOPS_AMD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-shared",
    # Packed fp32 VALU ops stay off: hipcc forms them from ordinary float code.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE_DIR}",
]


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    msg = "hipcc not found; set HIPCC or install ROCm"
    raise FileNotFoundError(msg)


def build(*, verbose: bool = False) -> Path:
    """Compile the MSDA library, atomically replacing it; return its path.

    Raises
    ------
    subprocess.CalledProcessError
        If hipcc fails; the compiler output is in the exception.
    """
    return compile_library(SOURCES, LIBRARY, verbose=verbose)


def compile_library(sources: list[Path], target: Path, *, verbose: bool) -> Path:
    target.parent.mkdir(parents=True, exist_ok=True)
    fd, tmp = tempfile.mkstemp(prefix=target.name + ".", suffix=".tmp", dir=target.parent)
    os.close(fd)
    cmd = [_hipcc(), *HIPCC_FLAGS, *map(str, sources), "-o", tmp]
    try:
        result = subprocess.run(cmd, capture_output=True, text=True, check=False)  # noqa: S603
        if verbose or result.returncode != 0:
            noise = "is not a recognized feature for this target"
            lines = [ln for ln in (result.stdout + result.stderr).splitlines() if noise not in ln]
            if lines:
                print("\n".join(lines), file=sys.stderr)
        if result.returncode != 0:
            raise subprocess.CalledProcessError(result.returncode, cmd, result.stdout, result.stderr)
        os.replace(tmp, target)
    finally:
        if os.path.exists(tmp):
            os.unlink(tmp)
    return target


if __name__ == "__main__":
    print(build(verbose=True))
