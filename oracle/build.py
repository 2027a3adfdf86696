"""TEST INFRASTRUCTURE ONLY: compile the C oracle (msda_oracle.c) with gcc.

Output: oracle/_build/libmsda_oracle.so. No reference source is compiled here:
deformops' own MSDA code is Python (eager and grid_sample references) and CUDA, so
there is no oracle/_ref build; see msda_oracle.c for what the restatement follows.

    python -m oracle.build
"""

from __future__ import annotations

import os
import subprocess
import tempfile
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
SOURCE = ORACLE_DIR / "msda_oracle.c"
LIBRARY = ORACLE_DIR / "_build" / "libmsda_oracle.so"

# -ffp-contract=off: the pixel map must round exactly as two separate operations.
GCC_FLAGS = ["-O2", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-std=c11"]


def build() -> Path:
    LIBRARY.parent.mkdir(parents=True, exist_ok=True)
    fd, tmp = tempfile.mkstemp(prefix="libmsda_oracle.", suffix=".tmp", dir=LIBRARY.parent)
    os.close(fd)
    try:
        subprocess.run(["gcc", *GCC_FLAGS, str(SOURCE), "-o", tmp, "-lm"], check=True)  # noqa: S603, S607
        os.replace(tmp, LIBRARY)
    finally:
        if os.path.exists(tmp):
            os.unlink(tmp)
    return LIBRARY


if __name__ == "__main__":
    print(build())
