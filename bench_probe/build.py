"""Build of libmsda_probe.so, the row-gather probe bench.py rates the MSDA kernels
against (msda_probe.h). Bench-side tooling: built in-tree beside its source with
the MSDA library's hipcc flags, loaded by bench.py with ctypes.

    python -m bench_probe.build
"""

from __future__ import annotations

from pathlib import Path

from deformops_amd import _build

HERE = Path(__file__).resolve().parent
SOURCE = HERE / "gather_probe.hip"
LIBRARY = HERE / "libmsda_probe.so"


def build(*, verbose: bool = False) -> Path:
    """Compile the probe library (atomically replaced); return its path."""
    return _build.compile_library([SOURCE], LIBRARY, verbose=verbose)


if __name__ == "__main__":
    print(build(verbose=True))
