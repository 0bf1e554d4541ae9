"""Builds ``oracle/liboracle.so`` from ``csr_oracle.c`` with gcc.

Test infrastructure only (see ``oracle/__init__.py``).  The AutoSAGE reference
itself is not built here: its native code is CUDA with a CMake/CUDA-toolkit
build (CMakeLists.txt:3-27), so there is no ``oracle/_ref``.
"""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SOURCE = HERE / "csr_oracle.c"
LIBRARY = HERE / "liboracle.so"
FLAGS = ["-O2", "-std=c11", "-fPIC", "-shared", "-mfma", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-Wall"]


def build() -> Path:
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = ["gcc", *FLAGS, str(SOURCE), "-o", str(tmp), "-lm"]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"building the oracle failed:\n{result.stdout}\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build())
