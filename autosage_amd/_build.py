"""Builds the gfx950 HIP library ``autosage_amd/lib/libautosage_hip.so``.

Every ``csrc/*.hip`` and ``csrc/*.cpp`` file is compiled with ``hipcc`` for
gfx950 only and linked into one shared library exporting the C ABI declared in
``include/autosage_hip.h``.  Run ``python -m autosage_amd._build``.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
LIBDIR = PACKAGE / "lib"
BUILDDIR = PACKAGE / "_build"
LIBRARY = LIBDIR / "libautosage_hip.so"
ARCH = "gfx950"

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-mcode-object-version=5",
    # No packed-fp32 (v_pk_*_f32) instructions anywhere.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(rocm) / "bin" / "hipcc"
    if candidate.exists():
        return str(candidate)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    return found


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(source: Path, builddir: Path, defines: tuple[str, ...]) -> Path:
    obj = builddir / (source.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *(f"-D{d}" for d in defines), "-c", str(source), "-o", str(obj)]
    if source.suffix == ".cpp":
        cmd[1:1] = ["-x", "hip"]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"compiling {source.name} failed:\n{result.stdout}\n{result.stderr}")
    return obj


def build(verbose: bool = False, output: Path = LIBRARY, defines: tuple[str, ...] = ()) -> Path:
    """Compiles every source for gfx950 and links ``output``; ``defines``
    are extra preprocessor definitions (tuning constants)."""
    output = Path(output)
    builddir = BUILDDIR if output == LIBRARY else output.parent / ("_build_" + output.stem)
    builddir.mkdir(parents=True, exist_ok=True)
    output.parent.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(lambda src: _compile(src, builddir, tuple(defines)), srcs))
    tmp = output.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", f"--offload-arch={ARCH}", "-fPIC", *map(str, objects), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"linking {output.name} failed:\n{result.stdout}\n{result.stderr}")
    os.replace(tmp, output)
    if verbose:
        print(f"built {output}")
    return output


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
