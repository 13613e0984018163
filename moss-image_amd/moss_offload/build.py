"""Build recipe for the engine's C-ABI library (``libmoss_offload.so``) for gfx950.

The library is compiled in-tree with ``hipcc`` (no torch extension machinery): two sources,
the HIP kernels and the host engine, linked into one shared object that ``_native`` loads
with ctypes. Run ``python -m moss_offload.build`` from ``moss-image_amd/`` or call
:func:`build`.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE_ROOT = PACKAGE_DIR.parent
CSRC = SOURCE_ROOT / "csrc"
INCLUDE = SOURCE_ROOT.parent / "include"
LIB_DIR = PACKAGE_DIR / "_lib"
LIB_PATH = LIB_DIR / "libmoss_offload.so"

SOURCES = ("mo_kernels.hip", "mo_engine.cpp")
HEADERS = ("mo_internal.h", "mo_layout.h")

ARCH = "gfx950"

# Packed-FP32 instructions are disabled for all device code of this project.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    """Return the hipcc executable (ROCm's, or the one on PATH)."""

    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(rocm) / "bin" / "hipcc"
    if candidate.exists():
        return str(candidate)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: the engine library cannot be built")
    return found


def build(verbose: bool = False) -> Path:
    """Compile the library into ``moss_offload/_lib`` and return its path.

    Always recompiles. The output is written to a temporary name and renamed, so a process
    that already loaded the previous library keeps a valid mapping.
    """

    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB_DIR / f"libmoss_offload.so.tmp{os.getpid()}"
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", "-o", str(tmp)]
    cmd += [str(CSRC / name) for name in SOURCES]
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        tmp.unlink(missing_ok=True)
        raise RuntimeError(f"hipcc failed ({result.returncode}):\n{result.stdout}\n{result.stderr}")
    if verbose and result.stderr.strip():
        print(result.stderr, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
