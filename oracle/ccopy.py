"""ctypes access to oracle/_build/liboracle_copy.so (TEST INFRASTRUCTURE ONLY)."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle_copy.so"

_lib = None


def build() -> Path:
    """Compile strided_copy.c with the committed Makefile."""

    subprocess.run(["make", "-s", "-B", "-C", str(HERE)], check=True)
    return LIB


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        i64p = ctypes.POINTER(ctypes.c_int64)
        intp = ctypes.POINTER(ctypes.c_int)
        for name in ("oracle_gather", "oracle_scatter"):
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int64
            fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, i64p, i64p, intp, ctypes.c_void_p]
        lib.oracle_storage_perm.restype = None
        lib.oracle_storage_perm.argtypes = [ctypes.c_int, i64p, i64p, intp]
        _lib = lib
    return _lib


def _arrays(shape, stride):
    n = len(shape)
    size = (ctypes.c_int64 * max(n, 1))(*shape)
    strd = (ctypes.c_int64 * max(n, 1))(*stride)
    return n, size, strd


def storage_perm(shape, stride) -> list[int]:
    lib = load()
    n, size, strd = _arrays(shape, stride)
    perm = (ctypes.c_int * max(n, 1))()
    lib.oracle_storage_perm(n, size, strd, perm)
    return list(perm[:n])


def gather(flat: np.ndarray, offset: int, shape, stride, storage_order: bool) -> np.ndarray:
    """Dense payload of the view ``(offset, shape, stride)`` over the 1-D array ``flat``."""

    lib = load()
    flat = np.ascontiguousarray(flat)
    n, size, strd = _arrays(shape, stride)
    perm = None
    if storage_order:
        perm = (ctypes.c_int * max(n, 1))(*storage_perm(shape, stride))
    count = int(np.prod(shape)) if n else 1
    out = np.empty(count, dtype=flat.dtype)
    base = flat.ctypes.data + offset * flat.itemsize
    lib.oracle_gather(base, flat.itemsize, n, size, strd, perm, out.ctypes.data)
    return out


def scatter(payload: np.ndarray, flat_out: np.ndarray, offset: int, shape, stride, storage_order: bool) -> None:
    """Write ``payload`` back into the view ``(offset, shape, stride)`` of ``flat_out``."""

    lib = load()
    payload = np.ascontiguousarray(payload)
    assert flat_out.flags["C_CONTIGUOUS"]
    n, size, strd = _arrays(shape, stride)
    perm = None
    if storage_order:
        perm = (ctypes.c_int * max(n, 1))(*storage_perm(shape, stride))
    base = flat_out.ctypes.data + offset * flat_out.itemsize
    lib.oracle_scatter(base, flat_out.itemsize, n, size, strd, perm, payload.ctypes.data)
