"""Brute-force layout oracle (numpy; TEST INFRASTRUCTURE ONLY, see oracle/__init__).

These functions enumerate every logical element's storage offset, which pins the overlap rule
of ``_offload_view`` (reference training/activation_offload.py:49-60) and the two payload
orders without reusing the reference's own sorted-stride argument:

- logical order: the order ``Tensor.copy_`` into a contiguous tensor produces (reference
  :123-124), i.e. row-major over the shape;
- storage order: the engine's payload order, logical elements sorted by storage offset.
"""

from __future__ import annotations

import numpy as np


def element_offsets(shape, stride) -> np.ndarray:
    """Storage offset (in elements) of every logical element, in logical (row-major) order."""

    shape = tuple(int(s) for s in shape)
    if not shape:
        return np.zeros(1, dtype=np.int64)
    if 0 in shape:
        return np.zeros(0, dtype=np.int64)
    grids = np.indices(shape, dtype=np.int64).reshape(len(shape), -1)
    return (grids * np.asarray(stride, dtype=np.int64)[:, None]).sum(0)


def overlaps(shape, stride) -> bool:
    """True when two logical elements share a storage offset (after narrowing stride-0 dims)."""

    shape = [1 if (st == 0 and sz > 1) else sz for sz, st in zip(shape, stride)]
    offs = element_offsets(shape, stride)
    return len(np.unique(offs)) != len(offs)


def odometer_offsets(shape, stride) -> np.ndarray:
    """Offsets visited by an odometer whose dimensions are nested by stride, largest outermost.

    Ties keep their logical order (stable), like every other stride ordering in this project.
    """

    dims = sorted(range(len(shape)), key=lambda d: -stride[d])
    return element_offsets([shape[d] for d in dims], [stride[d] for d in dims])


def offloadable(shape, stride) -> bool:
    """What ``_offload_view`` decides (reference training/activation_offload.py:32-61).

    No negative stride, and after narrowing expanded dimensions the layout must be *nested*:
    walking it with dimensions ordered by stride (largest outermost) must visit strictly
    increasing offsets. That is the reference's sorted-stride extent rule stated as an
    enumeration: it implies no overlap, but it also rejects some interleaved layouts whose
    offsets are distinct (``nested_but_overlap_free`` below finds them), which the reference
    keeps resident.
    """

    if any(s < 0 for s in stride):
        return False
    shape = narrowed_shape(shape, stride)
    offs = odometer_offsets(shape, stride)
    return bool(np.all(np.diff(offs) > 0))


def interleaved_overlap_free(shape, stride) -> bool:
    """Distinct offsets but not nested: the layouts the reference rule conservatively rejects."""

    if any(s < 0 for s in stride):
        return False
    return not overlaps(shape, stride) and not offloadable(shape, stride)


def narrowed_shape(shape, stride):
    return tuple(1 if (st == 0 and sz > 1) else sz for sz, st in zip(shape, stride))


def logical_payload(flat: np.ndarray, offset: int, shape, stride) -> np.ndarray:
    """Dense payload in logical order of the (narrowed) view over a flat storage array."""

    shape = narrowed_shape(shape, stride)
    return flat[offset + element_offsets(shape, stride)]


def storage_payload(flat: np.ndarray, offset: int, shape, stride) -> np.ndarray:
    """Dense payload in storage order (elements sorted by storage offset) of the narrowed view."""

    shape = narrowed_shape(shape, stride)
    offs = element_offsets(shape, stride)
    return flat[offset + np.sort(offs)]


def scatter_storage(payload: np.ndarray, flat_out: np.ndarray, offset: int, shape, stride) -> None:
    """Inverse of :func:`storage_payload`: write the payload back at the view's offsets."""

    shape = narrowed_shape(shape, stride)
    offs = np.sort(element_offsets(shape, stride))
    flat_out[offset + offs] = payload
