"""Pins the oracle's C copy routines (oracle/strided_copy.c) on the CPU.

- Logical-order gather equals numpy's strided view copied densely (what ``Tensor.copy_`` into
  a contiguous payload produces, reference activation_offload.py:123-124).
- Storage-order gather equals the element-offset sort of oracle/layout.py (the engine's
  payload order), computed independently.
- Scatter inverts gather in both orders, and leaves gaps of padded layouts untouched.
- A planted wrong permutation is caught.
"""

from __future__ import annotations

import random

import numpy as np
import pytest

from oracle import ccopy, layout


def _cases(seed: int, count: int):
    rng = random.Random(seed)
    for _ in range(count):
        ndim = rng.randint(0, 5)
        shape = tuple(rng.randint(1, 5) for _ in range(ndim))
        # build a non-overlapping layout by permuting a padded row-major layout
        order = list(range(ndim))
        rng.shuffle(order)
        stride = [0] * ndim
        step = 1
        for dim in reversed(order):
            stride[dim] = step
            step *= shape[dim] + rng.choice([0, 0, 1, 3])
        yield shape, tuple(stride), step


@pytest.mark.parametrize("dtype", [np.uint8, np.int16, np.float32, np.int64])
def test_gather_scatter_match_numpy(dtype) -> None:
    for shape, stride, span in _cases(5, 400):
        flat = (np.arange(span + 7) * 7 + 3).astype(dtype)
        offset = 3
        itemsize = flat.itemsize
        view = np.lib.stride_tricks.as_strided(
            flat[offset:], shape=shape, strides=tuple(s * itemsize for s in stride)
        )
        logical = ccopy.gather(flat, offset, shape, stride, storage_order=False)
        assert np.array_equal(logical, view.reshape(-1))
        storage = ccopy.gather(flat, offset, shape, stride, storage_order=True)
        assert np.array_equal(storage, layout.storage_payload(flat, offset, shape, stride))
        for order, payload in ((False, logical), (True, storage)):
            out = np.full_like(flat, 99)
            ccopy.scatter(payload, out, offset, shape, stride, storage_order=order)
            written = np.zeros(flat.shape, dtype=bool)
            written[offset + layout.element_offsets(shape, stride)] = True
            assert np.array_equal(out[written], flat[written])
            assert np.all(out[~written] == 99)


def test_storage_perm_is_stride_descending() -> None:
    assert ccopy.storage_perm((2, 3, 4), (1, 8, 2)) == [1, 2, 0]
    assert ccopy.storage_perm((4, 3), (3, 1)) == [0, 1]


def test_planted_wrong_order_is_caught() -> None:
    caught = 0
    for shape, stride, span in _cases(6, 200):
        if len(shape) < 2:
            continue
        flat = np.arange(span + 1, dtype=np.int32)
        right = layout.storage_payload(flat, 0, shape, stride)
        wrong = ccopy.gather(flat, 0, shape[::-1], stride[::-1], storage_order=False)
        if not np.array_equal(right, wrong):
            caught += 1
    assert caught > 0
