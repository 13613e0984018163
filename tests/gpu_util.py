"""Helpers shared by the GPU tests: layouts, oracle payloads and bitwise comparisons."""

from __future__ import annotations

import ctypes
import random

import numpy as np
import pytest
import torch

from oracle import ccopy, layout

requires_gpu = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="requires a HIP device"),
]

DTYPES = [torch.uint8, torch.bfloat16, torch.float16, torch.float32, torch.int64, torch.float64, torch.bool]

NP_OF = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}


def random_bytes_tensor(nbytes: int, device, seed: int) -> torch.Tensor:
    g = torch.Generator(device="cpu").manual_seed(seed)
    data = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, generator=g)
    return data.to(device)


def view_of(storage_u8: torch.Tensor, dtype: torch.dtype, offset_elems: int, shape, stride) -> torch.Tensor:
    """A ``dtype`` view over a uint8 buffer (element offset, shape, stride in elements)."""

    eb = torch.empty((), dtype=dtype).element_size()
    usable = storage_u8.numel() // eb * eb
    typed = storage_u8[:usable].view(dtype)
    return typed.as_strided(shape, stride, offset_elems)


def random_layout(rng: random.Random, max_elems: int = 4096):
    """A random offloadable (nested) layout: permuted padded row-major, maybe expanded dims."""

    ndim = rng.randint(0, 5)
    shape = [rng.randint(1, 9) for _ in range(ndim)]
    while ndim and int(np.prod(shape)) > max_elems:
        shape[rng.randrange(ndim)] = max(1, shape[rng.randrange(ndim)] // 2)
    order = list(range(ndim))
    rng.shuffle(order)
    stride = [0] * ndim
    step = rng.choice([1, 1, 1, 2, 3])
    for dim in reversed(order):
        stride[dim] = step
        step *= shape[dim] + rng.choice([0, 0, 0, 1, 5])
    for dim in range(ndim):
        if shape[dim] > 1 and rng.random() < 0.1:
            stride[dim] = 0  # expanded
    span = 1 + sum((s - 1) * st for s, st in zip(shape, stride))
    return tuple(shape), tuple(stride), span


def storage_payload_bytes(view: torch.Tensor) -> np.ndarray:
    """Oracle payload (storage order) of a narrowed view, as raw bytes, computed on the CPU."""

    eb = view.element_size()
    storage = view.untyped_storage()
    host = torch.empty(storage.nbytes(), dtype=torch.uint8)
    host.untyped_storage().copy_(storage)
    flat = host.numpy().view(NP_OF[eb])
    shape = tuple(view.shape)
    stride = tuple(view.stride())
    if shape:
        payload = ccopy.gather(flat, view.storage_offset(), shape, stride, storage_order=True)
    else:
        payload = flat[view.storage_offset() : view.storage_offset() + 1].copy()
    assert np.array_equal(payload, layout.storage_payload(flat, view.storage_offset(), shape, stride) if shape else payload)
    return payload.view(np.uint8)


def bits_cpu(t: torch.Tensor) -> torch.Tensor:
    eb = t.element_size()
    width = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[eb]
    t = t.detach()
    if t.dtype == torch.bool:
        t = t.view(torch.uint8)
    return t.cpu().contiguous().view(width)


def assert_bitwise(actual: torch.Tensor, expected: torch.Tensor) -> None:
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    assert actual.dtype == expected.dtype
    assert torch.equal(bits_cpu(actual), bits_cpu(expected))


def u64_array(values) -> ctypes.Array:
    return (ctypes.c_uint64 * max(len(values), 1))(*values)
