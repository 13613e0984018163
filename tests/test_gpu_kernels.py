"""Pack / unpack kernels (mo_gather / mo_scatter through the C ABI) against the oracle.

Every payload byte is compared with the oracle's storage-order payload computed on the CPU
(oracle/strided_copy.c), and every restored tensor's logical elements are compared bitwise
with the original; padding gaps of the destination must be left untouched. Layouts cover the
three kernel paths: contiguous (incl. the transposed SDPA views, which are dense), padded runs
(``chunk`` halves) and the LDS-staged element path (misaligned bases, element-strided
innermost dimension, odd sizes).
"""

from __future__ import annotations

import ctypes
import random

import numpy as np
import pytest
import torch

from moss_offload import _native, _offload_view

from gpu_util import (
    DTYPES,
    assert_bitwise,
    random_bytes_tensor,
    random_layout,
    requires_gpu,
    storage_payload_bytes,
    view_of,
)

pytestmark = requires_gpu


def _descs(views):
    arr = (_native.MoTensor * max(len(views), 1))()
    for i, v in enumerate(views):
        _native.describe(v, arr[i])
    return arr


def _layout(lib, descs, n):
    offsets = (ctypes.c_uint64 * max(n, 1))()
    total = ctypes.c_uint64()
    _native.check("mo_payload_layout", lib.mo_payload_layout(descs, n, offsets, ctypes.byref(total)))
    return list(offsets[:n]), int(total.value)


def _round_trip(views, device):
    """Gather views, check payload bytes against the oracle, scatter back, check bitwise."""

    lib = _native.load()
    n = len(views)
    descs = _descs(views)
    offsets, total = _layout(lib, descs, n)
    payload = torch.full((max(total, 1),), 0xC3, dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    _native.check("mo_gather", lib.mo_gather(descs, n, payload.data_ptr(), None, stream))
    host = payload.cpu().numpy()
    for view, off in zip(views, offsets):
        expected = storage_payload_bytes(view)
        assert np.array_equal(host[off : off + expected.size], expected), (view.shape, view.stride(), view.dtype)
    restored = []
    for view in views:
        dst = torch.empty_strided(view.shape, view.stride(), dtype=view.dtype, device=device)
        storage = torch.empty(0, dtype=torch.uint8, device=device).set_(dst.untyped_storage())
        storage.fill_(0x5A)
        restored.append((dst, storage))
    rdescs = _descs([d for d, _ in restored])
    _native.check("mo_scatter", lib.mo_scatter(rdescs, n, payload.data_ptr(), None, stream))
    torch.cuda.synchronize(device)
    for view, (dst, storage) in zip(views, restored):
        assert_bitwise(dst, view)
        # bytes of the destination storage that are not logical elements stay at the sentinel
        mask = torch.ones(storage.numel(), dtype=torch.bool)
        eb = view.element_size()
        if view.numel():
            from oracle import layout as L

            offs = L.element_offsets(tuple(view.shape), tuple(view.stride()))
            for b in range(eb):
                mask[torch.from_numpy(offs * eb + b)] = False
        assert torch.all(storage.cpu()[mask] == 0x5A)


@pytest.mark.parametrize("seed", range(6))
def test_random_layouts_round_trip(seed) -> None:
    device = torch.device("cuda", 0)
    rng = random.Random(seed)
    views = []
    backings = []
    for k in range(40):  # more than one launch's worth of descriptors
        dtype = rng.choice(DTYPES)
        eb = torch.empty((), dtype=dtype).element_size()
        shape, stride, span = random_layout(rng)
        offset = rng.choice([0, 0, 1, 3, 8])
        backing = random_bytes_tensor((offset + span + 4) * eb + 64, device, seed * 1000 + k)
        if dtype == torch.bool:
            backing = backing & 1
        view = view_of(backing, dtype, offset, shape, stride)
        narrowed = _offload_view(view)
        assert narrowed is not None
        views.append(narrowed[0])
        backings.append(backing)
    _round_trip(views, device)


def test_dit_shaped_views_round_trip() -> None:
    """The layouts a DiT block saves: dense, transposed SDPA views, chunk halves, stats."""

    device = torch.device("cuda", 0)
    g = torch.Generator(device=device).manual_seed(0)
    T, H, hd, F = 640, 8, 64, 1024
    D = H * hd
    tokens = torch.randn(1, T, D, device=device, generator=g, dtype=torch.bfloat16)
    q = tokens.reshape(1, T, H, hd).transpose(1, 2)  # [1, H, T, hd], strides (T*D, hd, D, 1)
    up_gate = torch.randn(T, 2 * F, device=device, generator=g, dtype=torch.bfloat16)
    up, gate = up_gate.chunk(2, -1)
    stats = torch.rand(1, T, 1, device=device, generator=g) + 0.8
    lse = torch.randn(1, H, T, device=device, generator=g) + 8
    odd = torch.randn(3, 7, 5, device=device, generator=g)[:, 1:, ::2]
    misaligned = torch.randn(4099, device=device, generator=g, dtype=torch.bfloat16)[1:]
    _round_trip([tokens, q, up, gate, stats, lse, odd, misaligned], device)


def test_large_contiguous_and_padded() -> None:
    device = torch.device("cuda", 0)
    g = torch.Generator(device=device).manual_seed(1)
    big = torch.randn(4096, 3072, device=device, generator=g, dtype=torch.bfloat16)  # 24 MiB
    rows = torch.randn(2048, 2 * 3000, device=device, generator=g, dtype=torch.bfloat16)[:, 3000:]
    _round_trip([big, rows], device)


def test_empty_and_scalar() -> None:
    device = torch.device("cuda", 0)
    views = [torch.empty(0, 5, device=device), torch.tensor(3.5, device=device), torch.ones(1, 1, device=device)]
    _round_trip(views, device)
