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


def _bf16_exact_f32(n: int, device, seed: int) -> torch.Tensor:
    """float32 values that are exactly bfloat16: every finite class plus NaNs with payloads."""

    g = torch.Generator().manual_seed(seed)
    bits = torch.randint(0, 1 << 16, (n,), generator=g, dtype=torch.int32)
    special = torch.tensor([0x0000, 0x8000, 0x7F80, 0xFF80, 0x7FC0, 0x7F81, 0xFFFF, 0x0001, 0x807F, 0x3F80],
                           dtype=torch.int32)  # +-0, +-inf, NaNs (quiet, signalling payloads), subnormals, 1.0
    bits[: min(n, special.numel())] = special[: min(n, special.numel())]
    return (bits << 16).view(torch.float32).to(device)


@pytest.mark.parametrize("numel", [1, 7, 8, 1000, 8192, 8193, 3 * 8192 + 5, 1 << 20])
def test_bf16_high_gather_keeps_the_high_halves_and_scatter_restores_the_bits(numel) -> None:
    """MO_TENSOR_BF16_HIGH: the payload is the high 16 bits of each float32 element (the
    oracle is the CPU's own bit shift), and the scatter restores every bit, NaN payloads,
    infinities, signed zeros and subnormals included. Sizes cover partial chunks, the
    element tail and several tiles."""

    device = torch.device("cuda", 0)
    lib = _native.load()
    t = _bf16_exact_f32(numel, device, seed=numel)
    plain = torch.randn(777, device=device)  # a normal piece in the same launch
    views = [t, plain]
    arr = (_native.MoTensor * 2)()
    _native.describe(t, arr[0], flags=_native.MO_TENSOR_BF16_HIGH)
    _native.describe(plain, arr[1])
    offsets, total = _layout(lib, arr, 2)
    assert offsets[1] - offsets[0] >= numel * 2 and total == offsets[1] + 777 * 4
    payload = torch.full((total,), 0xC3, dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    _native.check("mo_gather", lib.mo_gather(arr, 2, payload.data_ptr(), None, stream))
    host = payload.cpu()
    expected = (t.cpu().view(torch.int32) >> 16).to(torch.int16).view(torch.uint8)
    assert torch.equal(host[offsets[0] : offsets[0] + numel * 2], expected)
    assert torch.equal(host[offsets[1] : offsets[1] + 777 * 4], plain.cpu().view(torch.uint8))
    out = torch.full_like(t, float("nan"))
    out_plain = torch.zeros_like(plain)
    back = (_native.MoTensor * 2)()
    _native.describe(out, back[0], flags=_native.MO_TENSOR_BF16_HIGH)
    _native.describe(out_plain, back[1])
    _native.check("mo_scatter", lib.mo_scatter(back, 2, payload.data_ptr(), None, stream))
    assert_bitwise(out, t)
    assert_bitwise(out_plain, plain)
