"""``mo_pack_to_host``, the entry point that allocates nothing, against the engine's pack path.

The engine's ``mo_pack`` gathers saves into its own staging ring (device memory it allocates)
and DMAs them to its own pinned pool. ``mo_pack_to_host`` does the same gather into a device
array that is part of the library's code object, then DMAs the payload into a pinned buffer the
caller passes. For the same tensors both must give the same bytes: the payload is scattered
back with ``mo_scatter`` and compared bitwise with what the engine restores (``mo_pack`` ->
``mo_commit`` -> ``mo_unpack``), with the sources, and with ``mo_gather``'s device payload.
Two calls in a row, the second smaller, share the scratch; payloads beyond the scratch and
host buffers that are too small or not pinned are refused before anything is enqueued.
"""

from __future__ import annotations

import ctypes
import random

import pytest
import torch

from moss_offload import _native
from moss_offload.engine import EngineConfig, OffloadEngine

from gpu_util import DTYPES, assert_bitwise, random_bytes_tensor, random_layout, requires_gpu, view_of

pytestmark = requires_gpu

MiB = 1 << 20
SCRATCH = 64 * MiB


def _descs(tensors):
    arr = (_native.MoTensor * max(len(tensors), 1))()
    for i, t in enumerate(tensors):
        _native.describe(t, arr[i])
    return arr


def _tensors(rng: random.Random, count: int, device, big_mib: int):
    out = [torch.randn(big_mib * MiB // 2, device=device).to(torch.bfloat16)] if big_mib else []
    for _ in range(count):
        dtype = rng.choice(DTYPES)
        eb = torch.empty((), dtype=dtype).element_size()
        shape, stride, span = random_layout(rng, max_elems=40_000)
        backing = random_bytes_tensor((span + 8) * eb + 64, device, rng.randrange(1 << 30))
        if dtype == torch.bool:
            backing = backing & 1
        t = view_of(backing, dtype, rng.choice([0, 1, 3]), shape, stride)
        out.append(t.as_strided([1 if st == 0 else s for s, st in zip(t.shape, t.stride())], t.stride()))
    rng.shuffle(out)
    return out


def _layout(lib, tensors):
    descs = _descs(tensors)
    offsets = (ctypes.c_uint64 * max(len(tensors), 1))()
    total = ctypes.c_uint64()
    _native.check("mo_payload_layout", lib.mo_payload_layout(descs, len(tensors), offsets, ctypes.byref(total)))
    return descs, list(offsets)[: len(tensors)], total.value


def _engine_restores(tensors):
    device = tensors[0].device
    engine = OffloadEngine(device, EngineConfig(stage_slot_bytes=8 * MiB, stage_slots=2, restore_slots=2,
                                                host_chunk_bytes=32 * MiB, staged_restore=False,
                                                stage_slots_max=0, restore_slots_max=0, restore_small_slots=0))
    stream = torch.cuda.current_stream(device).cuda_stream
    try:
        refs = [engine.pack(t, stream) for t in tensors]
        engine.commit(stream)
        restored = [engine.restore(g, i, stream).as_strided(t.shape, t.stride()) for (g, i), t in zip(refs, tensors)]
        torch.cuda.synchronize(device)
        for g, i in refs:
            engine.drop(g, i)
        engine.synchronize()
    finally:
        engine.close()
    return restored


def _no_alloc_round_trip(lib, tensors):
    device = tensors[0].device
    stream = torch.cuda.current_stream(device).cuda_stream
    descs, offsets, total = _layout(lib, tensors)
    host = torch.empty(total + 4096, dtype=torch.uint8, pin_memory=True)
    got = (ctypes.c_uint64 * max(len(tensors), 1))()
    _native.check("mo_pack_to_host",
                  lib.mo_pack_to_host(descs, len(tensors), host.data_ptr(), host.numel(), got, stream))
    torch.cuda.synchronize(device)
    assert list(got)[: len(tensors)] == offsets
    # the payload back on the device, scattered into fresh tensors with the sources' strides
    payload = host[:total].to(device)
    outs = [torch.empty_strided(t.shape, t.stride(), dtype=t.dtype, device=device) for t in tensors]
    _native.check("mo_scatter", lib.mo_scatter(_descs(outs), len(outs), payload.data_ptr(),
                                               (ctypes.c_uint64 * len(offsets))(*offsets), stream))
    # mo_gather's device payload of the same tensors: the same bytes at every payload range
    gathered = torch.zeros(total, dtype=torch.uint8, device=device)
    _native.check("mo_gather", lib.mo_gather(descs, len(tensors), gathered.data_ptr(),
                                             (ctypes.c_uint64 * len(offsets))(*offsets), stream))
    torch.cuda.synchronize(device)
    gathered = gathered.cpu()
    for t, off in zip(tensors, offsets):
        n = t.numel() * t.element_size()  # no expanded dims here: the payload is every element
        assert torch.equal(host[off : off + n], gathered[off : off + n])
    return outs


@pytest.mark.parametrize("seed", [0, 1])
def test_pack_to_host_matches_the_engine_on_two_calls_in_a_row(seed) -> None:
    device = torch.device("cuda", 0)
    lib = _native.load()
    rng = random.Random(seed)
    first = _tensors(rng, 14, device, big_mib=48)  # near the scratch size
    second = _tensors(rng, 5, device, big_mib=0)  # smaller: the scratch keeps the first call's bytes
    for tensors in (first, second):
        expected = _engine_restores(tensors)
        actual = _no_alloc_round_trip(lib, tensors)
        for a, e, t in zip(actual, expected, tensors):
            assert_bitwise(a, e)
            assert_bitwise(a, t)


def test_pack_to_host_refuses_what_it_cannot_do_without_allocating() -> None:
    device = torch.device("cuda", 0)
    lib = _native.load()
    stream = torch.cuda.current_stream(device).cuda_stream
    big = torch.zeros(SCRATCH + 4096, dtype=torch.uint8, device=device)
    descs, _, total = _layout(lib, [big])
    host = torch.empty(total, dtype=torch.uint8, pin_memory=True)
    rc = lib.mo_pack_to_host(descs, 1, host.data_ptr(), host.numel(), None, stream)
    assert rc == 1001 and b"exceeds its device scratch" in lib.mo_last_error()
    small = torch.arange(1024, dtype=torch.float32, device=device)
    descs, _, total = _layout(lib, [small])
    tiny = torch.empty(total - 16, dtype=torch.uint8, pin_memory=True)
    assert lib.mo_pack_to_host(descs, 1, tiny.data_ptr(), tiny.numel(), None, stream) == 1001
    assert b"host buffer holds" in lib.mo_last_error()
    pageable = torch.empty(total, dtype=torch.uint8)
    assert lib.mo_pack_to_host(descs, 1, pageable.data_ptr(), pageable.numel(), None, stream) == 1001
    assert b"must be pinned" in lib.mo_last_error()
    # and it still works afterwards
    host = torch.empty(total, dtype=torch.uint8, pin_memory=True)
    _native.check("mo_pack_to_host", lib.mo_pack_to_host(descs, 1, host.data_ptr(), host.numel(), None, stream))
    torch.cuda.synchronize(device)
    assert torch.equal(host[: 4096].view(torch.float32), small.cpu())
