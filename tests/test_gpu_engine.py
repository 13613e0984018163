"""The engine (staging ring, pinned pool, copy streams, restore ring) through the C ABI.

Small slots force every mechanism: segments closing when a slot fills, tensors split across
slots, the compute stream waiting for a slot's D2H, restore-slot eviction, prefetch hits,
on-demand fetches, deferred host frees. Every restored tensor is compared bitwise with the
original, which is kept alive on the device for the comparison.
"""

from __future__ import annotations

import random

import pytest
import torch

from moss_offload.engine import EngineConfig, OffloadEngine

from gpu_util import DTYPES, assert_bitwise, random_bytes_tensor, random_layout, requires_gpu, view_of

pytestmark = requires_gpu

MiB = 1 << 20


def _engine(**kw) -> OffloadEngine:
    cfg = EngineConfig(stage_slot_bytes=2 * MiB, stage_slots=3, restore_slots=2, host_chunk_bytes=8 * MiB, **kw)
    return OffloadEngine(torch.device("cuda", 0), cfg)


def _tensors(rng: random.Random, count: int, device, big: bool):
    out = []
    for k in range(count):
        dtype = rng.choice(DTYPES)
        if big and rng.random() < 0.3:
            t = torch.randn(rng.randint(300_000, 1_400_000), device=device).to(dtype)  # up to 5.6 MB
        else:
            eb = torch.empty((), dtype=dtype).element_size()
            shape, stride, span = random_layout(rng, max_elems=60_000)
            backing = random_bytes_tensor((span + 8) * eb + 64, device, rng.randrange(1 << 30))
            if dtype == torch.bool:
                backing = backing & 1
            t = view_of(backing, dtype, rng.choice([0, 1, 2]), shape, stride)
            t = t.as_strided([1 if st == 0 else s for s, st in zip(t.shape, t.stride())], t.stride())
        out.append(t)
    return out


def _restore_and_check(engine, handles, device, order):
    stream = torch.cuda.current_stream(device).cuda_stream
    for i in order:
        original, gid, idx = handles[i]
        restored = engine.restore(gid, idx, stream)
        assert restored.stride() == original.stride()
        assert_bitwise(restored, original)


@pytest.mark.parametrize("staged", [False, True])
@pytest.mark.parametrize("kernel_copy", [False, True])
@pytest.mark.parametrize("seed", [0, 1])
def test_groups_round_trip_lifo(seed, kernel_copy, staged) -> None:
    device = torch.device("cuda", 0)
    engine = _engine(kernel_copy=kernel_copy, timing=True, staged_restore=staged)
    assert engine.link_name() == ("kernel" if kernel_copy else "sdma")
    rng = random.Random(seed)
    stream = torch.cuda.current_stream(device).cuda_stream
    handles = []
    groups = []
    for g in range(6):
        members = []
        for t in _tensors(rng, rng.randint(1, 12), device, big=True):
            gid, idx = engine.pack(t, stream)
            handles.append((t, gid, idx))
            members.append(len(handles) - 1)
        engine.commit(stream)
        groups.append(members)
    # backward order: last group first, entries in reverse
    order = [i for members in reversed(groups) for i in reversed(members)]
    _restore_and_check(engine, handles, device, order)
    torch.cuda.synchronize(device)
    stats = engine.stats()
    assert stats["bytes_d2h"] >= stats["bytes_packed"] > 0
    assert stats["bytes_unpacked"] == stats["bytes_packed"]
    assert stats["stage_slot_waits"] > 0  # the ring wrapped
    assert stats["prefetch_hits"] > 0
    assert stats["copy_failures"] == 0
    # the newest segments are still in the staging ring at backward start
    assert (stats["staged_hits"] > 0) == staged
    for _, gid, idx in handles:
        engine.drop(gid, idx)
    engine.synchronize()
    stats = engine.stats()
    assert stats["groups_live"] == 0 and stats["host_bytes_in_use"] == 0
    assert stats["d2h_ms"] > 0 and stats["timed_d2h_bytes"] == stats["bytes_d2h"]
    engine.close()


def test_restore_twice_and_release_without_restore() -> None:
    """retain_graph (restore twice), partial restore, and a group dropped unused."""

    device = torch.device("cuda", 0)
    engine = _engine()
    stream = torch.cuda.current_stream(device).cuda_stream
    rng = random.Random(7)
    first = [(t, *engine.pack(t, stream)) for t in _tensors(rng, 5, device, big=True)]
    engine.commit(stream)
    second = [(t, *engine.pack(t, stream)) for t in _tensors(rng, 5, device, big=True)]
    engine.commit(stream)
    unused = [(t, *engine.pack(t, stream)) for t in _tensors(rng, 3, device, big=False)]
    engine.commit(stream)
    for _ in range(2):  # two backward passes over the retained graph
        _restore_and_check(engine, second, device, range(len(second) - 1, -1, -1))
        _restore_and_check(engine, first, device, range(len(first) - 1, -1, -1))
    # only a subset of the next group
    _restore_and_check(engine, first, device, [2])
    for _, gid, idx in unused + second + first:
        engine.drop(gid, idx)
    engine.synchronize()
    assert engine.stats()["host_bytes_in_use"] == 0
    engine.close()


def test_open_group_restored_before_commit() -> None:
    """Unpack of a group that was never committed (backward inside the forward)."""

    device = torch.device("cuda", 0)
    engine = _engine()
    stream = torch.cuda.current_stream(device).cuda_stream
    t = torch.randn(1000, 37, device=device)
    gid, idx = engine.pack(t, stream)
    assert_bitwise(engine.restore(gid, idx, stream), t)
    engine.drop(gid, idx)
    engine.close()


def test_host_limit_raises_clear_error() -> None:
    device = torch.device("cuda", 0)
    cfg = EngineConfig(stage_slot_bytes=2 * MiB, stage_slots=2, restore_slots=2, host_chunk_bytes=2 * MiB,
                       host_limit_bytes=4 * MiB)
    engine = OffloadEngine(device, cfg)
    stream = torch.cuda.current_stream(device).cuda_stream
    t = torch.randn(3 * MiB // 4, device=device)  # 3 MiB per save
    handles = []
    with pytest.raises(RuntimeError, match="pinned host pool limit"):
        for _ in range(4):
            handles.append(engine.pack(t, stream))
            engine.commit(stream)
    torch.cuda.synchronize(device)
    engine.close()
