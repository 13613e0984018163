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
    # each commit sends its own segments unless a test asks for commit batching; the rings keep
    # their sizes, every slot allocated up front, unless a test asks for growth or small slots
    kw.setdefault("commit_batch_bytes", 0)
    kw.setdefault("stage_slots_max", 0)
    kw.setdefault("restore_slots_max", 0)
    kw.setdefault("restore_small_slots", 0)
    kw.setdefault("stage_slots", 3)
    kw.setdefault("restore_slots", 2)
    cfg = EngineConfig(stage_slot_bytes=2 * MiB, host_chunk_bytes=8 * MiB, **kw)
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
@pytest.mark.parametrize("link", ["sdma", "hipdma", "kernel"])
@pytest.mark.parametrize("seed", [0, 1])
def test_groups_round_trip_lifo(seed, link, staged) -> None:
    device = torch.device("cuda", 0)
    if link == "kernel":
        engine = _engine(kernel_copy=True, timing=True, staged_restore=staged)
    else:
        engine = _engine(link=link, timing=True, staged_restore=staged)
    assert engine.link_name() == link
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
    engine.synchronize()  # coded segments' link bytes are counted once their copies complete
    stats = engine.stats()
    # every packed byte crossed the link, raw or wire-coded (the default engine codes segments
    # while two staging slots of D2H bytes are queued)
    assert stats["bytes_d2h"] - stats["wire_bytes"] + stats["wire_raw_bytes"] >= stats["bytes_packed"] > 0
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
    if link != "sdma":
        assert stats["host_blocks"] == 0  # every copy -> compute order is a stream wait
    engine.close()


@pytest.mark.parametrize("d2h_engine", [0, 1])
def test_hipdma_link_split_and_single_d2h_round_trip(d2h_engine) -> None:
    # 8 MiB slots so that D2H copies reach the 2 MiB split size; d2h_engine=1 keeps one stream.
    device = torch.device("cuda", 0)
    cfg = EngineConfig(stage_slot_bytes=8 * MiB, stage_slots=3, restore_slots=2, host_chunk_bytes=32 * MiB,
                       link="hipdma", d2h_engine=d2h_engine, timing=True, stage_slots_max=0, restore_slots_max=0,
                       restore_small_slots=0)
    engine = OffloadEngine(device, cfg)
    stream = torch.cuda.current_stream(device).cuda_stream
    rng = random.Random(7 + d2h_engine)
    handles, groups = [], []
    for g in range(5):
        members = []
        for t in _tensors(rng, rng.randint(2, 8), device, big=True):
            gid, idx = engine.pack(t, stream)
            handles.append((t, gid, idx))
            members.append(len(handles) - 1)
        engine.commit(stream)
        groups.append(members)
    order = [i for members in reversed(groups) for i in reversed(members)]
    _restore_and_check(engine, handles, device, order)
    torch.cuda.synchronize(device)
    for _, gid, idx in handles:
        engine.drop(gid, idx)
    engine.synchronize()
    stats = engine.stats()
    assert stats["copy_failures"] == 0 and stats["host_blocks"] == 0
    assert stats["groups_live"] == 0 and stats["host_bytes_in_use"] == 0
    assert stats["timed_d2h_bytes"] == stats["bytes_d2h"] > 0
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
                       host_limit_bytes=4 * MiB, stage_slots_max=0, restore_slots_max=0, restore_small_slots=0)
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


def _scribble_like(t: torch.Tensor) -> None:
    """Allocate and fill a tensor the size of ``t``'s storage: if ``t``'s memory had been
    returned to the caching allocator, this would overwrite it."""

    torch.full((t.untyped_storage().nbytes() // 4 + 1,), -7.0, device=t.device)


@pytest.mark.parametrize("batch", [True, False])
def test_batched_packs_keep_freed_sources_until_launched(batch) -> None:
    """Saves whose only reference is dropped right after mo_pack: their gathers may still be
    pending, so the engine must keep them alive; the restores are bitwise either way, and
    batching launches fewer kernels for the same saves."""

    device = torch.device("cuda", 0)
    engine = _engine(batch_packs=batch)
    stream = torch.cuda.current_stream(device).cuda_stream
    rng = random.Random(11)
    handles, expected = [], []
    pending_seen = 0
    for g in range(4):
        for t in _tensors(rng, 10, device, big=g % 2 == 0):
            expected.append((t.clone(), t.stride()))
            gid, idx = engine.pack(t, stream)
            handles.append((gid, idx))
            pending_seen = max(pending_seen, len(engine._held))
            del t
            _scribble_like(expected[-1][0])
        engine.commit(stream)
        assert not engine._held  # a commit launches every pending gather
    assert (pending_seen > 0) == batch
    for (gid, idx), (original, stride) in reversed(list(zip(handles, expected))):
        restored = engine.restore(gid, idx, stream)
        assert restored.stride() == stride
        assert_bitwise(restored, original)
    stats = engine.stats()
    launches = stats["pack_launches"]
    assert stats["bytes_unpacked"] == stats["bytes_packed"]
    for gid, idx in handles:
        engine.drop(gid, idx)
    engine.synchronize()
    assert engine.stats()["host_bytes_in_use"] == 0
    engine.close()
    if batch:
        assert launches < len(handles)
    else:
        assert launches >= len(handles)


def test_batched_packs_on_two_streams() -> None:
    """A pack on another stream launches the pending gathers of the first stream first."""

    device = torch.device("cuda", 0)
    engine = _engine()
    main = torch.cuda.current_stream(device)
    side = torch.cuda.Stream(device)
    rng = random.Random(12)
    tensors = _tensors(rng, 12, device, big=False)
    side.wait_stream(main)
    handles = []
    for k, t in enumerate(tensors):
        stream = side if k % 3 == 2 else main
        with torch.cuda.stream(stream):
            handles.append(engine.pack(t, stream.cuda_stream))
            t.record_stream(stream)
    main.wait_stream(side)
    engine.commit(main.cuda_stream)
    assert not engine._held
    for (gid, idx), original in reversed(list(zip(handles, tensors))):
        assert_bitwise(engine.restore(gid, idx, main.cuda_stream), original)
    for gid, idx in handles:
        engine.drop(gid, idx)
    engine.synchronize()
    engine.close()


def test_release_of_the_open_group_drops_pending_gathers() -> None:
    device = torch.device("cuda", 0)
    engine = _engine()
    stream = torch.cuda.current_stream(device).cuda_stream
    small = [torch.randn(1000 + k, device=device) for k in range(5)]
    handles = [engine.pack(t, stream) for t in small]
    assert len(engine._held) == 5
    small[0].add_(1.0)  # a dropped graph's source modified afterwards: its gather never runs
    for gid, idx in handles:
        engine.drop(gid, idx)
    assert not engine._held and engine.live_groups() == 0
    assert engine.stats()["pack_launches"] == 0  # nothing was launched for the abandoned group
    # the engine carries on: a new group packs, commits and restores
    t = torch.randn(3000, 7, device=device)
    gid, idx = engine.pack(t, stream)
    engine.commit(stream)
    assert_bitwise(engine.restore(gid, idx, stream), t)
    engine.drop(gid, idx)
    engine.synchronize()
    assert engine.stats()["host_bytes_in_use"] == 0
    engine.close()


@pytest.mark.parametrize("batch", [True, False])
def test_save_modified_in_place_before_its_gather(batch) -> None:
    """Saved-tensor hooks switch off autograd's version check, so a save modified in place
    afterwards still reaches backward. Copying at the save keeps the bytes of the save; a
    batched gather not launched yet would read the new bytes, and raises instead."""

    device = torch.device("cuda", 0)
    engine = _engine(batch_packs=batch)
    stream = torch.cuda.current_stream(device).cuda_stream
    t = torch.randn(4096, device=device)
    saved = t.clone()
    gid, idx = engine.pack(t, stream)
    t.mul_(2.0)
    if batch:
        with pytest.raises(RuntimeError, match="modified in place"):
            engine.commit(stream)
    else:
        engine.commit(stream)
        assert_bitwise(engine.restore(gid, idx, stream), saved)
    # a modification after the commit (the gather is launched) is no longer the engine's concern
    u = torch.randn(4096, device=device)
    gid2, idx2 = engine.pack(u, stream)
    engine.commit(stream)
    expected = u.clone()
    u.mul_(3.0)
    assert_bitwise(engine.restore(gid2, idx2, stream), expected)
    engine.drop(gid, idx)
    engine.drop(gid2, idx2)
    engine.synchronize()
    engine.close()


@pytest.mark.parametrize("pack_nt_load", [False, True])
@pytest.mark.parametrize("unpack_nt_load", [False, True])
@pytest.mark.parametrize("unpack_nt_store", [False, True])
def test_narrowed_float32_pieces_across_slots(pack_nt_load, unpack_nt_load, unpack_nt_store) -> None:
    """bf16-exact float32 tensors packed narrowed (MO_TENSOR_BF16_HIGH), larger than a 2 MiB
    slot so that their pieces split across slots (the tensor side of a later piece starts at
    twice its payload offset), between plain tensors; every restore is bitwise. Run under every
    cache policy of the kernels: each policy is its own code path of the full CONTIG and NARROW
    tiles."""

    device = torch.device("cuda", 0)
    engine = _engine(pack_nt_load=pack_nt_load, unpack_nt_load=unpack_nt_load, unpack_nt_store=unpack_nt_store)
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator(device="cpu").manual_seed(21)
    handles, expected_bytes = [], 0
    for k in range(6):
        if k % 2 == 0:
            n = 700_000 + 4099 * k  # 1.4 MB payload, 2.8 MB float32
            bits = torch.randint(0, 1 << 16, (n,), generator=g, dtype=torch.int32) << 16
            t = bits.view(torch.float32).to(device)
            handles.append((t, *engine.pack(t, stream, narrow=True)))
            expected_bytes += n * 2
        else:
            t = torch.randn(300_001, generator=g).to(device)
            handles.append((t, *engine.pack(t, stream)))
            expected_bytes += t.numel() * 4
    engine.commit(stream)
    for t, gid, idx in reversed(handles):
        assert_bitwise(engine.restore(gid, idx, stream), t)
    engine.synchronize()
    assert engine.stats()["bytes_packed"] == expected_bytes
    for _, gid, idx in handles:
        engine.drop(gid, idx)
    engine.synchronize()
    engine.close()


@pytest.mark.parametrize("nbytes", [16, 4096 + 5, 16 * 1024, 16 * 1024 + 48, 3 * MiB + 7, 54 * MiB])
def test_equal_reports_equal_and_any_single_byte_difference(nbytes) -> None:
    """mo_equal: equal ranges report 1; one flipped byte at the start, in the middle or in the
    last (tail) byte reports 2. Buffers are exactly nbytes long, so the kernel's tail handling
    is exercised at every size, full tiles, partial tiles and a trailing partial 16-byte word."""

    engine = _engine()
    device = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator(device=device).manual_seed(nbytes)
    a = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=device, generator=g)
    try:
        for where in (None, 0, nbytes // 2, nbytes - 1):
            b = a.clone()
            if where is not None:
                b[where] ^= 0x10
            ticket = engine.equal(a, b, stream)
            assert ticket != 0
            assert engine.equal_result(ticket, wait=True) == (1 if where is None else 2), where
        # polling: 0 until known, then the result once
        ticket = engine.equal(a, a.clone(), stream)
        torch.cuda.synchronize()
        assert engine.equal_result(ticket, wait=False) == 1
        with pytest.raises(RuntimeError):
            engine.equal_result(ticket, wait=False)
    finally:
        engine.close()


def test_equal_tickets_run_out_and_come_back() -> None:
    """64 result slots: a 65th check starts nothing (ticket 0); a discarded ticket's slot and a
    reported one's are reused."""

    engine = _engine()
    device = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(device).cuda_stream
    a = torch.arange(4096, dtype=torch.int32, device=device)
    b = a.clone()
    try:
        tickets = [engine.equal(a, b, stream) for _ in range(64)]
        assert all(tickets) and len(set(tickets)) == 64
        assert engine.equal(a, b, stream) == 0
        engine.equal_discard(tickets[0])
        torch.cuda.synchronize()
        again = engine.equal(a, b, stream)
        assert again != 0 and again not in tickets
        for t in tickets[1:] + [again]:
            assert engine.equal_result(t, wait=True) == 1
        with pytest.raises(RuntimeError):
            engine.equal_discard(tickets[0])
        with pytest.raises(RuntimeError):
            engine.equal(a[1:], b[:-1], stream)  # 4-byte offset: not 16-byte aligned
        with pytest.raises(ValueError):
            engine.equal(a[1:], b, stream)  # sizes differ
    finally:
        engine.close()


def test_timed_link_rate_is_bounded_by_the_host_clock() -> None:
    """With timing on, the SDMA link times copies by the DMA engines' own stamps. Their busy time
    can be no longer than the host's view of the same copies (issue to observed completion) and
    must give a rate a PCIe x16 link can carry: between 10 and 70 GB/s for the 2 MiB segment
    copies of this small-slot engine."""

    import time

    engine = _engine(timing=True, wire_coding="off")  # raw copies: the link carries exactly the payload
    device = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(device).cuda_stream
    src = torch.randint(0, 256, (32 * MiB,), dtype=torch.uint8, device=device)
    try:
        engine.synchronize()
        engine.reset_stats()
        t0 = time.perf_counter()
        for _ in range(8):
            engine.pack(src, stream)
            engine.commit(stream)
        engine.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3
        st = engine.stats()
        assert st["timed_d2h_bytes"] == 8 * 32 * MiB
        assert 0 < st["d2h_ms"] <= wall_ms
        rate = st["timed_d2h_bytes"] / st["d2h_ms"] / 1e6
        assert 10 < rate < 70, rate
    finally:
        engine.close()


@pytest.mark.parametrize("mode", ["on", "auto"])
@pytest.mark.parametrize("staged", [False, True])
def test_wire_coded_segments_round_trip(mode, staged) -> None:
    """Segments wire-coded before their D2H and decoded after their H2D (MO_FLAG_WIRE_*):
    random layouts and dtypes plus bfloat16 activations, across slot boundaries, restored
    LIFO bitwise; the coded bytes are what crosses the link."""

    device = torch.device("cuda", 0)
    engine = _engine(wire_coding=mode, timing=True, staged_restore=staged)
    rng = random.Random(7)
    g = torch.Generator(device="cpu").manual_seed(7)
    stream = torch.cuda.current_stream(device).cuda_stream
    handles, groups = [], []
    for k in range(6):
        members = []
        batch = _tensors(rng, rng.randint(1, 6), device, big=True)
        batch.append(torch.randn(rng.randint(200_000, 900_000), generator=g).to(torch.bfloat16).to(device))
        for t in batch:
            gid, idx = engine.pack(t, stream)
            handles.append((t, gid, idx))
            members.append(len(handles) - 1)
        engine.commit(stream)
        groups.append(members)
    order = [i for members in reversed(groups) for i in reversed(members)]
    _restore_and_check(engine, handles, device, order)
    engine.synchronize()
    st = engine.stats()
    assert st["copy_failures"] == 0
    if mode == "on":
        assert st["wire_segments"] > 0
    if st["wire_segments"]:
        # random-bit tiles are stored raw (a little over raw with their headers); the coded size
        # never exceeds the format's worst case
        assert 0 < st["wire_bytes"] <= st["wire_raw_bytes"] * 1.003 + 4096 * st["wire_segments"]
    assert st["bytes_unpacked"] == st["bytes_packed"]
    for _, gid, idx in handles:
        engine.drop(gid, idx)
    engine.synchronize()
    assert engine.stats()["host_bytes_in_use"] == 0
    engine.close()


def test_prefetch_groups_takes_a_farther_group_only_when_all_of_it_fits() -> None:
    """mo_prefetch_groups: the nearest group as far as slots allow, a later one only when every
    segment it needs gets a free slot; restores stay bitwise whatever was prefetched."""

    device = torch.device("cuda", 0)
    engine = _engine(wire_coding="off", prefetch=False)  # 2 MiB slots: 3 staging, 2 restore
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator(device="cpu").manual_seed(5)
    slot_elems = MiB  # bfloat16 elements that fill one 2 MiB slot
    try:
        # one-slot groups g0-g3, a three-slot group g4, then g5-g8, which wrap the staging ring
        # past every segment before them
        sizes = [slot_elems] * 4 + [3 * slot_elems] + [slot_elems] * 4
        handles, gids = [], []
        for n in sizes:
            t = torch.randn(n, generator=g).to(torch.bfloat16).to(device)
            gid, idx = engine.pack(t, stream)
            engine.commit(stream)
            handles.append((t, gid, idx))
            gids.append(gid)
        engine.synchronize()
        issued = lambda: engine.stats()["prefetch_issued"]  # noqa: E731
        base = issued()
        # g3 and g2 take the two restore slots; g1 finds none
        engine._prefetch_groups([gids[3], gids[2], gids[1]], stream)
        assert issued() - base == 2
        _restore_and_check(engine, handles, device, [3, 2])
        # g1 takes one of the two freed slots; g4 needs three and is left alone
        base = issued()
        engine._prefetch_groups([gids[1], gids[4]], stream)
        assert issued() - base == 1
        _restore_and_check(engine, handles, device, [1, 4, 0, 5, 6, 7, 8])
        st = engine.stats()
        assert st["prefetch_hits"] >= 3 and st["copy_failures"] == 0
        for _, gid, idx in handles:
            engine.drop(gid, idx)
        engine.synchronize()
        assert engine.stats()["host_bytes_in_use"] == 0
    finally:
        engine.close()


@pytest.mark.parametrize("wire", ["on", "off"])
def test_coded_segments_keep_to_their_slot_limit(wire) -> None:
    """Wire-coded segments take at most the first max(8, segments of their group + 2) restore
    slots, raw ones the whole ring: with twelve slots, a prefetch of twelve one-segment groups
    fetches eight when they are coded and twelve when they are raw; every restore is bitwise."""

    device = torch.device("cuda", 0)
    cfg = EngineConfig(stage_slot_bytes=2 * MiB, stage_slots=3, restore_slots=12, host_chunk_bytes=8 * MiB,
                       commit_batch_bytes=0, wire_coding=wire, staged_restore=False, prefetch=False,
                       stage_slots_max=0, restore_slots_max=0, restore_small_slots=0)
    engine = OffloadEngine(device, cfg)
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator(device="cpu").manual_seed(11)
    try:
        handles, gids = [], []
        for _ in range(12):
            t = torch.randn(MiB - 4096, generator=g).to(torch.bfloat16).to(device)  # one segment each
            gid, idx = engine.pack(t, stream)
            engine.commit(stream)
            handles.append((t, gid, idx))
            gids.append(gid)
        engine.synchronize()
        assert engine.stats()["wire_segments"] == (12 if wire == "on" else 0)
        base = engine.stats()["prefetch_issued"]
        engine._prefetch_groups(list(reversed(gids)), stream)
        assert engine.stats()["prefetch_issued"] - base == (8 if wire == "on" else 12)
        _restore_and_check(engine, handles, device, list(reversed(range(12))))
        assert engine.stats()["copy_failures"] == 0
        for _, gid, idx in handles:
            engine.drop(gid, idx)
        engine.synchronize()
        assert engine.stats()["host_bytes_in_use"] == 0
    finally:
        engine.close()


@pytest.mark.parametrize("wire", ["off", "on"])
def test_rings_grow_at_the_commit_of_a_large_group(wire) -> None:
    """At the commit of a group of n segments the restore ring grows to n + 2 slots and the
    staging ring to ceil(n / 3), within their caps; smaller groups grow nothing. Groups packed
    and restored across the growth are bitwise, with and without wire coding (whose buffers the
    grown slots get as well)."""

    device = torch.device("cuda", 0)
    slot = 2 * MiB
    engine = _engine(stage_slots=2, restore_slots=2, stage_slots_max=4, restore_slots_max=10, wire_coding=wire,
                     staged_restore=False)
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator(device="cpu").manual_seed(5)
    handles = []

    def group(count: int) -> int:
        copies = engine.stats()["d2h_copies"]
        for _ in range(count):
            t = torch.randn(MiB - 4096, generator=g).to(torch.bfloat16).to(device)  # one slot each
            gid, idx = engine.pack(t, stream)
            handles.append((t, gid, idx))
        engine.commit(stream)
        return engine.stats()["d2h_copies"] - copies  # segments of the group

    try:
        assert engine.stats()["device_ring_bytes"] == 4 * slot
        sizes = []
        n = group(3)
        rings = [(2, max(2, min(10, n + 2)))]
        sizes.append(engine.stats()["device_ring_bytes"])
        n = group(14)
        assert n >= 13
        rings.append((min(4, (n + 2) // 3), min(10, n + 2)))
        sizes.append(engine.stats()["device_ring_bytes"])
        group(2)  # nothing more to grow
        sizes.append(engine.stats()["device_ring_bytes"])
        assert rings[1] == (4, 10)
        if wire == "off":
            assert sizes == [sum(rings[0]) * slot, sum(rings[1]) * slot, sum(rings[1]) * slot]
        else:
            assert engine.stats()["wire_segments"] > 0
            assert sizes[0] < sizes[1] == sizes[2]
        _restore_and_check(engine, handles, device, list(reversed(range(len(handles)))))
        stats = engine.stats()
        assert stats["copy_failures"] == 0 and stats["prefetch_hits"] > 0
        # a second step runs on the grown rings
        first = len(handles)
        group(14)
        group(3)
        assert engine.stats()["device_ring_bytes"] == sizes[2]
        _restore_and_check(engine, handles, device, list(reversed(range(first, len(handles)))))
        for _, gid, idx in handles:
            engine.drop(gid, idx)
        engine.synchronize()
        assert engine.stats()["host_bytes_in_use"] == 0
    finally:
        engine.close()


def test_shared_entry_of_an_older_large_group_is_restored_alone() -> None:
    """An entry of a large group asked for while a younger group still waits (a save later
    blocks share, kept once by deduplication) is restored alone: its group's other entries stay
    on the host until their own turn, nothing else is scattered, and every restore is bitwise.
    A small group asked for out of order is restored whole, as before."""

    device = torch.device("cuda", 0)
    engine = _engine(stage_slots=3, restore_slots=6, wire_coding="off", staged_restore=False,
                     restore_ahead_bytes=1 * MiB)
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator(device="cpu").manual_seed(7)

    def tensor(n):
        return torch.randn(n, generator=g).to(torch.bfloat16).to(device)

    try:
        old = [tensor(600_000) for _ in range(3)]  # about 3.6 MB: a large group
        refs_old = [engine.pack(t, stream) for t in old]
        engine.commit(stream)
        small = tensor(40_000)  # 80 KB: a small group
        ref_small = engine.pack(small, stream)
        small_other = tensor(30_000)
        ref_small_other = engine.pack(small_other, stream)
        engine.commit(stream)
        young = [tensor(500_000) for _ in range(2)]
        refs_young = [engine.pack(t, stream) for t in young]
        gid_shared, idx_shared = refs_old[1]
        assert engine.acquire(gid_shared, idx_shared)  # the younger block saves it again
        engine.commit(stream)
        engine.synchronize()

        before = engine.stats()
        got = engine.restore(gid_shared, idx_shared, stream)  # asked for before the young group
        assert_bitwise(got, old[1])
        after = engine.stats()
        assert after["py_ahead_alone"] - before["py_ahead_alone"] == 1
        assert after["bytes_unpacked"] - before["bytes_unpacked"] == old[1].numel() * 2
        # the small group asked for out of order comes back whole
        assert_bitwise(engine.restore(*ref_small, stream), small)
        assert engine.stats()["bytes_unpacked"] - after["bytes_unpacked"] == (small.numel() + small_other.numel()) * 2
        assert engine.stats()["py_ahead_alone"] == after["py_ahead_alone"]
        # backward order from here: the young group, the shared entry's second reference, the rest
        for (gid, idx), t in zip(refs_young, young):
            assert_bitwise(engine.restore(gid, idx, stream), t)
        assert_bitwise(engine.restore(gid_shared, idx_shared, stream), old[1])
        assert_bitwise(engine.restore(*ref_small_other, stream), small_other)
        for (gid, idx), t in zip(refs_old, old):
            if idx != idx_shared:
                assert_bitwise(engine.restore(gid, idx, stream), t)
        assert engine.stats()["copy_failures"] == 0
        for gid, idx in refs_old + refs_young + [ref_small, ref_small_other, (gid_shared, idx_shared)]:
            engine.drop(gid, idx)
        engine.synchronize()
        assert engine.stats()["groups_live"] == 0 and engine.stats()["host_bytes_in_use"] == 0
    finally:
        engine.close()


def test_prefetch_entry_fetches_only_the_segments_holding_it() -> None:
    """mo_prefetch_entry queues the H2D of the segments that hold one entry of a group, not the
    group's others: of four one-segment entries it fetches one, and the group's restore then
    finds that one resident and fetches the other three. A bad entry index is an error."""

    from moss_offload import _native

    device = torch.device("cuda", 0)
    engine = _engine(stage_slots=4, restore_slots=6, wire_coding="off", staged_restore=False, prefetch=False)
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator(device="cpu").manual_seed(12)
    try:
        ts = [torch.randn(MiB - 4096, generator=g).to(torch.bfloat16).to(device) for _ in range(4)]  # a slot each
        refs = [engine.pack(t, stream) for t in ts]
        engine.commit(stream)
        engine.synchronize()
        gid = refs[0][0]
        assert engine.stats()["d2h_copies"] == 4
        before = engine.stats()
        engine.prefetch_entry(gid, 2, stream)
        assert engine.stats()["prefetch_issued"] - before["prefetch_issued"] == 1
        assert_bitwise(engine.restore(gid, 2, stream), ts[2])  # restores the whole group
        after = engine.stats()
        assert after["prefetch_hits"] - before["prefetch_hits"] == 1
        assert after["restore_fetches"] - before["restore_fetches"] == 3
        for (_, idx), t in zip(refs, ts):
            if idx != 2:
                assert_bitwise(engine.restore(gid, idx, stream), t)
        with pytest.raises(RuntimeError, match="no entry 99"):
            _native.check("mo_prefetch_entry", engine._lib.mo_prefetch_entry(engine._handle, gid, 99, stream))
        for gid_, idx in refs:
            engine.drop(gid_, idx)
    finally:
        engine.close()


@pytest.mark.parametrize("layout", ["dense", "transposed", "padded"])
def test_each_reader_of_a_shared_entry_gets_its_own_bitwise_copy(layout) -> None:
    """A save deduplicated for three readers is restored once; the first two takes get copies
    of their own (the engine's scatter kernel for layouts without gaps, ``copy_`` otherwise),
    the last the restored tensor itself: all bitwise, all with the save's strides, no two
    sharing storage."""

    device = torch.device("cuda", 0)
    engine = _engine(stage_slots=3, restore_slots=4, wire_coding="off")
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator(device="cpu").manual_seed(9)
    base = torch.randn(4 * 384 * 130, generator=g).to(torch.bfloat16).to(device)
    if layout == "dense":
        t = base[: 384 * 520].view(384, 520)
    elif layout == "transposed":
        t = base[: 4 * 384 * 128].view(4, 384, 128).transpose(0, 1)  # [384, 4, 128], strides (128, 49152, 1)
    else:
        t = base.view(4 * 384, 130)[:, :128]  # rows of 128 with a 2-element gap
    try:
        gid, idx = engine.pack(t, stream)
        assert engine.acquire(gid, idx) and engine.acquire(gid, idx)
        engine.commit(stream)
        engine.synchronize()
        got = []
        for _ in range(3):
            r = engine.restore(gid, idx, stream)
            assert r.stride() == t.stride()
            assert_bitwise(r, t)
            got.append(r)
            engine.drop(gid, idx)
        ptrs = {r.untyped_storage().data_ptr() for r in got}
        assert len(ptrs) == 3
        torch.cuda.synchronize(device)
        for r in got:
            assert_bitwise(r, t)
        assert engine.stats()["copy_failures"] == 0
    finally:
        engine.close()


def _ring(engine) -> tuple[int, int, int]:
    st = engine.stats()
    return st["restore_slots_big"], st["restore_slots_small"], st["device_ring_bytes"]


def test_small_restore_slots_for_runs_of_small_groups() -> None:
    """restore_small_slots: after eight groups in a row whose segments fit a quarter slot, the
    restore ring gains small slots, which such segments take (given memory at first use) before
    a full-size one; a larger group's segments take full-size slots, the two past the first
    given memory at first use; trim gives back every slot past the first two. Restores stay
    bitwise throughout."""

    device = torch.device("cuda", 0)
    engine = _engine(restore_slots=4, restore_small_slots=6, wire_coding="off", staged_restore=False,
                     prefetch=False)  # 2 MiB slots: small ones of 512 KiB
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator(device="cpu").manual_seed(11)
    base = (3 + 2) * 2 * MiB
    try:
        assert _ring(engine) == (2, 0, base)

        def group(n):
            t = torch.randn(n, generator=g).to(torch.bfloat16).to(device)
            gid, idx = engine.pack(t, stream)
            engine.commit(stream)
            return t, gid, idx

        # seven groups of 400 KB, one segment each (five to a staging slot): no small slot yet,
        # so the last one comes back through a full-size slot
        handles = [group(200_000) for _ in range(7)]
        _restore_and_check(engine, handles, device, [6])
        assert _ring(engine) == (2, 0, base)
        # three more: the eighth in a row added six small slots, which the restores take
        handles += [group(200_000) for _ in range(3)]
        _restore_and_check(engine, handles, device, [9, 8, 7, 5, 4, 3, 2, 1, 0])
        assert _ring(engine) == (2, 6, base + 6 * MiB // 2)
        # a 3 MB group spans two full-size segments: its restore gives memory to one or both of
        # the full-size slots that had none
        handles.append(group(1_500_000))
        _restore_and_check(engine, handles, device, [10])
        big, small, ring = _ring(engine)
        assert big in (3, 4) and small == 6 and ring == (3 + big) * 2 * MiB + 6 * MiB // 2
        assert engine.stats()["copy_failures"] == 0
        for _, gid, idx in handles:
            engine.drop(gid, idx)
        engine.synchronize()
        engine.trim()
        assert _ring(engine) == (2, 0, base)
        # the small slots, their memory given back, take a second round again
        handles = [group(200_000) for _ in range(9)]
        _restore_and_check(engine, handles, device, list(reversed(range(9))))
        assert _ring(engine)[:2] == (2, 6)
        for _, gid, idx in handles:
            engine.drop(gid, idx)
        engine.synchronize()
        assert engine.stats()["host_bytes_in_use"] == 0
    finally:
        engine.close()


def test_prefetch_of_small_segments_gives_no_full_size_slot_memory() -> None:
    """A prefetch places segments that fit a small slot in small slots (given memory) or in
    full-size slots that already have memory, never in one it would have to give memory to."""

    device = torch.device("cuda", 0)
    engine = _engine(restore_slots=6, restore_small_slots=3, wire_coding="off", staged_restore=False,
                     prefetch=False)
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator(device="cpu").manual_seed(12)
    try:
        handles, gids = [], []
        for _ in range(12):
            t = torch.randn(120_000, generator=g).to(torch.bfloat16).to(device)  # 240 KB, one segment
            gid, idx = engine.pack(t, stream)
            engine.commit(stream)
            handles.append((t, gid, idx))
            gids.append(gid)
        engine.synchronize()
        before = engine.stats()["prefetch_issued"]
        # five groups nearest first: three small slots and the two full-size slots with memory;
        # the sixth would need a full-size slot given memory and is left
        engine._prefetch_groups(list(reversed(gids))[:6], stream)
        st = engine.stats()
        assert st["prefetch_issued"] - before == 5
        assert (st["restore_slots_big"], st["restore_slots_small"]) == (2, 3)
        _restore_and_check(engine, handles, device, list(reversed(range(12))))
        st = engine.stats()
        assert st["prefetch_hits"] >= 5 and st["copy_failures"] == 0
        assert st["restore_slots_big"] == 2  # every segment found a small or a full-size slot with memory
        for _, gid, idx in handles:
            engine.drop(gid, idx)
    finally:
        engine.close()


def test_fixed_rings_do_not_grow() -> None:
    """Caps of 0 keep the configured rings whatever the group size."""

    device = torch.device("cuda", 0)
    engine = _engine(stage_slots=2, restore_slots=2, wire_coding="off", staged_restore=False)
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator(device="cpu").manual_seed(6)
    try:
        handles = []
        for _ in range(9):
            t = torch.randn(MiB - 4096, generator=g).to(torch.bfloat16).to(device)
            handles.append((t, *engine.pack(t, stream)))
        engine.commit(stream)
        assert engine.stats()["device_ring_bytes"] == 4 * 2 * MiB
        _restore_and_check(engine, handles, device, list(reversed(range(len(handles)))))
        for _, gid, idx in handles:
            engine.drop(gid, idx)
    finally:
        engine.close()


def test_trim_frees_wire_buffers_only_with_no_group_live() -> None:
    """mo_trim keeps the wire buffers while a group is live (its restore still decodes
    bitwise) and frees them once none is; the next coded segment allocates them again."""

    device = torch.device("cuda", 0)
    engine = _engine(wire_coding="on")
    stream = torch.cuda.current_stream(device).cuda_stream
    rings = engine.stats()["device_ring_bytes"]  # no wire buffers yet
    assert rings == (3 + 2) * 2 * MiB
    g = torch.Generator(device="cpu").manual_seed(11)

    def round_trip(trim_while_live: bool) -> None:
        t = torch.randn(700_000, generator=g).to(torch.bfloat16).to(device)
        gid, idx = engine.pack(t, stream)
        engine.commit(stream)
        engine.synchronize()
        st = engine.stats()
        coded = st["device_ring_bytes"]
        assert coded > rings  # the segment was coded: wire buffers exist
        # its host copy, sized for the largest stream, shrank to the stream once the D2H landed
        assert st["wire_bytes"] > 0
        assert st["host_bytes_in_use"] <= 0.72 * t.numel() * 2 + 4096
        if trim_while_live:
            engine.trim()
            assert engine.stats()["device_ring_bytes"] == coded
        assert_bitwise(engine.restore(gid, idx, stream), t)
        engine.drop(gid, idx)
        engine.synchronize()
        engine.trim()
        assert engine.stats()["device_ring_bytes"] == rings

    try:
        round_trip(trim_while_live=True)
        round_trip(trim_while_live=False)  # buffers allocated again after the trim
        assert engine.stats()["wire_segments"] >= 2
    finally:
        engine.close()


def test_wire_coding_is_skipped_on_the_hip_stream_link() -> None:
    """The HIP-stream transport enqueues copies before their sizes exist, so segments stay raw."""

    device = torch.device("cuda", 0)
    engine = _engine(wire_coding="on", link="hipdma")
    stream = torch.cuda.current_stream(device).cuda_stream
    t = torch.randn(600_000, device=device).to(torch.bfloat16)
    gid, idx = engine.pack(t, stream)
    engine.commit(stream)
    assert_bitwise(engine.restore(gid, idx, stream), t)
    engine.synchronize()
    assert engine.stats()["wire_segments"] == 0
    engine.drop(gid, idx)
    engine.synchronize()
    engine.close()


def test_wire_buffers_past_the_device_limit_fall_back_to_raw_segments() -> None:
    """Wire buffers are an optimisation: where they would pass ``wire_device_limit`` (or their
    allocation fails) segments cross raw, the step goes on, and the next forward tries again."""

    device = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator(device="cpu").manual_seed(13)
    engine = _engine(wire_coding="on", wire_device_limit=1)
    try:
        for forward in range(2):
            handles = []
            for _ in range(3):
                t = torch.randn(600_000, generator=g).to(torch.bfloat16).to(device)
                handles.append((t, *engine.pack(t, stream)))
                engine.commit(stream)
            _restore_and_check(engine, handles, device, range(len(handles) - 1, -1, -1))
            for _, gid, idx in handles:
                engine.drop(gid, idx)
            engine.synchronize()
            st = engine.stats()
            assert st["wire_segments"] == 0 and st["wire_fallbacks"] >= 3 * (forward + 1), st["wire_fallbacks"]
            assert st["device_ring_bytes"] == (3 + 2) * 2 * MiB  # no wire buffer was kept
            assert st["bytes_d2h"] >= st["bytes_packed"] and st["copy_failures"] == 0
    finally:
        engine.close()
    # a limit the buffers fit in codes as usual
    engine = _engine(wire_coding="on", wire_device_limit=1 << 30)
    try:
        t = torch.randn(600_000, generator=g).to(torch.bfloat16).to(device)
        gid, idx = engine.pack(t, stream)
        engine.commit(stream)
        assert_bitwise(engine.restore(gid, idx, stream), t)
        engine.drop(gid, idx)
        engine.synchronize()
        assert engine.stats()["wire_segments"] == 1 and engine.stats()["wire_fallbacks"] == 0
    finally:
        engine.close()


def test_resident_coded_slot_restored_on_a_second_stream() -> None:
    """A wire-coded segment decoded into its restore slot by an unpack on one stream, then
    unpacked again from the slot on another stream (a retained graph's second backward there):
    the second stream is ordered after the first one's decode and scatter, and the slot's next
    refill after both streams' reads."""

    device = torch.device("cuda", 0)
    main = torch.cuda.current_stream(device)
    side = torch.cuda.Stream(device=device)
    g = torch.Generator(device="cpu").manual_seed(17)
    engine = _engine(wire_coding="on", staged_restore=False, prefetch=False)
    try:
        tensors = [torch.randn(450_000, generator=g).to(torch.bfloat16).to(device) for _ in range(4)]
        handles = []
        for t in tensors:
            handles.append((t, *engine.pack(t, main.cuda_stream)))
            engine.commit(main.cuda_stream)
        engine.synchronize()
        t, gid, idx = handles[-1]
        first = engine.restore(gid, idx, main.cuda_stream)  # fetch, decode and scatter on main
        side.wait_stream(main)  # the restored tensor's allocation is main's; the slot is not
        with torch.cuda.stream(side):
            second = engine.restore(gid, idx, side.cuda_stream)  # the resident slot, read on side
            second_bits = second.clone()
        main.wait_stream(side)
        assert_bitwise(first, t)
        assert_bitwise(second_bits, t)
        # the other groups reuse the two restore slots after both reads
        _restore_and_check(engine, handles, device, [2, 1, 0])
        assert engine.stats()["wire_segments"] == 4
        for _, gid_, idx_ in handles:
            engine.drop(gid_, idx_)
        engine.synchronize()
    finally:
        engine.close()


def test_small_groups_restored_ahead_share_one_scatter_launch() -> None:
    """mo_unpack_groups through ``restore``: when a group is asked for, the next groups backward
    needs join its scatter launch if their bytes are on the device already (prefetched and
    landed), within ``restore_ahead_bytes``; a group whose H2D was never issued is left for its
    own unpack. Every restore is bitwise, whichever launch wrote it."""

    device = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator(device="cpu").manual_seed(19)
    # 8 MiB slots: each 1.5 MB group is one segment; 6 restore slots hold the prefetched ones
    cfg = EngineConfig(stage_slot_bytes=8 * MiB, stage_slots=2, restore_slots=6, host_chunk_bytes=32 * MiB,
                       wire_coding="off", staged_restore=False, prefetch=False, restore_ahead_bytes=5 * MiB,
                       stage_slots_max=0, restore_slots_max=0, restore_small_slots=0)
    engine = OffloadEngine(device, cfg)
    try:
        handles = []
        for k in range(8):
            group = [torch.randn(n, generator=g).to(device) for n in (300_000, 70_000, 5)]
            members = [(t, *engine.pack(t, stream)) for t in group]
            engine.commit(stream)
            handles.append(members)
        engine.synchronize()
        gids = [members[0][1] for members in handles]
        # groups 7..3 prefetched and landed; 2..0 never fetched
        engine._prefetch_groups(gids[7:2:-1], stream)
        engine.synchronize()
        torch.cuda.synchronize(device)
        base = engine.stats()["unpack_launches"]
        t, gid, idx = handles[7][0]
        assert_bitwise(engine.restore(gid, idx, stream), t)
        # group 7 plus groups 6, 5 and 4 (3 x 1.48 MB within 5 MiB; group 3 would pass it): one launch
        assert engine.stats()["unpack_launches"] - base == 1
        for k in (6, 5, 4):
            assert all(engine._groups[gids[k]].entries[j].restored is not None for j in range(3))
        assert engine._groups[gids[3]].entries[0].restored is None
        taken = {(7, 0)}
        for k in (7, 6, 5, 4):
            for j, (t, gid, idx) in enumerate(handles[k]):
                if (k, j) not in taken:
                    assert_bitwise(engine.restore(gid, idx, stream), t)
                    taken.add((k, j))
        assert engine.stats()["unpack_launches"] - base == 1  # 6, 5, 4 came from the cache
        # group 3 is resident and landed, groups 2 and 1 were never fetched: 3 alone
        t, gid, idx = handles[3][0]
        assert_bitwise(engine.restore(gid, idx, stream), t)
        taken.add((3, 0))
        assert engine.stats()["unpack_launches"] - base == 2
        assert engine._groups[gids[2]].entries[0].restored is None
        for k in (3, 2, 1, 0):
            for j, (t, gid, idx) in enumerate(handles[k]):
                if (k, j) not in taken:
                    assert_bitwise(engine.restore(gid, idx, stream), t)
        st = engine.stats()
        assert st["bytes_unpacked"] == st["bytes_packed"] and st["copy_failures"] == 0
        for members in handles:
            for _, gid, idx in members:
                engine.drop(gid, idx)
        engine.synchronize()
        assert engine.stats()["host_bytes_in_use"] == 0
    finally:
        engine.close()


def _d2h_complete(engine, gid: int) -> bool:
    import ctypes

    done = ctypes.c_int(-1)
    assert engine._lib.mo_group_info(engine._handle, gid, None, None, ctypes.byref(done)) == 0
    return bool(done.value)


def test_commits_gather_together_up_to_commit_batch_bytes() -> None:
    """commit_batch_bytes: a committed group's segment waits, gathers and all, for later
    commits until the batch would pass the limit; then one launch gathers the waiting groups
    and their D2Hs follow. A restore, a release and a filled staging slot send what waits
    first. Every restore is bitwise; a waiting group reports its D2H as not complete."""

    device = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(device).cuda_stream
    g = torch.Generator(device="cpu").manual_seed(23)
    # 2 MB groups; an 8 MiB slot holds four of them
    cfg = EngineConfig(stage_slot_bytes=8 * MiB, stage_slots=3, restore_slots=4, host_chunk_bytes=32 * MiB,
                       commit_batch_bytes=5 * MiB, wire_coding="off", prefetch=False, stage_slots_max=0,
                       restore_slots_max=0, restore_small_slots=0)
    engine = OffloadEngine(device, cfg)
    try:
        groups = []

        def add_group():
            t = torch.randn(500_000, generator=g).to(device)
            gid, idx = engine.pack(t, stream)
            engine.commit(stream)
            groups.append((t, gid, idx))
            return gid

        base = engine.stats()["pack_launches"]
        g0 = add_group()
        g1 = add_group()
        # 4 MB wait: nothing gathered, nothing sent, their sources held
        assert engine.stats()["pack_launches"] - base == 0
        assert engine.stats()["d2h_copies"] == 0 and engine._held
        assert not _d2h_complete(engine, g0) and not _d2h_complete(engine, g1)
        add_group()  # 6 MB would pass 5 MiB: the three go out in one launch
        assert engine.stats()["pack_launches"] - base == 1
        assert engine.stats()["d2h_copies"] == 3 and not engine._held
        g3 = add_group()  # waits again
        assert engine.stats()["d2h_copies"] == 3
        # the fifth group does not fit the slot's last 0.39 MB: the ring moves on, which sends
        # group 3 first; group 4 then waits in the next slot
        g4 = add_group()
        assert engine.stats()["d2h_copies"] == 4 and not _d2h_complete(engine, g4)
        g5 = add_group()  # waits beside group 4
        assert engine.stats()["d2h_copies"] == 4 and not _d2h_complete(engine, g5)
        # a release of a waiting group sends the waiting segments first, then drops it
        t5, _, idx5 = groups[5]
        engine.drop(g5, idx5)
        assert engine.stats()["d2h_copies"] == 6 and not engine._held
        g6 = add_group()  # waits
        assert engine.stats()["d2h_copies"] == 6 and not _d2h_complete(engine, g6)
        # restores, newest first, each bitwise (a restore sends what waits first)
        for t, gid, idx in reversed(groups):
            if gid == g5:
                continue
            assert_bitwise(engine.restore(gid, idx, stream), t)
        engine.synchronize()
        assert all(_d2h_complete(engine, gid) for _, gid, _ in groups if gid != g5)
        assert _d2h_complete(engine, g3)
        st = engine.stats()
        assert st["bytes_unpacked"] == st["bytes_packed"] - t5.numel() * 4 and st["copy_failures"] == 0
        for _, gid, idx in groups:
            if gid != g5:
                engine.drop(gid, idx)
        engine.synchronize()
        assert engine.stats()["host_bytes_in_use"] == 0
    finally:
        engine.close()
