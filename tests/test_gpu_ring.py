"""The native block ring (``mo_streamer_stage`` .. ``mo_streamer_slot_info``) through its C ABI.

Three blocks with distinct byte patterns live in pinned masters; a two-slot ring makes them
resident on demand. Checked: a resident block is not copied again; a new block takes an empty
slot, else the least recently staged one that is neither pinned nor kept; a slot's contents
equal its block's master after ``ready``; generations reject calls about a slot that moved on;
a dirty slot is copied back to its master before the slot takes another block (and by evict);
with every slot pinned, staging fails loudly instead of overwriting a slot in use.
"""

from __future__ import annotations

import pytest
import torch

from moss_offload._native import EngineError
from moss_offload.ring import BlockRing, Master, PinnedArena

from gpu_util import requires_gpu

pytestmark = requires_gpu

KiB = 1 << 10


def _masters(count=3, nbytes=256 * KiB):
    arena = PinnedArena(count * nbytes)
    masters = []
    for k in range(count):
        view = arena.tensor[k * nbytes : (k + 1) * nbytes]
        view.copy_(torch.arange(nbytes, dtype=torch.int64).mul(7 + 13 * k).add(k).to(torch.uint8))
        masters.append(Master(arena.address + k * nbytes, nbytes, view))
    return arena, masters


def _slot_bytes(ring, lease, nbytes):
    ring.ready(lease)
    return ring.buffers[lease.slot][:nbytes].cpu()


def test_stage_reuses_resident_blocks_and_replaces_the_least_recent() -> None:
    device = torch.device("cuda", 0)
    _, (m0, m1, m2) = _masters()
    ring = BlockRing(device, 2, 256 * KiB)
    try:
        a = ring.stage(0, m0)
        assert a.filled and ring.resident() == (0,)
        again = ring.stage(0, m0)
        assert not again.filled and (again.slot, again.generation) == (a.slot, a.generation)
        b = ring.stage(1, m1, keep=0)
        assert b.filled and b.slot != a.slot and ring.resident() == (0, 1)
        assert torch.equal(_slot_bytes(ring, a, m0.nbytes), m0.tensor)
        assert torch.equal(_slot_bytes(ring, b, m1.nbytes), m1.tensor)
        # block 0 staged longest ago: block 2 replaces it (nothing pinned or kept)
        ring.stage(1, m1)
        c = ring.stage(2, m2)
        assert c.filled and c.slot == a.slot and c.generation == a.generation + 1
        assert ring.resident() == (1, 2)
        assert torch.equal(_slot_bytes(ring, c, m2.nbytes), m2.tensor)
        # keep: block 0 may not replace block 2 (kept) and so replaces block 1
        d = ring.stage(0, m0, keep=2)
        assert d.slot == b.slot and ring.resident() == (0, 2)
        assert ring.fills == 4 and ring.stats()["fills"] == 4
    finally:
        torch.cuda.synchronize()
        ring.close()


def test_pins_and_generations() -> None:
    device = torch.device("cuda", 0)
    _, (m0, m1, m2) = _masters()
    ring = BlockRing(device, 2, 256 * KiB)
    try:
        a = ring.stage(0, m0)
        b = ring.stage(1, m1)
        ring.pin(a)
        ring.pin(b)
        assert ring.info(a.slot)[1] == 1
        with pytest.raises(EngineError, match="no staging slot can take block 2"):
            ring.stage(2, m2)
        ring.unpin(b)
        c = ring.stage(2, m2)  # block 1's slot, the only unpinned one
        assert c.slot == b.slot
        with pytest.raises(EngineError, match="no longer holds"):
            ring.unpin(b)  # generation of the block that left
        with pytest.raises(EngineError, match="not pinned"):
            ring.unpin(c)
        with pytest.raises(EngineError, match="in use by a running block"):
            ring.evict(a.slot)
        ring.unpin(a)
        ring.evict(a.slot)
        assert ring.info(a.slot)[0] == -1 and ring.resident() == (2,)
    finally:
        torch.cuda.synchronize()
        ring.close()


def test_dirty_slots_are_written_back_before_reuse_and_on_evict() -> None:
    device = torch.device("cuda", 0)
    arena, (m0, m1, m2) = _masters()
    ring = BlockRing(device, 2, 256 * KiB)
    try:
        a = ring.stage(0, m0)
        b = ring.stage(1, m1)
        ring.pin(a)
        ring.ready(a)
        ring.buffers[a.slot][: m0.nbytes].add_(1)  # an in-place update on the device
        expected0 = ring.buffers[a.slot][: m0.nbytes].cpu()
        ring.mark_dirty(a)
        ring.unpin(a)  # release point after the update
        assert ring.info(a.slot)[2] is True
        ring.stage(1, m1)  # block 0 is now the least recent
        c = ring.stage(2, m2)  # replaces dirty block 0: write-back, then the fill
        assert c.slot == a.slot
        assert torch.equal(_slot_bytes(ring, c, m2.nbytes), m2.tensor)
        ring.synchronize()
        assert torch.equal(m0.tensor, expected0)
        # a clean slot is not written back; evict writes a dirty one
        ring.pin(b)
        ring.ready(b)
        ring.buffers[b.slot][: m1.nbytes].mul_(3)
        expected1 = ring.buffers[b.slot][: m1.nbytes].cpu()
        ring.mark_dirty(b)
        ring.unpin(b)
        writebacks = ring.stats()["writebacks"]
        ring.evict(b.slot)
        ring.synchronize()
        assert ring.stats()["writebacks"] == writebacks + 1
        assert torch.equal(m1.tensor, expected1)
        ring.evict(c.slot)  # clean
        ring.synchronize()
        assert ring.stats()["writebacks"] == writebacks + 1 and ring.stats()["copy_failures"] == 0
    finally:
        torch.cuda.synchronize()
        ring.close()
    del arena
