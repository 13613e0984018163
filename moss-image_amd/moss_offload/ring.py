"""Device slots for streamed blocks; residency lives in the native ring.

Both block streamers (:mod:`moss_offload.memory` for frozen blocks, :mod:`moss_offload.trainable_offload`
for blocks a fused optimizer updates in place) keep a block's tensors in one pinned host
*master* and run it from one of a few device *slots*. Which block a slot holds, which slot a new
block replaces, how many running executions still read a slot, and whether a slot must be written
back before reuse are decided by the native streamer (``mo_streamer_stage`` and the calls after
it, ``csrc/mo_streamer.cpp``); the copies themselves run on SDMA engines, ordered against the
compute stream by the slot's release points. This module is the thin Python face of that ring
plus the bookkeeping both streamers share: where the tensors of a block sit in its master, and
whether the checkpoint is recomputing (backward) or running forward.
"""

from __future__ import annotations

import ctypes
import threading
import weakref
from dataclasses import dataclass

import torch

from . import _native

ALIGN = 256


def align(offset: int) -> int:
    return (offset + ALIGN - 1) // ALIGN * ALIGN


class PinnedArena:
    """One exact-size pinned host allocation (``mo_pinned_alloc``), as a CPU ``uint8`` tensor.

    Views of :attr:`tensor` keep the allocation alive; it returns to the HIP runtime with the last
    view. Torch's caching host allocator, by contrast, rounds every pin up to a power of two.
    """

    def __init__(self, nbytes: int) -> None:
        lib = _native.load()
        host = ctypes.c_uint64()
        _native.check("mo_pinned_alloc", lib.mo_pinned_alloc(max(nbytes, 1), ctypes.byref(host)))
        self.address = int(host.value)
        self.nbytes = nbytes
        buffer = (ctypes.c_uint8 * max(nbytes, 1)).from_address(self.address)
        weakref.finalize(buffer, lib.mo_pinned_free, self.address)
        self.tensor = torch.frombuffer(buffer, dtype=torch.uint8)[:nbytes]


@dataclass(frozen=True)
class Placement:
    """Where one tensor of a block sits in the block's packed bytes."""

    offset: int
    nbytes: int
    shape: torch.Size
    dtype: torch.dtype

    def view(self, flat: torch.Tensor) -> torch.Tensor:
        return flat[self.offset : self.offset + self.nbytes].view(self.dtype).view(self.shape)


def plan(tensors) -> tuple[list[Placement], int]:
    """Placements of ``tensors`` packed back to back at ``ALIGN``-byte offsets, and the size."""

    out, end = [], 0
    for tensor in tensors:
        start = align(end)
        nbytes = tensor.numel() * tensor.element_size()
        out.append(Placement(start, nbytes, tensor.shape, tensor.dtype))
        end = start + nbytes
    return out, align(end)


@dataclass(frozen=True)
class Master:
    """A block's packed tensors in pinned host memory: ``host`` address, ``nbytes`` long."""

    host: int
    nbytes: int
    tensor: torch.Tensor  # CPU uint8 view of the same bytes


@dataclass(frozen=True)
class Lease:
    """A block resident in ``slot`` since fill ``generation``; ``filled``: this stage copied it."""

    block: int
    slot: int
    generation: int
    filled: bool


class BlockRing:
    """``slots`` device buffers of ``capacity`` bytes driven by one native streamer."""

    def __init__(self, device: torch.device, slots: int, capacity: int, h2d_engine: int = 0) -> None:
        self.device = torch.device(device)
        index = self.device.index if self.device.index is not None else torch.cuda.current_device()
        self.capacity = capacity
        self._lib = _native.load()
        handle = ctypes.c_void_p()
        _native.check("mo_streamer_create",
                      self._lib.mo_streamer_create(index, slots, h2d_engine, ctypes.byref(handle)))
        self._handle = handle
        self.buffers: list[torch.Tensor | None] = [None] * slots
        for slot in range(slots):
            self._attach(slot)
        self._out_slot = ctypes.c_uint32()
        self._out_generation = ctypes.c_uint64()
        self._out_filled = ctypes.c_int()
        self.fills = 0
        self.lock = threading.RLock()

    def _attach(self, slot: int) -> None:
        buffer = torch.empty(self.capacity, dtype=torch.uint8, device=self.device)
        _native.check("mo_streamer_attach",
                      self._lib.mo_streamer_attach(self._handle, slot, buffer.data_ptr(), self.capacity))
        self.buffers[slot] = buffer

    @property
    def open(self) -> bool:
        return bool(self._handle)

    def _stream(self, stream) -> int:
        return (stream or torch.cuda.current_stream(self.device)).cuda_stream

    def stage(self, block: int, master: Master, keep: int | None = None) -> Lease:
        """Make ``block`` resident (a fill on the SDMA engine if it is not); never blocks."""

        _native.check(
            "mo_streamer_stage",
            self._lib.mo_streamer_stage(self._handle, block, master.host, master.nbytes,
                                        -1 if keep is None else keep, ctypes.byref(self._out_slot),
                                        ctypes.byref(self._out_generation), ctypes.byref(self._out_filled)),
        )
        filled = bool(self._out_filled.value)
        self.fills += filled
        return Lease(block, int(self._out_slot.value), int(self._out_generation.value), filled)

    def pin(self, lease: Lease) -> None:
        _native.check("mo_streamer_pin", self._lib.mo_streamer_pin(self._handle, lease.slot, lease.generation))

    def unpin(self, lease: Lease, stream=None) -> None:
        """The slot may be reused once ``stream`` (default: current) reaches this point."""

        _native.check("mo_streamer_unpin",
                      self._lib.mo_streamer_unpin(self._handle, lease.slot, lease.generation, self._stream(stream)))

    def ready(self, lease: Lease, stream=None) -> None:
        """Order work enqueued on ``stream`` from now on after the lease's fill."""

        _native.check("mo_streamer_acquire",
                      self._lib.mo_streamer_acquire(self._handle, lease.slot, self._stream(stream)))

    def mark_dirty(self, lease: Lease, dirty: bool = True) -> None:
        _native.check("mo_streamer_mark_dirty",
                      self._lib.mo_streamer_mark_dirty(self._handle, lease.slot, lease.generation, int(dirty)))

    def evict(self, slot: int) -> None:
        _native.check("mo_streamer_evict", self._lib.mo_streamer_evict(self._handle, slot))

    def info(self, slot: int) -> tuple[int, int, bool, int]:
        """``(block or -1, pins, dirty, generation)`` of ``slot``."""

        block, pins, dirty, generation = ctypes.c_int64(), ctypes.c_uint32(), ctypes.c_int(), ctypes.c_uint64()
        _native.check("mo_streamer_slot_info",
                      self._lib.mo_streamer_slot_info(self._handle, slot, ctypes.byref(block), ctypes.byref(pins),
                                                      ctypes.byref(dirty), ctypes.byref(generation)))
        return int(block.value), int(pins.value), bool(dirty.value), int(generation.value)

    def resident(self) -> tuple[int, ...]:
        if not self._handle:
            return ()
        return tuple(sorted(b for b in (self.info(k)[0] for k in range(len(self.buffers))) if b >= 0))

    def slot_of(self, block: int) -> int | None:
        for slot in range(len(self.buffers)):
            if self.info(slot)[0] == block:
                return slot
        return None

    def synchronize(self) -> None:
        _native.check("mo_streamer_synchronize", self._lib.mo_streamer_synchronize(self._handle))

    def stats(self) -> dict:
        out = _native.MoStreamerStats()
        _native.check("mo_streamer_get_stats", self._lib.mo_streamer_get_stats(self._handle, ctypes.byref(out)))
        return out.as_dict()

    def reset_stats(self) -> None:
        _native.check("mo_streamer_reset_stats", self._lib.mo_streamer_reset_stats(self._handle))

    def close(self) -> None:
        """Finish every copy and free the streamer; the slot buffers go with it."""

        if not self._handle:
            return
        _native.check("mo_streamer_destroy", self._lib.mo_streamer_destroy(self._handle))
        self._handle = ctypes.c_void_p()
        self.buffers = [None] * len(self.buffers)


class RecomputePhase:
    """Whether this thread is inside a checkpoint's recomputation (backward) right now.

    A block run by a non-reentrant checkpoint executes twice: in the forward, and again when
    backward first needs its saved tensors. The checkpoint's ``context_fn`` enters
    :meth:`recomputing` around the second run; recomputations nest (a depth count per thread).
    """

    def __init__(self) -> None:
        self._local = threading.local()

    @property
    def active(self) -> bool:
        return getattr(self._local, "depth", 0) > 0

    def recomputing(self):
        phase = self

        class _Enter:
            def __enter__(self_inner):
                phase._local.depth = getattr(phase._local, "depth", 0) + 1

            def __exit__(self_inner, *exc):
                depth = getattr(phase._local, "depth", 0)
                if depth <= 0:
                    raise RuntimeError("checkpoint recomputation ended without having started")
                phase._local.depth = depth - 1
                return False

        return _Enter()


def stopped_recomputation(error: BaseException) -> bool:
    """Non-reentrant checkpointing ends a recomputation early, by raising this error, once the
    tensors backward needs exist; the block's run is then complete as far as backward goes."""

    kind = type(error)
    return kind.__name__ == "_StopRecomputationError" and kind.__module__ == "torch.utils.checkpoint"
