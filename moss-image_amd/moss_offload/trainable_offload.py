"""Streaming of blocks that train in place: drop-in for ``training/trainable_offload.py``.

``TrainableBlockStreamer`` keeps every parameter and buffer of ``layers[first_streamed_block:]``
in a pinned host *master* (one exact-size arena for all blocks) and runs each block from one of
two device slots of a :class:`~moss_offload.ring.BlockRing`. The ``Parameter`` objects stay the
same; what changes is the storage they point at: the slot while the block is resident, the
master otherwise. A fused optimizer updates a block's parameters in place during its backward
(post-accumulate-grad hooks) and reports each update through :meth:`mark_updated`; the block's
slot is then *dirty*, and the native ring copies it back to the master (SDMA, after the slot's
release point) before the slot takes another block.

Settling a block. In backward a block's recomputation leaves its slot pinned: its gradient
kernels and then the optimizer hooks of its parameters are still to be enqueued. Nothing marks
the moment those are done, but two later events bound it: the next streamed block starting to
run (in a backward traversal it is the block before, whose gradients need this block's), and
:meth:`finish_backward` / :meth:`commit`, which the training loop calls after ``backward()``
returns. At either one the block is *settled*: its updates are checked against the parameters it
owns, the ring learns whether it is dirty, and the pin is dropped on the compute stream.

Contract (as in the reference, trainable_offload.py:89-477): one process per GPU,
non-reentrant checkpointing, one backward graph at a time through the streamed blocks; call
:meth:`finish_backward` after each backward and :meth:`commit` before evaluation, state export
or loading weights (``close`` commits).
"""

from __future__ import annotations

from contextlib import nullcontext
from dataclasses import dataclass, field

import torch
from torch import nn
from torch.utils.checkpoint import checkpoint

from .ring import BlockRing, Lease, Master, PinnedArena, Placement, RecomputePhase, align, plan, stopped_recomputation

__all__ = ["TrainableBlockStreamer"]


@dataclass
class _Member:
    """One tensor of a streamed block: a parameter, or a buffer of ``module``."""

    module: nn.Module
    attribute: str
    parameter: nn.Parameter | None
    place: Placement


@dataclass
class _Streamed:
    index: int
    master: Master
    members: list[_Member]
    owned: frozenset[int] = field(default_factory=frozenset)  # ids of its trainable parameters

    def point_at(self, flat: torch.Tensor) -> None:
        """Every member becomes a view of ``flat`` (the master or a slot)."""

        for member in self.members:
            view = member.place.view(flat)
            if member.parameter is not None:
                member.parameter.data = view
            else:
                member.module._buffers[member.attribute] = view


@dataclass
class _Ledger:
    """The optimizer protocol's state across one backward."""

    stepping: bool = True  # this backward is an optimizer-update boundary
    require_all: bool = True  # a settled block must have every trainable parameter updated
    updated: set[int] = field(default_factory=set)
    failed: dict[int, str] = field(default_factory=dict)
    broken: bool = False  # a block was settled without its updates: reload the checkpoint

    def clear(self) -> None:
        self.updated.clear()
        self.failed.clear()


def _collect(layer: nn.Module) -> list[tuple[nn.Module, str, nn.Parameter | None, torch.Tensor]]:
    found, seen = [], set()
    for module in layer.modules():
        for name, parameter in module._parameters.items():
            if parameter is not None and id(parameter) not in seen:
                seen.add(id(parameter))
                found.append((module, name, parameter, parameter.detach()))
        for name, buffer in module._buffers.items():
            if buffer is not None and id(buffer) not in seen:
                seen.add(id(buffer))
                found.append((module, name, None, buffer.detach()))
    return found


class TrainableBlockStreamer:
    """Two device slots for checkpointed blocks whose parameters a fused optimizer updates."""

    def __init__(self, layers: nn.ModuleList, device: torch.device | str, first_streamed_block: int = 0, *,
                 master_dtype: torch.dtype | None = None, ring_size: int = 2, h2d_engine: int = 0) -> None:
        device = torch.device(device)
        if device.type != "cuda":
            raise ValueError(f"Trainable block streaming requires a CUDA device, got {device}")
        if ring_size != 2:
            raise ValueError(f"the trainable ring has two slots (ring_size=2), got {ring_size}")
        if not 0 <= first_streamed_block < len(layers):
            raise ValueError(f"first_streamed_block must leave at least one of {len(layers)} layers to stream")
        if master_dtype not in (None, torch.float32, torch.bfloat16):
            raise TypeError(f"master_dtype must be None, torch.float32 or torch.bfloat16, got {master_dtype}")
        self.layers = layers
        self.device = device
        self.first_streamed_block = first_streamed_block
        self.master_dtype = master_dtype
        self._names: dict[int, str] = {}  # parameter id -> "layers.<i>.<name>"
        self._blocks = self._pack(range(first_streamed_block, len(layers)))
        self._ring = BlockRing(device, 2, max(b.master.nbytes for b in self._blocks.values()), h2d_engine)
        self._occupant: list[int | None] = [None, None]  # block bound to each slot
        self._phase = RecomputePhase()
        self._ledger = _Ledger()
        self._unsettled: Lease | None = None  # a block whose backward may still be enqueuing
        self.peak_resident_blocks = 0
        self._closed = False

    # ------------------------------------------------------------------ masters
    def _pack(self, indices) -> dict[int, _Streamed]:
        owners: dict[int, int] = {}
        staged = []
        for index in indices:
            entries = _collect(self.layers[index])
            converted = []
            for module, name, parameter, tensor in entries:
                if parameter is not None:
                    if owners.setdefault(id(parameter), index) != index:
                        raise ValueError(
                            f"Trainable block streaming cannot stream a parameter shared by blocks "
                            f"{owners[id(parameter)]} and {index}"
                        )
                    if not parameter.is_floating_point():
                        raise TypeError(f"streamed parameter layers.{index}.{name} must be floating point")
                dtype = self.master_dtype if parameter is not None and self.master_dtype is not None else tensor.dtype
                converted.append(tensor.to(device="cpu", dtype=dtype).contiguous())
            places, nbytes = plan(converted)
            staged.append((index, entries, converted, places, nbytes))
        arena = PinnedArena(sum(align(s[4]) for s in staged))
        blocks, start = {}, 0
        for index, entries, converted, places, nbytes in staged:
            flat = arena.tensor[start : start + nbytes]
            members = []
            for (module, name, parameter, _), source, place in zip(entries, converted, places):
                place.view(flat).copy_(source)
                members.append(_Member(module, name, parameter, place))
            owned = frozenset(id(m.parameter) for m in members if m.parameter is not None and m.parameter.requires_grad)
            for member in members:
                if member.parameter is not None:
                    self._names[id(member.parameter)] = f"layers.{index}.{member.attribute}"
            block = _Streamed(index, Master(arena.address + start, nbytes, flat), members, owned)
            block.point_at(flat)
            blocks[index] = block
            start += align(nbytes)
        return blocks

    # ------------------------------------------------------------------ introspection
    @property
    def closed(self) -> bool:
        return self._closed

    @property
    def requires_reload(self) -> bool:
        return self._ledger.broken

    @property
    def resident_block_indices(self) -> tuple[int, ...]:
        return () if self._closed else self._ring.resident()

    @property
    def h2d_copy_count(self) -> int:
        return self._ring.fills

    @property
    def d2h_copy_count(self) -> int:
        return 0 if self._closed else int(self._ring.stats()["writebacks"])

    def owned_cuda_buffers(self) -> tuple[torch.Tensor, ...]:
        return tuple(b for b in self._ring.buffers if b is not None)

    def stats(self) -> dict:
        return self._ring.stats()

    def reset_stats(self) -> None:
        self._ring.reset_stats()

    # ------------------------------------------------------------------ optimizer protocol
    def set_step_enabled(self, enabled: bool) -> None:
        """Whether the coming backward updates parameters (False: an accumulation backward)."""

        if self._unsettled is not None:
            raise RuntimeError("the optimizer-step boundary cannot change while a block's backward is pending")
        if self._ledger.broken:
            raise RuntimeError("the trainable block streamer requires checkpoint reload after a failed update")
        self._ledger.stepping = bool(enabled)
        self._ledger.clear()

    def set_require_all_updates(self, required: bool) -> None:
        if self._unsettled is not None:
            raise RuntimeError("update requirements cannot change while a block's backward is pending")
        self._ledger.require_all = bool(required)

    def mark_updated(self, parameter: nn.Parameter) -> None:
        """A fused optimizer hook finished updating ``parameter`` in place."""

        if self._ledger.stepping and id(parameter) in self._names:
            self._ledger.updated.add(id(parameter))

    def mark_failed(self, parameter: nn.Parameter) -> None:
        """A fused optimizer hook failed for ``parameter``: its block must not be written back."""

        if self._ledger.stepping and id(parameter) in self._names:
            self._ledger.failed[id(parameter)] = self._names[id(parameter)]

    def mark_reloaded(self) -> None:
        if self._unsettled is not None or self.resident_block_indices:
            raise RuntimeError("commit the trainable block streamer before marking it reloaded")
        self._ledger.broken = False
        self._ledger.clear()

    def _settle(self) -> None:
        """The unsettled block's backward and optimizer hooks are all enqueued: check its updates,
        tell the ring whether to write it back, and let the slot go at this stream position."""

        lease, self._unsettled = self._unsettled, None
        if lease is None:
            return
        ring, ledger = self._ring, self._ledger
        ring.unpin(lease)
        owned = self._blocks[lease.block].owned
        if not ledger.stepping:
            ring.mark_dirty(lease, False)
            return
        problem = None
        failed = sorted(ledger.failed[p] for p in owned & ledger.failed.keys())
        missing = sorted(self._names[p] for p in owned - ledger.updated)
        if failed:
            problem = f"the fused optimizer update failed for {failed[:3]}"
        elif missing and ledger.require_all:
            problem = f"its backward finished before all parameter updates; missing {missing[:3]}"
        if problem is not None:
            ring.mark_dirty(lease, False)  # the master keeps the weights from before the step
            ledger.broken = True
            raise RuntimeError(f"trainable block {lease.block}: {problem}")
        ring.mark_dirty(lease, bool(owned & ledger.updated))

    # ------------------------------------------------------------------ execution
    def _make_resident(self, index: int, keep: int | None) -> Lease:
        lease = self._ring.stage(index, self._blocks[index].master, keep=keep)
        if lease.filled or self._occupant[lease.slot] != index:
            previous = self._occupant[lease.slot]
            if previous is not None and previous != index:
                # the ring wrote it back (if dirty) before the fill: its parameters are the master again
                self._blocks[previous].point_at(self._blocks[previous].master.tensor)
            self._occupant[lease.slot] = index
            self._blocks[index].point_at(self._ring.buffers[lease.slot][: self._blocks[index].master.nbytes])
        return lease

    def _execute(self, index: int, inputs, neighbours) -> torch.Tensor:
        if self._closed:
            raise RuntimeError("the trainable block streamer has been closed")
        in_backward = self._phase.active
        beside = neighbours[1] if in_backward else neighbours[0]
        if beside is not None and beside not in self._blocks:
            raise ValueError(f"Prefetch block {beside} is not streamed.")
        ring = self._ring
        with ring.lock:
            # a block starting means the unsettled one is done enqueuing (in backward: its
            # gradients fed this one; in a forward: the backward call has returned)
            self._settle()
            lease = self._make_resident(index, beside)
            ring.pin(lease)
            try:
                if beside is not None:
                    self._make_resident(beside, index)
                ring.ready(lease)
            except BaseException:
                ring.unpin(lease)
                raise
            self.peak_resident_blocks = max(self.peak_resident_blocks, len(ring.resident()))
        try:
            output = self.layers[index](*inputs)
        except BaseException as error:
            with ring.lock:
                if in_backward and stopped_recomputation(error):
                    self._unsettled = lease
                else:
                    ring.unpin(lease)
            raise
        with ring.lock:
            if in_backward:
                self._unsettled = lease
            else:
                ring.unpin(lease)
        return output

    def block(self, index: int, *inputs: torch.Tensor, forward_prefetch: int | None,
              backward_prefetch: int | None, checkpoint_block: bool) -> torch.Tensor:
        """Run streamed block ``index`` (the block-manager contract of the reference model)."""

        if index not in self._blocks:
            raise ValueError(f"Block {index} is not configured for trainable streaming.")
        neighbours = (forward_prefetch, backward_prefetch)
        if not checkpoint_block:
            return self._execute(index, inputs, neighbours)
        fresh = tuple(t.view_as(t) if isinstance(t, torch.Tensor) and t.requires_grad else t for t in inputs)
        return checkpoint(lambda *flat: self._execute(index, flat, neighbours), *fresh, use_reentrant=False,
                          context_fn=lambda: (nullcontext(),
                                              self._phase.recomputing()))

    # ------------------------------------------------------------------ boundaries
    def finish_backward(self) -> None:
        """After ``backward()`` returned: settle the last block and write dirty blocks back."""

        if self._closed:
            raise RuntimeError("the trainable block streamer has been closed")
        self.commit()

    def commit(self) -> None:
        """Settle, write every dirty slot back, and point every streamed parameter at its master."""

        if self._closed:
            return
        ring = self._ring
        with ring.lock:
            try:
                self._settle()
            finally:
                for slot, occupant in enumerate(self._occupant):
                    ring.evict(slot)
                    if occupant is not None:
                        self._blocks[occupant].point_at(self._blocks[occupant].master.tensor)
                    self._occupant[slot] = None
                torch.cuda.synchronize(self.device)
                ring.synchronize()
                self._ledger.clear()

    drain = commit

    def close(self) -> None:
        """Commit the authoritative weights and free the slots."""

        if self._closed:
            return
        try:
            self.commit()
        finally:
            self._ring.close()
            self._closed = True
