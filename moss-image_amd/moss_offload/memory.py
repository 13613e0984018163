"""Where the joint blocks live, and how swapped blocks run: drop-in for ``training/memory.py``.

``place_model(model, device, blocks_to_swap, *, block_swap_mode)`` (the reference's entry point,
memory.py:486-532) keeps ``len(model.layers) - blocks_to_swap`` blocks on the device and swaps
the rest in one of three ways:

``"sync"``
    the swapped blocks stay on the CPU; :func:`offloaded_block` copies a block's tensors to the
    device for every run (inside a checkpoint, so backward copies them again).
``"async"``
    frozen parameters and buffers of the swapped blocks are packed, block after block, into one
    pinned host arena; LoRA adapters move to the device. :class:`AsyncBlockStreamer` runs each
    block from one of two device slots of a :class:`~moss_offload.ring.BlockRing`, filled by an
    SDMA engine ahead of use.
``"async_full"``
    every tensor of the swapped blocks streams, and blocks a fused optimizer updated are written
    back (:mod:`moss_offload.trainable_offload`).

The native ring owns residency (which block each slot holds, pins, fill generations, the slot a
new block replaces); this module maps a block's frozen tensors onto a slot's bytes and ties slot
pins to the autograd graph: a forward run pins its slot while it enqueues kernels, a
recomputation in backward keeps its slot pinned until the gradients of the block's inputs exist.
"""

from __future__ import annotations

from contextlib import nullcontext
from dataclasses import dataclass

import torch
from torch import nn
from torch.func import functional_call
from torch.utils.checkpoint import checkpoint

from .ring import BlockRing, Lease, Master, PinnedArena, Placement, RecomputePhase, align, plan, stopped_recomputation

__all__ = ["AsyncBlockStreamer", "offloaded_block", "place_model", "PinnedArena"]


# ---------------------------------------------------------------------------------------------
# synchronous swapping (reference memory.py:23-37)


def offloaded_block(layer: nn.Module, *args: torch.Tensor) -> torch.Tensor:
    """Run ``layer``, whose tensors live on the CPU, on the device of ``args[0]``.

    Parameters and buffers are copied to the device inside the call, so the device copies are
    temporaries. With grad enabled the call runs under a non-reentrant checkpoint: backward
    copies them again instead of holding them from forward to backward.
    """

    target = args[0].device
    parameter_items = list(layer.named_parameters())
    buffer_items = list(layer.named_buffers())
    split = len(parameter_items)

    def on_device(*flat: torch.Tensor) -> torch.Tensor:
        state = {name: value.to(target) for (name, _), value in zip(parameter_items, flat[:split])}
        for name, buffer in buffer_items:
            state[name] = buffer.to(target)
        return functional_call(layer, state, flat[split:], strict=True)

    flat = (*(p for _, p in parameter_items), *args)
    return checkpoint(on_device, *flat, use_reentrant=False) if torch.is_grad_enabled() else on_device(*flat)


# ---------------------------------------------------------------------------------------------
# frozen blocks in pinned memory


@dataclass
class FrozenBlock:
    """One swapped block: its frozen tensors packed in ``master``, its adapters on the device."""

    master: Master
    places: dict[str, Placement]  # frozen parameter or buffer name -> bytes in the master
    adapters: dict[str, nn.Parameter]  # trainable parameters (LoRA), read at every run


def _move_parameter(parameter: nn.Parameter, data: torch.Tensor) -> None:
    # the Parameter object survives (optimizers and hooks hold it); only its tensor changes
    moved = nn.Parameter(data, requires_grad=parameter.requires_grad)
    if parameter.grad is not None:
        moved.grad = parameter.grad.detach().to(data.device)
    torch.utils.swap_tensors(parameter, moved)


def pack_frozen_blocks(layers: dict[int, nn.Module], device: torch.device) -> dict[int, FrozenBlock]:
    """Pack the frozen tensors of ``layers`` into one pinned arena; adapters move to ``device``.

    Afterwards every frozen parameter and buffer of those layers is a CPU view of the arena
    (same name, shape and dtype), which is where the slots are filled from.
    """

    layouts = {}
    for index, layer in layers.items():
        frozen = {n: p for n, p in layer.named_parameters() if not p.requires_grad}
        frozen.update(layer.named_buffers())
        places, nbytes = plan(frozen.values())
        layouts[index] = (frozen, dict(zip(frozen, places)), nbytes)
    offsets, total = {}, 0
    for index, (_, _, nbytes) in layouts.items():
        offsets[index] = total
        total += align(nbytes)
    arena = PinnedArena(total)
    blocks = {}
    for index, layer in layers.items():
        frozen, places, nbytes = layouts[index]
        start = offsets[index]
        packed = arena.tensor[start : start + nbytes]
        parameters = dict(layer.named_parameters())
        modules = dict(layer.named_modules())
        for name, source in frozen.items():
            target = places[name].view(packed)
            target.copy_(source.detach().to("cpu").contiguous())
            if name in parameters:
                _move_parameter(parameters[name], target)
            else:
                owner, _, local = name.rpartition(".")
                modules[owner]._buffers[local] = target
        adapters = {n: p for n, p in parameters.items() if p.requires_grad}
        for parameter in adapters.values():
            _move_parameter(parameter, parameter.detach().to(device))
        blocks[index] = FrozenBlock(Master(arena.address + start, nbytes, packed), places, adapters)
    return blocks


# ---------------------------------------------------------------------------------------------
# asynchronous frozen-block streaming (reference memory.py:93-361)


class AsyncBlockStreamer:
    """Runs swapped frozen blocks from two device slots, filled over SDMA ahead of use.

    The block-manager contract of the reference model (``model._run_layers`` calls
    :meth:`block`; the activation-offload hook asks :meth:`owned_cuda_buffers`), with the
    reference's introspection (``resident_block_indices``, ``peak_resident_blocks``,
    ``h2d_copy_count``, ``closed``). Adapters are read from the module at every run, so an
    optimizer step is never shadowed by a stale copy.
    """

    SLOTS = 2

    def __init__(self, layers: nn.ModuleList, device: torch.device, first_streamed_block: int,
                 blocks: dict[int, FrozenBlock], h2d_engine: int = 0) -> None:
        self.layers = layers
        self.device = torch.device(device)
        self.first_streamed_block = first_streamed_block
        self._blocks = blocks
        self._ring = BlockRing(self.device, self.SLOTS, max(b.master.nbytes for b in blocks.values()), h2d_engine)
        self._phase = RecomputePhase()
        self._slot_views: dict[int, tuple[int, dict[str, torch.Tensor]]] = {}  # slot -> (generation, views)
        self.peak_resident_blocks = 0
        self._closed = False

    # ------------------------------------------------------------------ introspection
    @property
    def closed(self) -> bool:
        return self._closed

    @property
    def resident_block_indices(self) -> tuple[int, ...]:
        return () if self._closed else self._ring.resident()

    @property
    def h2d_copy_count(self) -> int:
        return self._ring.fills

    def owned_cuda_buffers(self) -> tuple[torch.Tensor, ...]:
        """The device slot buffers (weight storage: never offloaded as activations)."""

        return tuple(b for b in self._ring.buffers if b is not None)

    def stats(self) -> dict:
        return self._ring.stats()

    def reset_stats(self) -> None:
        self._ring.reset_stats()

    # ------------------------------------------------------------------ execution
    def block(self, index: int, *inputs: torch.Tensor, forward_prefetch: int | None,
              backward_prefetch: int | None, checkpoint_block: bool) -> torch.Tensor:
        """Run streamed block ``index``; the block after it in traversal order is staged beside
        it (``forward_prefetch`` in the forward, ``backward_prefetch`` in recomputation)."""

        frozen = self._blocks.get(index)
        if frozen is None:
            raise ValueError(f"Block {index} is not configured for async streaming.")
        neighbours = (forward_prefetch, backward_prefetch)
        if not checkpoint_block:
            return self._execute(index, inputs, frozen.adapters, (), neighbours)
        names = tuple(frozen.adapters)
        count = len(inputs)

        def body(*flat: torch.Tensor) -> torch.Tensor:
            needs_grad = tuple(t for t in flat if isinstance(t, torch.Tensor) and t.requires_grad)
            return self._execute(index, flat[:count], dict(zip(names, flat[count:])), needs_grad, neighbours)

        # fresh views as the checkpoint's inputs: two runs of one block in one graph stay apart
        # (inputs that are not tensors, such as packed sequence lengths, pass as they are)
        flat = tuple(t.view_as(t) if isinstance(t, torch.Tensor) and t.requires_grad else t for t in inputs)
        flat += tuple(p.view_as(p) for p in frozen.adapters.values())
        return checkpoint(body, *flat, use_reentrant=False,
                          context_fn=lambda: (nullcontext(), self._phase.recomputing()))

    def _views(self, lease: Lease) -> dict[str, torch.Tensor]:
        cached = self._slot_views.get(lease.slot)
        if cached is None or cached[0] != lease.generation:
            buffer = self._ring.buffers[lease.slot]
            places = self._blocks[lease.block].places
            cached = (lease.generation, {name: place.view(buffer) for name, place in places.items()})
            self._slot_views[lease.slot] = cached
        return cached[1]

    def _execute(self, index, inputs, adapters, needs_grad, neighbours) -> torch.Tensor:
        if self._closed:
            raise RuntimeError("the async block streamer has been closed")
        in_backward = self._phase.active
        beside = neighbours[1] if in_backward else neighbours[0]
        ring = self._ring
        with ring.lock:
            lease = ring.stage(index, self._blocks[index].master, keep=beside)
            ring.pin(lease)
            try:
                if beside is not None:
                    ring.stage(beside, self._blocks[beside].master, keep=index)
                ring.ready(lease)
            except BaseException:
                ring.unpin(lease)
                raise
            self.peak_resident_blocks = max(self.peak_resident_blocks, len(ring.resident()))
        state = dict(self._views(lease))
        state.update(adapters)
        # In backward the kernels that read the slot are the recomputation and the block's
        # gradient kernels after it; the pin is dropped once the gradients of every input exist.
        # Registered before running: the checkpoint may end the recomputation early.
        grad_watch = self._unpin_after_gradients(lease, needs_grad) if in_backward else None
        try:
            output = functional_call(self.layers[index], state, inputs, strict=True)
        except BaseException as error:
            if in_backward and stopped_recomputation(error):
                raise
            if grad_watch is not None:
                grad_watch.remove()
            with ring.lock:
                ring.unpin(lease)
            raise
        if not in_backward:
            with ring.lock:
                ring.unpin(lease)
        return output

    def _unpin_after_gradients(self, lease: Lease, needs_grad: tuple[torch.Tensor, ...]):
        if not needs_grad:
            raise RuntimeError("recomputing a streamed block needs at least one input that requires grad")
        ring = self._ring
        watch = []

        def gradients_ready(_grads) -> None:
            watch[0].remove()
            with ring.lock:
                ring.unpin(lease)  # fails loudly if the slot took another block meanwhile

        watch.append(torch.autograd.graph.register_multi_grad_hook(needs_grad, gradients_ready, mode="all"))
        return watch[0]

    def close(self) -> None:
        """Wait for every copy, free the slots and forget the blocks."""

        if self._closed:
            return
        if any(self._ring.info(slot)[1] for slot in range(self.SLOTS)):
            raise RuntimeError("cannot close the async block streamer: a streamed block's backward is still pending")
        torch.cuda.synchronize(self.device)
        self._ring.close()
        self._slot_views.clear()
        self._blocks.clear()
        self._closed = True


# ---------------------------------------------------------------------------------------------
# placement (reference memory.py:366-532)


def _check_placement(model: nn.Module, device: torch.device, blocks_to_swap: int, mode: str) -> None:
    """Every reason to refuse a placement, checked before anything moves."""

    if mode not in ("sync", "async", "async_full"):
        raise ValueError(f"block_swap_mode must be 'sync' or 'async' (or 'async_full' for full training), got {mode!r}")
    depth = len(model.layers)
    if not 0 <= blocks_to_swap <= depth:
        raise ValueError(f"blocks_to_swap must be between 0 and {depth} (the joint blocks), got {blocks_to_swap}")
    if mode == "sync":
        return
    if device.type != "cuda":
        raise ValueError(f"{mode} block swapping requires a CUDA device, got {device}")
    swapped = list(enumerate(model.layers))[depth - blocks_to_swap:]
    if mode == "async":
        for index, layer in swapped:
            for name, parameter in layer.named_parameters():
                if parameter.requires_grad and not name.endswith(("lora_A", "lora_B")):
                    raise ValueError(
                        f"async block swapping is H2D-only and streams frozen base weights; layers.{index}.{name} "
                        "is trainable and only LoRA adapters may be (use async_full for full training)"
                    )
        return
    trainable = [p for p in model.parameters() if p.requires_grad]
    if not trainable:
        raise ValueError("async_full requires at least one trainable parameter in the model")
    if len({p.dtype for p in trainable}) != 1 or trainable[0].dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("async_full requires all trainable parameters in one dtype, float32 or bfloat16")
    owner: dict[int, str] = {}
    for index, layer in swapped:
        for name, parameter in layer.named_parameters():
            where = f"layers.{index}.{name}"
            if not parameter.is_floating_point():
                raise TypeError(f"async_full streams floating tensors only: non-floating parameter {where}")
            first = owner.setdefault(id(parameter), where)
            if first != where:
                raise ValueError(f"async_full cannot stream a parameter shared across streamed blocks ({first}, {where})")


def place_model(model: nn.Module, device: torch.device, blocks_to_swap: int, *, block_swap_mode: str = "sync",
                h2d_engine: int = 0) -> None:
    """Place ``model``: resident blocks on ``device``, the last ``blocks_to_swap`` swapped."""

    device = torch.device(device)
    _check_placement(model, device, blocks_to_swap, block_swap_mode)
    old = getattr(model, "block_swap_manager", None)
    if old is not None:
        old.close()
    model.blocks_to_swap = blocks_to_swap
    model.block_swap_mode = block_swap_mode
    model.block_swap_manager = None
    for name, child in model.named_children():
        if name != "layers":
            child.to(device)
    boundary = len(model.layers) - blocks_to_swap
    resident, swapped = model.layers[:boundary], dict(list(enumerate(model.layers))[boundary:])
    for layer in resident:
        layer.to(device)
    if block_swap_mode == "sync":
        for layer in swapped.values():
            layer.to("cpu")
    elif swapped and block_swap_mode == "async":
        blocks = pack_frozen_blocks(swapped, device)
        model.block_swap_manager = AsyncBlockStreamer(model.layers, device, boundary, blocks, h2d_engine)
    elif swapped:
        from .trainable_offload import TrainableBlockStreamer

        model.block_swap_manager = TrainableBlockStreamer(model.layers, device, boundary, master_dtype=None,
                                                          h2d_engine=h2d_engine)
