"""Block placement and frozen-block streaming: drop-in for MOSS-Image's ``training/memory.py``.

``place_model(model, device, blocks_to_swap, *, block_swap_mode)`` (reference memory.py:486-532)
keeps the first ``len(model.layers) - blocks_to_swap`` joint blocks on the device and swaps the
rest:

- ``"sync"``: swapped blocks stay on the CPU; every invocation copies their parameters to the
  device inside a checkpoint (``offloaded_block``, reference :23-37).
- ``"async"``: the frozen parameters and buffers of each swapped block are packed into one
  pinned host *master*; LoRA adapters move to the device. An :class:`AsyncBlockStreamer` copies
  masters into two reusable device staging slots ahead of use (reference :93-361).
- ``"async_full"``: every parameter and buffer of the swapped blocks streams through a
  two-slot ring with write-back of updated blocks (``moss_offload.trainable_offload``, reference
  trainable_offload.py:89-477).

What is MI355X-specific: the masters of all swapped blocks live in one pinned host arena of
exactly the packed size (``mo_pinned_alloc``; the reference pins each block through torch's
caching host allocator, which rounds every pin up to a power of two), and slot fills run on an
SDMA engine through ``mo_streamer_*`` (no compute units, no interference with the step's GEMMs)
instead of ``copy_`` on a side stream. Ordering is the reference's: a fill starts once the GPU
has passed the slot's last release point, and the compute stream uses a slot only after its
fill completed (the host waits for it, bounded; no GPU queue waits on host memory).
"""

from __future__ import annotations

import ctypes
import threading
import weakref
from contextlib import nullcontext
from contextvars import ContextVar
from dataclasses import dataclass, field

import torch
from torch import nn
from torch.func import functional_call
from torch.utils.checkpoint import checkpoint

from . import _native

_ALIGN = 256


def _align(offset: int) -> int:
    return (offset + _ALIGN - 1) // _ALIGN * _ALIGN


# ---------------------------------------------------------------------------------------------
# synchronous swapping (reference memory.py:23-37)


def offloaded_block(layer: nn.Module, *args: torch.Tensor) -> torch.Tensor:
    """Run a CPU-resident block: its parameters and buffers are copied to the inputs' device on
    every invocation (inside a non-reentrant checkpoint when grad mode is on, so backward
    copies them again instead of keeping device copies alive)."""

    device = args[0].device
    names, parameters = zip(*layer.named_parameters())
    buffers = dict(layer.named_buffers())
    count = len(names)

    def run(*values: torch.Tensor) -> torch.Tensor:
        state = {name: value.to(device) for name, value in zip(names, values[:count])}
        state.update({name: buffer.to(device) for name, buffer in buffers.items()})
        return functional_call(layer, state, values[count:], strict=True)

    if torch.is_grad_enabled():
        return checkpoint(run, *parameters, *args, use_reentrant=False)
    return run(*parameters, *args)


# ---------------------------------------------------------------------------------------------
# pinned host arena for block masters


class PinnedArena:
    """One exact-size pinned host allocation, exposed as a CPU ``uint8`` tensor.

    Views of :attr:`tensor` keep the allocation alive; it is returned to the HIP runtime when
    the last view is gone.
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
class _TensorView:
    offset: int
    nbytes: int
    shape: torch.Size
    dtype: torch.dtype


@dataclass
class _BlockMaster:
    host: int  # address of the block's packed frozen tensors in pinned host memory
    nbytes: int
    views: dict[str, _TensorView]
    trainable: dict[str, nn.Parameter]
    arena: PinnedArena


def _typed(buffer: torch.Tensor, view: _TensorView) -> torch.Tensor:
    return buffer[view.offset : view.offset + view.nbytes].view(view.dtype).view(view.shape)


def _swap_storage(parameter: nn.Parameter, moved: torch.Tensor) -> None:
    replacement = nn.Parameter(moved, requires_grad=parameter.requires_grad)
    if parameter.grad is not None:
        replacement.grad = parameter.grad.detach().to(moved.device)
    torch.utils.swap_tensors(parameter, replacement)


def _frozen_tensors(layer: nn.Module) -> dict[str, torch.Tensor]:
    parameters = dict(layer.named_parameters())
    frozen = {name: p for name, p in parameters.items() if not p.requires_grad}
    frozen.update(dict(layer.named_buffers()))
    return frozen


def _layout(layer: nn.Module) -> tuple[dict[str, _TensorView], int]:
    views, offset = {}, 0
    for name, tensor in _frozen_tensors(layer).items():
        offset = _align(offset)
        nbytes = tensor.numel() * tensor.element_size()
        views[name] = _TensorView(offset, nbytes, tensor.shape, tensor.dtype)
        offset += nbytes
    return views, _align(offset)


def _place_async_layers(layers: dict[int, nn.Module], device: torch.device) -> dict[int, _BlockMaster]:
    """Pack the frozen tensors of ``layers`` into one pinned arena; adapters go to ``device``.

    Frozen parameters and buffers become CPU views of the arena (same names, shapes and dtypes),
    the way the reference turns them into views of each block's pinned buffer (memory.py:442-470).
    """

    layouts = {index: _layout(layer) for index, layer in layers.items()}
    starts, total = {}, 0
    for index, (_, nbytes) in layouts.items():
        starts[index] = total
        total += _align(nbytes)
    arena = PinnedArena(total)
    masters = {}
    for index, layer in layers.items():
        views, nbytes = layouts[index]
        block = arena.tensor[starts[index] : starts[index] + nbytes]
        parameters = dict(layer.named_parameters())
        trainable = {name: p for name, p in parameters.items() if p.requires_grad}
        for parameter in trainable.values():
            _swap_storage(parameter, parameter.detach().to(device))
        modules = dict(layer.named_modules())
        for name, source in _frozen_tensors(layer).items():
            packed = _typed(block, views[name])
            packed.copy_(source.detach().to("cpu").contiguous())
            if name in parameters:
                _swap_storage(parameters[name], packed)
            else:
                prefix, _, local = name.rpartition(".")
                modules[prefix]._buffers[local] = packed
        masters[index] = _BlockMaster(arena.address + starts[index], nbytes, views, trainable, arena)
    return masters


# ---------------------------------------------------------------------------------------------
# asynchronous frozen-block streaming (reference memory.py:93-361)


@dataclass
class _Slot:
    native: int
    index: int | None = None
    buffer: torch.Tensor | None = None
    tensors: dict[str, torch.Tensor] = field(default_factory=dict)
    leased: bool = False
    generation: int = 0


class _RecomputeScope:
    """Marks checkpoint recomputation (backward) so a block prefetches the previous block."""

    def __init__(self, flag: ContextVar) -> None:
        self._flag = flag
        self._tokens = ContextVar("moss_stream_recompute_tokens", default=())

    def __enter__(self) -> None:
        token = self._flag.set(True)
        self._tokens.set((*self._tokens.get(), token))

    def __exit__(self, *exc) -> bool:
        tokens = self._tokens.get()
        if not tokens:
            raise RuntimeError("Async block recompute context exited without being entered.")
        self._tokens.set(tokens[:-1])
        self._flag.reset(tokens[-1])
        return False


def _is_recompute_early_stop(error: BaseException) -> bool:
    # torch.utils.checkpoint stops a non-reentrant recomputation by raising this once the
    # tensors it needs exist.
    kind = type(error)
    return kind.__name__ == "_StopRecomputationError" and kind.__module__ == "torch.utils.checkpoint"


class AsyncBlockStreamer:
    """H2D-only streaming of frozen block masters through two reusable device staging slots.

    Trainable adapters are read from the module on every invocation, so an optimizer step can
    never leave a stale copy behind. Same interface as the reference's ``AsyncBlockStreamer``
    (``block``, ``owned_cuda_buffers``, ``resident_block_indices``, ``close``,
    ``peak_resident_blocks``, ``h2d_copy_count``).
    """

    SLOTS = 2

    def __init__(
        self,
        layers: nn.ModuleList,
        device: torch.device,
        first_streamed_block: int,
        blocks: dict[int, _BlockMaster],
        h2d_engine: int = 0,
    ) -> None:
        self.layers = layers
        self.device = torch.device(device)
        self.index = self.device.index if self.device.index is not None else torch.cuda.current_device()
        self.first_streamed_block = first_streamed_block
        self._blocks = blocks
        self._capacity = max(block.nbytes for block in blocks.values())
        self._lib = _native.load()
        handle = ctypes.c_void_p()
        _native.check(
            "mo_streamer_create",
            self._lib.mo_streamer_create(self.index, self.SLOTS, h2d_engine, ctypes.byref(handle)),
        )
        self._handle = handle
        self._lock = threading.RLock()
        self._slots = [_Slot(native=i) for i in range(self.SLOTS)]
        self._recomputing = ContextVar("moss_stream_recompute", default=False)
        self._recompute_scope = _RecomputeScope(self._recomputing)
        self.peak_resident_blocks = 0
        self.h2d_copy_count = 0
        self._closed = False

    # ------------------------------------------------------------------ introspection
    @property
    def resident_block_indices(self) -> tuple[int, ...]:
        return tuple(sorted(slot.index for slot in self._slots if slot.index is not None))

    @property
    def closed(self) -> bool:
        return self._closed

    def owned_cuda_buffers(self) -> tuple[torch.Tensor, ...]:
        """The staging buffers allocated so far (never allocates)."""

        return tuple(slot.buffer for slot in self._slots if slot.buffer is not None)

    def stats(self) -> dict:
        out = _native.MoStreamerStats()
        _native.check("mo_streamer_get_stats", self._lib.mo_streamer_get_stats(self._handle, ctypes.byref(out)))
        return out.as_dict()

    def reset_stats(self) -> None:
        _native.check("mo_streamer_reset_stats", self._lib.mo_streamer_reset_stats(self._handle))

    # ------------------------------------------------------------------ slots
    def _slot_of(self, index: int) -> _Slot | None:
        return next((slot for slot in self._slots if slot.index == index), None)

    def _pick(self, protected: frozenset[int]) -> _Slot:
        for slot in self._slots:
            if slot.index is None:
                return slot
        for slot in self._slots:
            if slot.index not in protected and not slot.leased:
                return slot
        raise RuntimeError("Async block streamer exhausted its two protected staging slots.")

    def _stage(self, index: int, protected: frozenset[int]) -> _Slot:
        slot = self._slot_of(index)
        if slot is not None:
            return slot
        slot = self._pick(protected)
        block = self._blocks[index]
        if slot.buffer is None:
            slot.buffer = torch.empty(self._capacity, dtype=torch.uint8, device=self.device)
        # The fill waits (on the SDMA issuer, not the host) for the slot's last release point.
        _native.check(
            "mo_streamer_fill",
            self._lib.mo_streamer_fill(self._handle, slot.native, slot.buffer.data_ptr(), block.host, block.nbytes),
        )
        self.h2d_copy_count += 1
        slot.index = index
        slot.tensors = {name: _typed(slot.buffer, view) for name, view in block.views.items()}
        slot.leased = False
        slot.generation += 1
        self.peak_resident_blocks = max(self.peak_resident_blocks, len(self.resident_block_indices))
        return slot

    def _release(self, slot: _Slot, stream) -> None:
        _native.check("mo_streamer_release", self._lib.mo_streamer_release(self._handle, slot.native, stream.cuda_stream))
        slot.leased = False

    def _release_after_backward(self, slot: _Slot, index: int, generation: int, tensors) -> object:
        """Keep the slot leased until every gradient of the block's inputs is computed."""

        differentiable = tuple(t for t in tensors if t.requires_grad)
        if not differentiable:
            raise RuntimeError("Async block checkpoint recomputation requires differentiable tensors.")
        box: list = []

        def done(_grads) -> None:
            try:
                if slot.index != index or slot.generation != generation:
                    raise RuntimeError("Async block staging slot changed before backward completed.")
                with self._lock:
                    self._release(slot, torch.cuda.current_stream(self.device))
            finally:
                box[0].remove()

        handle = torch.autograd.graph.register_multi_grad_hook(differentiable, done, mode="all")
        box.append(handle)
        return handle

    def _run(self, index, inputs, trainable, completion, forward_prefetch, backward_prefetch):
        if self._closed:
            raise RuntimeError("Async block streamer is closed.")
        recomputing = self._recomputing.get()
        prefetch = backward_prefetch if recomputing else forward_prefetch
        protected = frozenset(i for i in (index, prefetch) if i is not None)
        stream = torch.cuda.current_stream(self.device)
        with self._lock:
            slot = self._stage(index, protected)
            if slot.leased:
                raise RuntimeError(f"Async block {index} is already executing in another graph.")
            slot.leased = True
            generation = slot.generation
        backward_handle = None
        try:
            with self._lock:
                if prefetch is not None:
                    self._stage(prefetch, protected)
                _native.check(
                    "mo_streamer_acquire",
                    self._lib.mo_streamer_acquire(self._handle, slot.native, stream.cuda_stream),
                )
            values = dict(slot.tensors)
            values.update(trainable)
            if recomputing:
                # registered first: non-reentrant checkpointing may stop the recomputation as
                # soon as the tensors it needs exist
                backward_handle = self._release_after_backward(slot, index, generation, completion)
            output = functional_call(self.layers[index], values, inputs, strict=True)
        except BaseException as error:
            if not recomputing or not _is_recompute_early_stop(error):
                if backward_handle is not None:
                    backward_handle.remove()
                with self._lock:
                    self._release(slot, stream)
            raise
        if not recomputing:
            with self._lock:
                self._release(slot, stream)
        return output

    def _checkpoint_contexts(self):
        return nullcontext(), self._recompute_scope

    def block(self, index: int, *inputs: torch.Tensor, forward_prefetch: int | None,
              backward_prefetch: int | None, checkpoint_block: bool) -> torch.Tensor:
        """Run streamed block ``index``, prefetching the next block in traversal order."""

        if index not in self._blocks:
            raise ValueError(f"Block {index} is not configured for async streaming.")
        if not checkpoint_block:
            return self._run(index, inputs, self._blocks[index].trainable, (), forward_prefetch, backward_prefetch)
        count = len(inputs)
        names = tuple(self._blocks[index].trainable)
        # fresh aliases so the checkpoint sees distinct autograd inputs for every invocation
        input_aliases = tuple(t.view_as(t) if t.requires_grad else t for t in inputs)
        adapter_aliases = tuple(p.view_as(p) for p in self._blocks[index].trainable.values())

        def run(*arguments: torch.Tensor) -> torch.Tensor:
            adapters = dict(zip(names, arguments[count:]))
            completion = tuple(t for t in arguments if t.requires_grad)
            return self._run(index, arguments[:count], adapters, completion, forward_prefetch, backward_prefetch)

        return checkpoint(run, *input_aliases, *adapter_aliases, use_reentrant=False,
                          context_fn=self._checkpoint_contexts)

    def close(self) -> None:
        """Finish outstanding fills and release the staging slots."""

        if self._closed:
            return
        if any(slot.leased for slot in self._slots):
            raise RuntimeError("Cannot replace async block placement while a block backward is active.")
        torch.cuda.synchronize(self.device)
        _native.check("mo_streamer_destroy", self._lib.mo_streamer_destroy(self._handle))
        self._handle = ctypes.c_void_p()
        for slot in self._slots:
            slot.index = None
            slot.buffer = None
            slot.tensors.clear()
            slot.leased = False
            slot.generation += 1
        self._blocks.clear()
        self._closed = True


# ---------------------------------------------------------------------------------------------
# placement (reference memory.py:366-532)


def _is_lora(name: str) -> bool:
    return name.endswith("lora_A") or name.endswith("lora_B")


def _validate(model: nn.Module, device: torch.device, blocks_to_swap: int, mode: str) -> None:
    if mode not in {"sync", "async", "async_full"}:
        raise ValueError("block_swap_mode must be 'sync' or 'async'. Full training additionally accepts 'async_full'.")
    if not 0 <= blocks_to_swap <= len(model.layers):
        raise ValueError("blocks_to_swap must be between zero and the number of joint blocks.")
    if mode == "sync":
        return
    if device.type != "cuda":
        raise ValueError(f"{mode} block swapping requires a CUDA device.")
    boundary = len(model.layers) - blocks_to_swap
    if mode == "async_full":
        trainable = [p for p in model.parameters() if p.requires_grad]
        if not trainable:
            raise ValueError("async_full requires at least one trainable model parameter.")
        dtypes = {p.dtype for p in trainable}
        if len(dtypes) != 1 or not dtypes <= {torch.float32, torch.bfloat16}:
            raise ValueError("async_full requires homogeneous FP32 or BF16 trainable model parameters.")
        seen: dict[int, str] = {}
        for index, layer in enumerate(model.layers):
            if index < boundary:
                continue
            for name, parameter in layer.named_parameters():
                qualified = f"layers.{index}.{name}"
                if not parameter.is_floating_point():
                    raise TypeError(f"async_full cannot stream non-floating parameter {qualified}.")
                first = seen.setdefault(id(parameter), qualified)
                if first != qualified:
                    raise ValueError(
                        f"async_full does not support parameters shared across streamed blocks ({first} and {qualified})."
                    )
        return
    invalid = [
        f"layers.{index}.{name}"
        for index, layer in enumerate(model.layers)
        if index >= boundary
        for name, parameter in layer.named_parameters()
        if parameter.requires_grad and not _is_lora(name)
    ]
    if invalid:
        raise ValueError(
            "async block swapping is H2D-only and requires frozen base weights; "
            f"only LoRA adapters may be trainable (found {invalid[0]})."
        )


def place_model(model: nn.Module, device: torch.device, blocks_to_swap: int, *, block_swap_mode: str = "sync",
                h2d_engine: int = 0) -> None:
    """Place a model for resident, synchronously swapped or frozen-async execution."""

    device = torch.device(device)
    _validate(model, device, blocks_to_swap, block_swap_mode)
    previous = getattr(model, "block_swap_manager", None)
    if previous is not None:
        previous.close()
    model.blocks_to_swap = blocks_to_swap
    model.block_swap_mode = block_swap_mode
    model.block_swap_manager = None
    for name, child in model.named_children():
        if name != "layers":
            child.to(device)
    boundary = len(model.layers) - blocks_to_swap
    if block_swap_mode == "sync":
        for index, layer in enumerate(model.layers):
            layer.to("cpu" if index >= boundary else device)
        return
    if block_swap_mode == "async_full":
        from .trainable_offload import TrainableBlockStreamer

        for layer in model.layers[:boundary]:
            layer.to(device)
        if blocks_to_swap:
            model.block_swap_manager = TrainableBlockStreamer(model.layers, device, boundary, master_dtype=None,
                                                              h2d_engine=h2d_engine)
        return
    swapped = {}
    for index, layer in enumerate(model.layers):
        if index < boundary:
            layer.to(device)
        else:
            swapped[index] = layer
    if swapped:
        masters = _place_async_layers(swapped, device)
        model.block_swap_manager = AsyncBlockStreamer(model.layers, device, boundary, masters, h2d_engine)
