"""Bidirectional block streaming for full-parameter training: drop-in for MOSS-Image's
``training/trainable_offload.py`` (``TrainableBlockStreamer``, :89-477).

Every parameter and buffer of ``layers[first_streamed_block:]`` is packed into a pinned host
*master* (one exact-size arena for all blocks, ``mo_pinned_alloc``). The existing
``Parameter`` objects stay; their ``.data`` is rebound between the master and one of two
device staging slots. The forward traversal prefetches upward, checkpoint recomputation
downward. A fused optimizer updates a block's parameters in place during its backward
(post-accumulate-grad hooks) and reports each update with :meth:`mark_updated`. The block's
slot is then *dirty* and is written back to its master before the slot is refilled.

MI355X specifics: fills (H2D) and write-backs (D2H) run on the SDMA engines through the same
``mo_streamer_*`` C-ABI as the frozen streamer. A write-back starts once the GPU passed the
slot's release point (recorded when the next block's backward begins, after the optimizer
hooks of this block). The slot's next fill waits for the write-back, and the compute stream uses a
slot only after its fill completed (host-side wait, bounded). No GPU queue waits on host memory.

Contract (as in the reference): one process per GPU, non-reentrant checkpointing, sequential
forward/backward shape groups. Call :meth:`finish_backward` after every backward and
:meth:`commit` before evaluation, state export or model load (``close`` commits).
"""

from __future__ import annotations

import ctypes
import threading
from contextlib import nullcontext
from contextvars import ContextVar
from dataclasses import dataclass, field

import torch
from torch import nn
from torch.utils.checkpoint import checkpoint

from . import _native
from .memory import PinnedArena, _align


@dataclass(frozen=True)
class _View:
    offset: int
    nbytes: int
    shape: torch.Size
    dtype: torch.dtype


@dataclass
class _Binding:
    module: nn.Module
    local_name: str
    parameter: nn.Parameter | None
    view: _View


@dataclass
class _Block:
    index: int
    host: int  # master address in pinned host memory
    master: torch.Tensor  # CPU uint8 view of the master
    nbytes: int
    bindings: list[_Binding]


@dataclass
class _Slot:
    native: int
    buffer: torch.Tensor
    index: int | None = None
    dirty: bool = False
    views: list[torch.Tensor] = field(default_factory=list)


def _typed(buffer: torch.Tensor, view: _View) -> torch.Tensor:
    return buffer[view.offset : view.offset + view.nbytes].view(view.dtype).view(view.shape)


class _RecomputeScope:
    def __init__(self, flag: ContextVar) -> None:
        self._flag = flag
        self._tokens = ContextVar("moss_trainable_recompute_tokens", default=())

    def __enter__(self) -> None:
        token = self._flag.set(True)
        self._tokens.set((*self._tokens.get(), token))

    def __exit__(self, *exc) -> bool:
        tokens = self._tokens.get()
        if not tokens:
            raise RuntimeError("Trainable block recompute context exited without entry.")
        self._tokens.set(tokens[:-1])
        self._flag.reset(tokens[-1])
        return False


def _is_recompute_early_stop(error: BaseException) -> bool:
    kind = type(error)
    return kind.__name__ == "_StopRecomputationError" and kind.__module__ == "torch.utils.checkpoint"


class TrainableBlockStreamer:
    """Two-slot H2D/D2H ring for checkpointed full-parameter blocks."""

    def __init__(self, layers: nn.ModuleList, device: torch.device | str, first_streamed_block: int = 0, *,
                 master_dtype: torch.dtype | None = None, ring_size: int = 2, h2d_engine: int = 0) -> None:
        device = torch.device(device)
        if device.type != "cuda":
            raise ValueError("Trainable block streaming requires a CUDA device.")
        if ring_size != 2:
            raise ValueError("Trainable block streaming uses exactly two staging slots.")
        if not 0 <= first_streamed_block < len(layers):
            raise ValueError("first_streamed_block must select at least one layer.")
        if master_dtype not in {None, torch.float32, torch.bfloat16}:
            raise TypeError("master_dtype must be torch.float32 or torch.bfloat16.")
        self.layers = layers
        self.device = device
        self.first_streamed_block = first_streamed_block
        self.master_dtype = master_dtype
        self._recomputing = ContextVar("moss_trainable_recompute", default=False)
        self._recompute_scope = _RecomputeScope(self._recomputing)
        self._lock = threading.RLock()
        self._blocks: dict[int, _Block] = {}
        self._parameter_block: dict[int, int] = {}
        self._parameter_name: dict[int, str] = {}
        self._expected_updates: dict[int, set[int]] = {}
        self._updated: set[int] = set()
        self._failed: dict[int, str] = {}
        self._step_enabled = True
        self._require_all_updates = True
        self._requires_reload = False
        self._last_backward_index: int | None = None
        self._closed = False
        self.h2d_copy_count = 0
        self.d2h_copy_count = 0
        self.peak_resident_blocks = 0

        self._pack(range(first_streamed_block, len(layers)))
        capacity = max(block.nbytes for block in self._blocks.values())
        self._lib = _native.load()
        index = device.index if device.index is not None else torch.cuda.current_device()
        handle = ctypes.c_void_p()
        _native.check("mo_streamer_create", self._lib.mo_streamer_create(index, 2, h2d_engine, ctypes.byref(handle)))
        self._handle = handle
        self._slots = [_Slot(i, torch.empty(capacity, dtype=torch.uint8, device=device)) for i in range(2)]

    # ------------------------------------------------------------------ packing
    def _pack(self, indices) -> None:
        """Pack every block's parameters and buffers into one pinned arena (CPU masters)."""

        seen_parameters: set[int] = set()
        plans = []
        total = 0
        for index in indices:
            sources = []
            seen: set[int] = set()
            for module in self.layers[index].modules():
                for name, parameter in module._parameters.items():
                    if parameter is None or id(parameter) in seen:
                        continue
                    if id(parameter) in seen_parameters:
                        raise ValueError("Trainable block streaming does not support parameters shared across blocks.")
                    if not parameter.is_floating_point():
                        raise TypeError(f"Streamed parameter {name} must be floating point.")
                    seen.add(id(parameter))
                    seen_parameters.add(id(parameter))
                    sources.append((module, name, parameter, parameter.detach()))
                for name, buffer in module._buffers.items():
                    if buffer is None or id(buffer) in seen:
                        continue
                    seen.add(id(buffer))
                    sources.append((module, name, None, buffer.detach()))
            views, converted, offset = [], [], 0
            for _, _, parameter, tensor in sources:
                dtype = self.master_dtype if parameter is not None and self.master_dtype is not None else tensor.dtype
                source = tensor.to(device="cpu", dtype=dtype).contiguous()
                offset = _align(offset)
                nbytes = source.numel() * source.element_size()
                views.append(_View(offset, nbytes, source.shape, source.dtype))
                converted.append(source)
                offset += nbytes
            plans.append((index, sources, views, converted, _align(offset), total))
            total += _align(offset)
        arena = PinnedArena(total)
        for index, sources, views, converted, nbytes, start in plans:
            master = arena.tensor[start : start + nbytes]
            bindings = []
            for (module, name, parameter, _), view, source in zip(sources, views, converted):
                target = _typed(master, view)
                target.copy_(source)
                bindings.append(_Binding(module, name, parameter, view))
                if parameter is not None:
                    parameter.data = target
                else:
                    module._buffers[name] = target
            block = _Block(index, arena.address + start, master, nbytes, bindings)
            self._blocks[index] = block
            expected = set()
            for binding in bindings:
                parameter = binding.parameter
                if parameter is not None and parameter.requires_grad:
                    expected.add(id(parameter))
                    self._parameter_block[id(parameter)] = index
                    self._parameter_name[id(parameter)] = f"layers.{index}.{binding.local_name}"
            self._expected_updates[index] = expected

    @staticmethod
    def _bind(block: _Block, flat: torch.Tensor) -> list[torch.Tensor]:
        views = [_typed(flat, binding.view) for binding in block.bindings]
        for binding, view in zip(block.bindings, views):
            if binding.parameter is not None:
                binding.parameter.data = view
            else:
                binding.module._buffers[binding.local_name] = view
        return views

    # ------------------------------------------------------------------ introspection
    @property
    def closed(self) -> bool:
        return self._closed

    @property
    def requires_reload(self) -> bool:
        return self._requires_reload

    @property
    def resident_block_indices(self) -> tuple[int, ...]:
        return tuple(sorted(slot.index for slot in self._slots if slot.index is not None))

    def owned_cuda_buffers(self) -> tuple[torch.Tensor, ...]:
        return tuple(slot.buffer for slot in self._slots if slot.buffer.device.type == "cuda")

    def stats(self) -> dict:
        out = _native.MoStreamerStats()
        _native.check("mo_streamer_get_stats", self._lib.mo_streamer_get_stats(self._handle, ctypes.byref(out)))
        return out.as_dict()

    def reset_stats(self) -> None:
        _native.check("mo_streamer_reset_stats", self._lib.mo_streamer_reset_stats(self._handle))

    # ------------------------------------------------------------------ ring
    def _slot_of(self, index: int) -> _Slot | None:
        return next((slot for slot in self._slots if slot.index == index), None)

    def _pick(self, protected: frozenset[int]) -> _Slot:
        for slot in self._slots:
            if slot.index is None:
                return slot
        for slot in self._slots:
            if slot.index not in protected:
                return slot
        raise RuntimeError("Both trainable staging slots are protected by active blocks.")

    def _release(self, slot: _Slot) -> None:
        stream = torch.cuda.current_stream(self.device).cuda_stream
        _native.check("mo_streamer_release", self._lib.mo_streamer_release(self._handle, slot.native, stream))

    def _evict(self, slot: _Slot) -> None:
        if slot.index is None:
            return
        block = self._blocks[slot.index]
        if slot.dirty:
            _native.check(
                "mo_streamer_writeback",
                self._lib.mo_streamer_writeback(self._handle, slot.native, block.host, slot.buffer.data_ptr(),
                                                block.nbytes),
            )
            self.d2h_copy_count += 1
        self._bind(block, block.master)
        slot.index = None
        slot.dirty = False
        slot.views.clear()

    def _stage(self, index: int, protected: frozenset[int]) -> _Slot:
        slot = self._slot_of(index)
        if slot is not None:
            return slot
        slot = self._pick(protected)
        self._evict(slot)
        block = self._blocks[index]
        _native.check(
            "mo_streamer_fill",
            self._lib.mo_streamer_fill(self._handle, slot.native, slot.buffer.data_ptr(), block.host, block.nbytes),
        )
        slot.index = index
        slot.dirty = False
        slot.views = self._bind(block, slot.buffer[: block.nbytes])
        self.h2d_copy_count += 1
        self.peak_resident_blocks = max(self.peak_resident_blocks, len(self.resident_block_indices))
        return slot

    def _finish_previous_backward(self) -> None:
        if self._last_backward_index is None:
            return
        index = self._last_backward_index
        slot = self._slot_of(index)
        if slot is None:
            raise RuntimeError("A trainable block was evicted before its backward completed.")
        # the block's backward and its optimizer hooks are enqueued: the slot may be written
        # back / refilled once the GPU gets here
        self._release(slot)
        if self._step_enabled:
            failed = self._expected_updates[index] & self._failed.keys()
            if failed:
                names = sorted(self._failed[p] for p in failed)
                slot.dirty = False
                self._last_backward_index = None
                self._requires_reload = True
                raise RuntimeError(f"Trainable block {index} had a failed fused optimizer update for {names[:3]}.")
            missing = self._expected_updates[index] - self._updated
            if self._require_all_updates and missing:
                names = sorted(self._parameter_name[p] for p in missing)
                slot.dirty = False
                self._last_backward_index = None
                self._requires_reload = True
                raise RuntimeError(
                    f"Trainable block {index} backward completed before all parameter updates; missing {names[:3]}."
                )
            slot.dirty = bool(self._expected_updates[index] & self._updated)
        else:
            slot.dirty = False
        self._last_backward_index = None

    # ------------------------------------------------------------------ optimizer protocol
    def set_step_enabled(self, enabled: bool) -> None:
        """Select whether this backward is the optimizer-update boundary."""

        if self._last_backward_index is not None:
            raise RuntimeError("Cannot change the trainable streamer boundary during backward.")
        if self._requires_reload:
            raise RuntimeError("Trainable block streamer requires checkpoint reload after a failed step.")
        self._step_enabled = bool(enabled)
        self._updated.clear()
        self._failed.clear()

    def set_require_all_updates(self, required: bool) -> None:
        if self._last_backward_index is not None:
            raise RuntimeError("Cannot change update requirements during backward.")
        self._require_all_updates = bool(required)

    def mark_updated(self, parameter: nn.Parameter) -> None:
        """A fused optimizer hook finished updating ``parameter`` in place."""

        if self._step_enabled and id(parameter) in self._parameter_block:
            self._updated.add(id(parameter))

    def mark_failed(self, parameter: nn.Parameter) -> None:
        """A fused optimizer hook failed for ``parameter``: its block must not be written back."""

        if self._step_enabled and id(parameter) in self._parameter_block:
            self._failed[id(parameter)] = self._parameter_name[id(parameter)]

    def mark_reloaded(self) -> None:
        if self._last_backward_index is not None or self.resident_block_indices:
            raise RuntimeError("Commit the trainable block streamer before marking it reloaded.")
        self._requires_reload = False
        self._updated.clear()
        self._failed.clear()

    # ------------------------------------------------------------------ execution
    def _run(self, index, inputs, forward_prefetch, backward_prefetch):
        if self._closed:
            raise RuntimeError("Trainable block streamer is closed.")
        recomputing = self._recomputing.get()
        with self._lock:
            if recomputing or self._last_backward_index is not None:
                # in recomputation: the previous block's backward is complete; in a new forward:
                # the previous backward call has returned, so its optimizer hooks have run
                self._finish_previous_backward()
            prefetch = backward_prefetch if recomputing else forward_prefetch
            protected = frozenset(i for i in (index, prefetch) if i is not None)
            slot = self._stage(index, protected)
            if prefetch is not None:
                if prefetch not in self._blocks:
                    raise ValueError(f"Prefetch block {prefetch} is not streamed.")
                self._stage(prefetch, protected)
            stream = torch.cuda.current_stream(self.device).cuda_stream
            _native.check("mo_streamer_acquire", self._lib.mo_streamer_acquire(self._handle, slot.native, stream))
        try:
            output = self.layers[index](*inputs)
        except BaseException as error:
            with self._lock:
                if recomputing and _is_recompute_early_stop(error):
                    self._last_backward_index = index
                else:
                    self._release(slot)
                    slot.dirty = recomputing
            raise
        with self._lock:
            if recomputing:
                self._last_backward_index = index
            else:
                self._release(slot)
        return output

    def _checkpoint_contexts(self):
        return nullcontext(), self._recompute_scope

    def block(self, index: int, *inputs: torch.Tensor, forward_prefetch: int | None,
              backward_prefetch: int | None, checkpoint_block: bool) -> torch.Tensor:
        """Run one streamed block (the block-manager contract of the reference model)."""

        if index not in self._blocks:
            raise ValueError(f"Block {index} is not configured for trainable streaming.")
        if not checkpoint_block:
            return self._run(index, inputs, forward_prefetch, backward_prefetch)
        aliases = tuple(t.view_as(t) if t.requires_grad else t for t in inputs)

        def run(*arguments: torch.Tensor) -> torch.Tensor:
            return self._run(index, arguments, forward_prefetch, backward_prefetch)

        return checkpoint(run, *aliases, use_reentrant=False, context_fn=self._checkpoint_contexts)

    def finish_backward(self) -> None:
        """Commit the last dirty block after all optimizer hooks have run."""

        if self._closed:
            raise RuntimeError("Trainable block streamer is closed.")
        self.commit()

    def commit(self) -> None:
        """Write back dirty slots and park every streamed parameter on its CPU master."""

        if self._closed:
            return
        with self._lock:
            self._finish_previous_backward()
            for slot in self._slots:
                self._evict(slot)
            torch.cuda.synchronize(self.device)
            _native.check("mo_streamer_synchronize", self._lib.mo_streamer_synchronize(self._handle))
            self._updated.clear()
            self._failed.clear()

    drain = commit

    def close(self) -> None:
        """Commit authoritative weights and release the staging slots."""

        if self._closed:
            return
        self.commit()
        _native.check("mo_streamer_destroy", self._lib.mo_streamer_destroy(self._handle))
        self._handle = ctypes.c_void_p()
        for slot in self._slots:
            slot.buffer = torch.empty(0, dtype=torch.uint8, device="cpu")
        self._closed = True
