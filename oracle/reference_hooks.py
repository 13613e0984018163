"""Restatement of the reference hook algorithm (TEST INFRASTRUCTURE ONLY; see oracle/__init__).

Every function cites the lines of RyukoMatoiFan/MOSS-Image ``training/activation_offload.py``
it follows. Two modes:

- ``activation_cpu_offload(model, enabled, device)`` behaves like the reference: on a
  CUDA/HIP device each offloadable save becomes a pinned CPU tensor filled by
  ``copy_(non_blocking=True)`` on the current stream plus an event; unpack waits for the event
  and restores with ``_restore_layout``. On CPU devices it is a no-op (:92-93).
- ``emulated_offload(model)`` runs the same pack/unpack decisions on CPU tensors with a CPU
  payload (a dense copy), so the plumbing can be checked without a GPU.

Parity status: ``offload_view`` and ``restore_layout`` are pinned by the reference's own
known-answer tests (tests/golden/layout_kats.json) and by brute-force element-offset checks
(oracle/layout.py). The hook pair is pinned by the identity invariant: restored tensors are
bitwise equal to the saved ones, and a model step with hooks is bitwise equal to one without.
"""

from __future__ import annotations

from contextlib import nullcontext
from dataclasses import dataclass, field

import torch
from torch import nn


@dataclass
class OffloadedTensor:
    """Reference ``_OffloadedTensor`` (:17-24)."""

    cpu: torch.Tensor
    device: torch.device
    ready: object
    shape: tuple
    stride: tuple
    payload_shape: tuple


def storage_key(tensor: torch.Tensor):
    """Reference ``_storage_key`` (:27-29)."""

    return tensor.device.type, tensor.device.index, tensor.untyped_storage().data_ptr()


def offload_view(tensor: torch.Tensor):
    """Reference ``_offload_view`` (:32-61), restated step by step."""

    shape = list(tensor.shape)
    source = tensor
    strides = tensor.stride()
    for dim in range(tensor.dim()):  # :42-47
        if strides[dim] < 0:
            return None
        if strides[dim] == 0 and shape[dim] > 1:
            source = source.narrow(dim, 0, 1)
            shape[dim] = 1
    extent = 1  # :51-60
    for stride, size in sorted((strides[d], shape[d]) for d in range(tensor.dim()) if shape[d] > 1):
        if stride < extent:
            return None
        extent += (size - 1) * stride
    return source, tuple(shape)


def restore_layout(payload, device, shape, stride, payload_shape, *, non_blocking):
    """Reference ``_restore_layout`` (:64-77)."""

    restored = torch.empty_strided(payload_shape, stride, dtype=payload.dtype, device=device)
    restored.copy_(payload, non_blocking=non_blocking)
    return restored.as_strided(shape, stride)


def _resident_storages(model: nn.Module, device_type: str):
    # :95-99
    return {
        storage_key(t)
        for t in (*model.parameters(), *model.buffers())
        if t.device.type == device_type and t.untyped_storage().nbytes()
    }


def _weight_backed(model, resident, tensor, device_type):
    # :101-114
    key = storage_key(tensor)
    if key in resident:
        return True
    manager = getattr(model, "block_swap_manager", None)
    owned = getattr(manager, "owned_cuda_buffers", None)
    if not callable(owned):
        return False
    return any(b.device.type == device_type and storage_key(b) == key for b in owned())


@dataclass
class Recorder:
    """Optional observer of the hook traffic (what was offloaded and what came back)."""

    packed: list = field(default_factory=list)  # (original tensor, payload) per offloaded save
    restored: list = field(default_factory=list)  # restored tensors, in unpack order
    resident: int = 0

    @property
    def payload_bytes(self) -> int:
        return sum(p.numel() * p.element_size() for _, p in self.packed)


def activation_cpu_offload(model: nn.Module, enabled: bool, device: torch.device, recorder: Recorder | None = None):
    """Reference ``activation_cpu_offload`` (:80-149)."""

    if not enabled or device.type != "cuda" or not torch.is_grad_enabled():  # :92-93
        return nullcontext()
    resident = _resident_storages(model, "cuda")

    def pack(tensor):  # :116-134
        if tensor.device.type != "cuda" or _weight_backed(model, resident, tensor, "cuda"):
            if recorder is not None:
                recorder.resident += 1
            return tensor
        view = offload_view(tensor)
        if view is None:
            if recorder is not None:
                recorder.resident += 1
            return tensor
        source, payload_shape = view
        cpu = torch.empty(payload_shape, dtype=tensor.dtype, device="cpu", pin_memory=True)
        cpu.copy_(source, non_blocking=True)
        ready = torch.cuda.Event()
        ready.record(torch.cuda.current_stream(tensor.device))
        if recorder is not None:
            recorder.packed.append((tensor, cpu))
        return OffloadedTensor(cpu, tensor.device, ready, tuple(tensor.shape), tuple(tensor.stride()), payload_shape)

    def unpack(saved):  # :136-147
        if isinstance(saved, torch.Tensor):
            return saved
        torch.cuda.current_stream(saved.device).wait_event(saved.ready)
        out = restore_layout(saved.cpu, saved.device, saved.shape, saved.stride, saved.payload_shape, non_blocking=True)
        if recorder is not None:
            recorder.restored.append(out)
        return out

    return torch.autograd.graph.saved_tensors_hooks(pack, unpack)


def emulated_offload(model: nn.Module, recorder: Recorder | None = None):
    """The reference pack/unpack decisions applied to CPU tensors with CPU payloads.

    Same steps as :116-147 with ``device.type == "cpu"`` standing in for CUDA and a plain
    dense CPU tensor standing in for the pinned buffer (no event: CPU copies are synchronous).
    """

    resident = _resident_storages(model, "cpu")

    def pack(tensor):
        if tensor.device.type != "cpu" or _weight_backed(model, resident, tensor, "cpu"):
            if recorder is not None:
                recorder.resident += 1
            return tensor
        view = offload_view(tensor)
        if view is None:
            if recorder is not None:
                recorder.resident += 1
            return tensor
        source, payload_shape = view
        payload = torch.empty(payload_shape, dtype=tensor.dtype)
        payload.copy_(source)
        if recorder is not None:
            recorder.packed.append((tensor, payload))
        return OffloadedTensor(payload, tensor.device, None, tuple(tensor.shape), tuple(tensor.stride()), payload_shape)

    def unpack(saved):
        if isinstance(saved, torch.Tensor):
            return saved
        out = restore_layout(saved.cpu, saved.device, saved.shape, saved.stride, saved.payload_shape, non_blocking=False)
        if recorder is not None:
            recorder.restored.append(out)
        return out

    return torch.autograd.graph.saved_tensors_hooks(pack, unpack)


def bits(tensor: torch.Tensor) -> torch.Tensor:
    """Integer view of a tensor's logical elements, in logical order (bitwise comparison:
    -0.0 != +0.0, a NaN equals a NaN of the same payload only, and a bool is its stored byte)."""

    width = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[tensor.element_size()]
    return tensor.contiguous().view(width)


def bitwise_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Same shape, dtype and bits of every logical element."""

    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    return torch.equal(bits(a.detach().cpu()), bits(b.detach().cpu()))
