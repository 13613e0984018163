"""Saved-tensor manifest: what the offload hook receives, recorded at run time.

A ``saved_tensors_hooks`` probe (the instrument the reference's own tests use to count saves,
``training/tests/test_quantization.py:19-31``) that records, for every pack call, the shape,
stride, dtype, storage identity and version, whether the reference rules would keep it
resident (weight-backed, non-CUDA, or not offloadable, ``activation_offload.py:101-121``),
its payload bytes after narrowing, and which earlier save it duplicates: same storage, dtype
and version, and the same payload bytes (any view of them, as the engine's hook dedupes), or,
for a save that stays resident, the same view. The probe returns tensors unchanged, so the forward and
backward it observes are exactly the un-hooked ones.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import nn

from .activation_offload import _offload_view, _payload_key, _storage_key


@dataclass
class SavedRecord:
    index: int
    shape: tuple
    stride: tuple
    dtype: torch.dtype
    device: str
    storage: int
    offset: int
    version: int
    payload_shape: tuple | None
    payload_bytes: int
    resident: str  # "" (offloaded), "weight", "device", "layout"
    dup_of: int | None


class ManifestRecorder:
    """Context manager recording every save of the enclosed autograd recording."""

    def __init__(self, model: nn.Module | None = None, device_type: str = "cuda") -> None:
        self.device_type = device_type
        self.records: list[SavedRecord] = []
        self._resident = set()
        if model is not None:
            self._resident = {
                _storage_key(t) for t in (*model.parameters(), *model.buffers()) if t.untyped_storage().nbytes()
            }
        self._seen: dict[tuple, int] = {}
        self._hooks = torch.autograd.graph.saved_tensors_hooks(self._pack, lambda t: t)

    def __enter__(self):
        self._hooks.__enter__()
        return self

    def __exit__(self, *exc):
        return self._hooks.__exit__(*exc)

    def _pack(self, tensor: torch.Tensor) -> torch.Tensor:
        resident = ""
        payload_shape = None
        payload_bytes = 0
        layout_key = (tensor.storage_offset(), tuple(tensor.shape), tuple(tensor.stride()))
        if tensor.device.type != self.device_type:
            resident = "device"
        elif _storage_key(tensor) in self._resident:
            resident = "weight"
        else:
            view = _offload_view(tensor)
            if view is None:
                resident = "layout"
            else:
                payload_shape = view[1]
                layout_key = _payload_key(view[0])
                numel = 1
                for size in payload_shape:
                    numel *= size
                payload_bytes = numel * tensor.element_size()
        key = (tensor.untyped_storage().data_ptr(), layout_key, tensor.dtype, tensor._version)
        dup_of = self._seen.get(key)
        index = len(self.records)
        if dup_of is None:
            self._seen[key] = index
        self.records.append(
            SavedRecord(
                index,
                tuple(tensor.shape),
                tuple(tensor.stride()),
                tensor.dtype,
                tensor.device.type,
                key[0],
                tensor.storage_offset(),
                tensor._version,
                payload_shape,
                payload_bytes,
                resident,
                dup_of,
            )
        )
        # A detached alias, not the tensor itself: a node that saves its own output would
        # otherwise hold that output, whose grad_fn holds the node, a cycle through C++ that
        # the collector cannot break (the whole graph would outlive the forward).
        return tensor.detach()

    # summaries -------------------------------------------------------------------------------
    def offloaded(self) -> list[SavedRecord]:
        return [r for r in self.records if not r.resident]

    def payload_bytes(self, unique: bool = True) -> int:
        """Bytes the hooks move: each offloaded save once (unique) or as often as saved."""

        return sum(r.payload_bytes for r in self.offloaded() if not unique or r.dup_of is None)

    def table(self) -> list[dict]:
        return [
            {
                "index": r.index,
                "shape": list(r.shape),
                "stride": list(r.stride),
                "dtype": str(r.dtype).replace("torch.", ""),
                "resident": r.resident,
                "payload_bytes": r.payload_bytes,
                "dup_of": r.dup_of,
            }
            for r in self.records
        ]
