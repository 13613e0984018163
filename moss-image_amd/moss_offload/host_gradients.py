"""Host fp32 gradient accumulation without a blocking copy: drop-in for the CPU mode of
MOSS-Image's ``FusedAdafactor`` (``training/fused_adafactor.py:327-369``).

The reference keeps ``self._host_gradients: dict[int, torch.Tensor]``. For a device gradient,
``_stash_gradient_on_host`` allocates an fp32 pinned tensor, copies the gradient into it with a
blocking ``copy_`` and adds it into the parameter's entry on the host (``:336-352``).
``_take_accumulated_gradient`` pops the entry and adds it to the current gradient on the device
(``:357-369``).

:class:`HostGradientAccumulator` is that mapping with one more method,
:meth:`~HostGradientAccumulator.accumulate`, which replaces the copy and the add. The gradient
is copied into a device staging slot on the current stream, and the call returns, so the caller
may release ``parameter.grad`` at once as the reference does. An SDMA engine then moves the slot
to pinned host memory, and a native worker adds it into the entry's fp32 buffer in call order
(``csrc/mo_gradacc.cpp``). Reading an entry (``acc[key]``, ``pop``, ``get``, ``values()``)
waits for that entry's pending additions only. ``key in acc``, ``len(acc)`` and iteration never
wait.

The additions are the reference's: the first contribution of a step is the gradient converted to
fp32, and every later one is one IEEE fp32 add per element, in call order, so the entries are
bitwise the reference's. The link carries the gradient in its own dtype (bf16: half the bytes of
the reference, which converts on the device before its copy). CPU gradients take the reference's
own path (``gradient.to(cpu, fp32).clone()`` then ``add_``).

An entry's fp32 buffer is pinned, allocated at the key's first use and reused by later steps:
a tensor read from the mapping stays valid until the next ``accumulate`` into the same key.

:meth:`~HostGradientAccumulator.pop_to_device` replaces the take's blocking
``previous.to(device, non_blocking=False)`` (``:369``). It returns the entry as a device fp32
tensor and starts SDMA copies of the next entries, in the order of their first contribution,
while the caller computes. That is the order the next micro-batch's hooks ask for them. The
copies use a frozen-block streamer (``mo_streamer_*``): each is ordered after the compute
stream's work on the fresh device tensor, and the host waits for it only when it is popped.
"""

from __future__ import annotations

import ctypes
import threading
from collections.abc import Hashable, Iterator, MutableMapping

import torch

from . import _native
from .memory import PinnedArena

# the reference's value-kind codes (quant_kernels.py:280-287), include/moss_offload.h MO_DTYPE_*
_DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


class _Buffer:
    """One key's pinned fp32 accumulator."""

    def __init__(self, numel: int) -> None:
        self.arena = PinnedArena(numel * 4)
        self.flat = self.arena.tensor.view(torch.float32)[:numel]
        self.address = self.arena.address
        self.numel = numel


class HostGradientAccumulator(MutableMapping):
    """``key -> fp32 host tensor`` of the gradients accumulated in the current step."""

    def __init__(self, device: torch.device | str | int | None = None, *, slots: int = 4,
                 slot_bytes: int = 64 << 20, host_threads: int = 8, d2h_engine: int = 0,
                 prefetch: int = 4) -> None:
        if device is not None:
            device = torch.device("cuda", device) if isinstance(device, int) else torch.device(device)
            if device.type != "cuda":
                raise ValueError("HostGradientAccumulator stages device gradients; pass a CUDA (HIP) device or None.")
            device = torch.device("cuda", device.index or 0)
        self._device = device  # None: the device of the first device gradient
        self._config = (int(slots), int(slot_bytes), int(host_threads), int(d2h_engine))
        self._handle: ctypes.c_void_p | None = None
        self._lib = None
        self._buffers: dict[Hashable, _Buffer] = {}
        self._entries: dict[Hashable, torch.Tensor] = {}  # keys with a gradient this step
        self._device_keys: set[Hashable] = set()  # entries filled by the native path
        self._lock = threading.Lock()
        self._closed = False
        self._order: list[Hashable] = []  # keys of this step in the order of their first contribution
        self._pos: dict[Hashable, int] = {}  # key -> index in _order
        self._prefetch_slots = int(prefetch)
        self._streamer: ctypes.c_void_p | None = None
        self._free_slots: list[int] = []
        self._prefetched: dict[Hashable, tuple[int, torch.Tensor]] = {}

    # ---- native accumulator ------------------------------------------------------------------
    def _native(self, device: torch.device):
        if self._handle is not None:
            if device != self._device:
                raise RuntimeError(f"HostGradientAccumulator serves {self._device}; got a gradient on {device}.")
            return self._lib, self._handle
        if self._device is not None and device != self._device:
            raise RuntimeError(f"HostGradientAccumulator serves {self._device}; got a gradient on {device}.")
        lib = _native.load()
        handle = ctypes.c_void_p()
        slots, slot_bytes, threads, engine = self._config
        _native.check("mo_gradacc_create",
                      lib.mo_gradacc_create(device.index or 0, slots, slot_bytes, threads, engine, ctypes.byref(handle)))
        self._lib, self._handle, self._device = lib, handle, device
        return lib, handle

    def _wait(self, key: Hashable | None) -> None:
        if self._handle is None:
            return
        if key is not None:
            if key not in self._device_keys:
                return
            address = self._buffers[key].address
        else:
            address = 0
        _native.check("mo_gradacc_wait", self._lib.mo_gradacc_wait(self._handle, address))

    # ---- the stash --------------------------------------------------------------------------
    @torch.no_grad()
    def accumulate(self, key: Hashable, gradient: torch.Tensor) -> None:
        """Add ``gradient`` (any shape; fp16, bf16 or fp32) into ``key``'s fp32 entry.

        A device gradient returns as soon as it is copied into a staging slot on the current
        stream (the host waits only while every slot is in flight). Replaces the blocking copy and
        host add of ``FusedAdafactor._stash_gradient_on_host`` (fused_adafactor.py:336-352).
        """

        if self._closed:
            raise RuntimeError("HostGradientAccumulator is closed.")
        gradient = gradient.detach()
        with self._lock:
            if gradient.device.type != "cuda":
                host = gradient.to(device="cpu", dtype=torch.float32).clone()
                current = self._entries.get(key)
                if current is None:
                    self._entries[key] = host
                else:
                    self._wait(key)
                    current.add_(host.reshape(current.shape))
                return
            code = _DTYPE_CODES.get(gradient.dtype)
            if code is None:
                raise TypeError(f"HostGradientAccumulator takes fp16, bf16 or fp32 gradients, not {gradient.dtype}.")
            lib, handle = self._native(gradient.device)
            self._discard_prefetch(key)
            numel = gradient.numel()
            first = key not in self._entries
            if first:
                self._pos[key] = len(self._order)
                self._order.append(key)
            if not first and key not in self._device_keys:
                # a CPU-path or assigned entry: continue it in the native buffer
                self._adopt(key, numel)
            buffer = self._buffers.get(key)
            if buffer is None or buffer.numel != numel:
                if not first:
                    raise ValueError(f"gradient for {key!r} changed size within a step.")
                # a key's first contribution of a step has no pending additions
                buffer = self._buffers[key] = _Buffer(numel)
            source = gradient.contiguous()
            stream = torch.cuda.current_stream(gradient.device).cuda_stream
            _native.check("mo_gradacc_accumulate",
                          lib.mo_gradacc_accumulate(handle, buffer.address, int(first), source.data_ptr(), code, numel,
                                                    stream))
            self._entries[key] = buffer.flat.view(gradient.shape)
            self._device_keys.add(key)

    def _adopt(self, key: Hashable, numel: int) -> None:
        """Move a host-side entry into the key's native buffer so that device contributions
        continue it (keeps one fp32 sum per key whatever path produced each contribution)."""

        value = self._entries[key]
        if value.numel() != numel:
            raise ValueError(f"gradient for {key!r} changed size within a step.")
        buffer = self._buffers.get(key)
        if buffer is None or buffer.numel != numel:
            buffer = self._buffers[key] = _Buffer(numel)
        buffer.flat.copy_(value.reshape(-1))
        self._entries[key] = buffer.flat.view(value.shape)
        self._device_keys.add(key)

    # ---- the take on the device --------------------------------------------------------------
    def _h2d_streamer(self):
        if self._streamer is None:
            streamer = ctypes.c_void_p()
            _native.check("mo_streamer_create", self._lib.mo_streamer_create(
                self._device.index or 0, max(self._prefetch_slots, 1), 0, ctypes.byref(streamer)))
            self._streamer = streamer
            self._free_slots = list(range(max(self._prefetch_slots, 1)))
        return self._streamer

    def _issue(self, key: Hashable, stream: int) -> None:
        """Start the SDMA copy of ``key``'s completed sum into a fresh device tensor."""

        streamer = self._h2d_streamer()
        self._wait(key)
        value = self._entries[key]
        slot = self._free_slots.pop()
        tensor = torch.empty(value.shape, dtype=torch.float32, device=self._device)
        # the fill waits for the compute stream to pass this point: the fresh tensor's memory
        # is no longer in use by earlier kernels
        _native.check("mo_streamer_release", self._lib.mo_streamer_release(streamer, slot, stream))
        _native.check("mo_streamer_fill", self._lib.mo_streamer_fill(
            streamer, slot, tensor.data_ptr(), self._buffers[key].address, value.numel() * 4))
        self._prefetched[key] = (slot, tensor)

    def _claim(self, key: Hashable, stream: int) -> torch.Tensor:
        slot, tensor = self._prefetched.pop(key)
        try:
            _native.check("mo_streamer_acquire", self._lib.mo_streamer_acquire(self._streamer, slot, stream))
        finally:
            self._free_slots.append(slot)
        return tensor

    def _discard_prefetch(self, key: Hashable) -> None:
        if key in self._prefetched:
            stream = torch.cuda.current_stream(self._device).cuda_stream
            self._claim(key, stream)

    def pop_to_device(self, key: Hashable, device: torch.device | str | None = None) -> torch.Tensor | None:
        """``pop(key)`` as an fp32 tensor on the device, or None without an entry.

        Waits for the key's own copy only (usually already done), then prefetches the entries
        that follow it in first-contribution order into free slots. A CPU-path entry is moved
        with a plain copy.
        """

        with self._lock:
            if key not in self._entries:
                return None
            if key not in self._device_keys or self._handle is None:
                # a CPU-path entry: moved only when a device is named (the reference keeps a
                # host-only sum on the host, fused_adafactor.py:365-366)
                value = self._entries.pop(key)
                self._end_of_step()
                return value if device is None else value.to(device=device, dtype=torch.float32, non_blocking=False)
            if device is not None and torch.device(device) != self._device:
                raise RuntimeError(f"HostGradientAccumulator serves {self._device}; asked for {device}.")
            stream = torch.cuda.current_stream(self._device).cuda_stream
            if key not in self._prefetched:
                self._h2d_streamer()
                if not self._free_slots:  # every slot holds a prefetch of another key: take one back
                    self._claim(next(reversed(self._prefetched)), stream)
                self._issue(key, stream)
            tensor = self._claim(key, stream)
            del self._entries[key]
            self._device_keys.discard(key)
            # the following keys, while the caller computes
            index = self._pos.pop(key, len(self._order)) + 1
            while self._free_slots and index < len(self._order):
                other = self._order[index]
                if other in self._device_keys and other not in self._prefetched:
                    self._issue(other, stream)
                index += 1
            self._end_of_step()
            return tensor

    def _end_of_step(self) -> None:
        if not self._entries:
            self._order.clear()
            self._pos.clear()

    # ---- the mapping ------------------------------------------------------------------------
    def __getitem__(self, key: Hashable) -> torch.Tensor:
        with self._lock:
            value = self._entries[key]
            self._wait(key)
            return value

    def __setitem__(self, key: Hashable, value: torch.Tensor) -> None:
        if not isinstance(value, torch.Tensor):
            raise TypeError("HostGradientAccumulator values are tensors.")
        with self._lock:
            self._wait(key)
            self._entries[key] = value
            self._device_keys.discard(key)

    def __delitem__(self, key: Hashable) -> None:
        with self._lock:
            if key not in self._entries:
                raise KeyError(key)
            self._wait(key)
            self._discard_prefetch(key)
            del self._entries[key]
            self._device_keys.discard(key)
            self._end_of_step()

    def __contains__(self, key: object) -> bool:
        return key in self._entries

    def __iter__(self) -> Iterator[Hashable]:
        return iter(list(self._entries))

    def __len__(self) -> int:
        return len(self._entries)

    def clear(self) -> None:
        with self._lock:
            self._wait(None)
            for key in list(self._prefetched):
                self._discard_prefetch(key)
            self._entries.clear()
            self._device_keys.clear()
            self._end_of_step()

    def synchronize(self) -> None:
        """Wait for every pending addition."""

        with self._lock:
            self._wait(None)

    def stats(self) -> dict:
        if self._handle is None:
            return {name: 0 for name, _ in _native.MoGradaccStats._fields_}
        out = _native.MoGradaccStats()
        _native.check("mo_gradacc_get_stats", self._lib.mo_gradacc_get_stats(self._handle, ctypes.byref(out)))
        return out.as_dict()

    def reset_stats(self) -> None:
        if self._handle is not None:
            _native.check("mo_gradacc_reset_stats", self._lib.mo_gradacc_reset_stats(self._handle))

    def trim(self) -> None:
        """Free the pinned buffers of keys without an entry this step."""

        with self._lock:
            for key in [k for k in self._buffers if k not in self._entries]:
                del self._buffers[key]

    def close(self) -> None:
        """Wait for pending additions, then free the native accumulator and the buffers."""

        with self._lock:
            if self._closed:
                return
            self._closed = True
            for key in list(self._prefetched):
                self._discard_prefetch(key)
            self._entries.clear()
            self._device_keys.clear()
            self._end_of_step()
            if self._streamer is not None:
                streamer, self._streamer = self._streamer, None
                _native.check("mo_streamer_destroy", self._lib.mo_streamer_destroy(streamer))
            if self._handle is not None:
                handle, self._handle = self._handle, None
                _native.check("mo_gradacc_destroy", self._lib.mo_gradacc_destroy(handle))
            self._buffers.clear()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass
