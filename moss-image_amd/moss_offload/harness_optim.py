"""Harness optimizer that drives host gradient accumulation the way MOSS-Image's
``FusedAdafactor`` does in its CPU accumulation mode, with a plain SGD update in place of the
Adafactor math (which is not part of the offload path).

Control flow restated from ``training/fused_adafactor.py``:

- post-accumulate-grad hooks (``install_hooks``, ``:456-513``). While the step is disabled
  (an early micro-batch), a hook stashes the gradient on the host and releases ``parameter.grad``
  (``_stash_gradient_on_host``, ``:327-355``). While it is enabled (the boundary micro-batch),
  a hook applies the update (``step_parameter``, ``:456-471``).
- the update uses the current gradient plus the popped host sum, ``current.float() +
  previous.to(device)`` (``_take_accumulated_gradient``, ``:357-369``); with the engine the sum
  comes from ``pop_to_device`` (prefetched over SDMA) instead of a blocking copy.
- ``finish_backward`` (``:515-524``) updates the parameters that only have a host sum.

Stashes:

- ``"engine"``: :class:`moss_offload.host_gradients.HostGradientAccumulator`.
- ``"device"``: none; early gradients stay in ``parameter.grad`` on the device (the reference's
  default ``gradient_accumulation_device="device"``), the point of comparison.
- ``"reference"``: the reference's own, an fp32 pinned ``torch.empty`` per stash, a blocking
  ``copy_`` and a host ``add_`` into a plain dict (``:336-352``). It is the baseline of the bench's
  host-gradient leg and the oracle of the GPU tests.
"""

from __future__ import annotations

from collections.abc import Iterable, MutableMapping

import torch
from torch import nn

from .host_gradients import HostGradientAccumulator


class HostModeSGD:
    """In-backward SGD with host fp32 gradient accumulation across micro-batches."""

    def __init__(self, parameters: Iterable[nn.Parameter], lr: float, *, stash: str = "engine",
                 accumulator: MutableMapping | None = None) -> None:
        if stash not in ("engine", "reference", "device"):
            raise ValueError("stash must be 'engine', 'reference' or 'device'")
        self.lr = float(lr)
        self.stash_kind = stash
        self.parameters = [p for p in parameters if p.requires_grad]
        if accumulator is None:
            accumulator = HostGradientAccumulator() if stash == "engine" else {}
        self.host_gradients = accumulator
        self.step_enabled = True
        self.updated: set[int] = set()
        self._handles = [p.register_post_accumulate_grad_hook(self._hook) for p in self.parameters]

    def set_step_enabled(self, enabled: bool) -> None:
        self.step_enabled = bool(enabled)

    def _hook(self, parameter: nn.Parameter) -> None:
        if self.step_enabled:
            self.step_parameter(parameter)
        elif self.stash_kind != "device":
            self.stash(parameter)

    @torch.no_grad()
    def stash(self, parameter: nn.Parameter) -> None:
        gradient = parameter.grad
        if gradient is None:
            return
        key = id(parameter)
        if self.stash_kind == "engine":
            self.host_gradients.accumulate(key, gradient)
        else:
            if gradient.device.type == "cuda":
                host = torch.empty(gradient.shape, dtype=torch.float32, device="cpu", pin_memory=True)
                host.copy_(gradient.detach(), non_blocking=False)
            else:
                host = gradient.detach().to(device="cpu", dtype=torch.float32).clone()
            accumulated = self.host_gradients.get(key)
            if accumulated is None:
                self.host_gradients[key] = host
            else:
                accumulated.add_(host)
        parameter.grad = None

    @torch.no_grad()
    def take(self, parameter: nn.Parameter) -> torch.Tensor | None:
        current = parameter.grad
        pop_to_device = getattr(self.host_gradients, "pop_to_device", None)
        if pop_to_device is not None:  # the engine: prefetched by SDMA, no blocking copy
            previous = pop_to_device(id(parameter), None if current is None else current.device)
        else:
            previous = self.host_gradients.pop(id(parameter), None)
        if previous is None:
            return current
        if current is None:
            return previous
        return current.detach().float().add(previous.to(device=current.device, non_blocking=False))

    @torch.no_grad()
    def step_parameter(self, parameter: nn.Parameter) -> bool:
        gradient = self.take(parameter)
        if gradient is None:
            return False
        gradient = gradient.to(device=parameter.device, dtype=torch.float32)
        updated = parameter.detach().float().add_(gradient, alpha=-self.lr)
        parameter.copy_(updated.to(parameter.dtype))
        parameter.grad = None
        self.updated.add(id(parameter))
        return True

    def finish_backward(self) -> None:
        for parameter in self.parameters:
            if id(parameter) in self.host_gradients:
                self.step_parameter(parameter)

    def zero_grad(self, set_to_none: bool = True) -> None:
        for parameter in self.parameters:
            parameter.grad = None

    def close(self) -> None:
        for handle in self._handles:
            handle.remove()
        self._handles.clear()
        close = getattr(self.host_gradients, "close", None)
        if close is not None:
            close()
