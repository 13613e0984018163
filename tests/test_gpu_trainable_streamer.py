"""Bidirectional (trainable) block streaming on the GPU: full-parameter training through the
two-slot ring matches a resident model.

Restates the scenarios of the reference's training/tests/test_trainable_offload.py with a
minimal in-backward optimizer instead of FusedAdafactor: every parameter is updated by its
post-accumulate-grad hook, which reports the update to the streamer (``mark_updated``), and
gradients are stashed on the host while stepping is disabled (accumulation backwards). The ring
must write each updated block back to its pinned master before reusing the slot, keep
accumulation backwards clean (no write-back), and refuse to write back a block whose update
is missing.
"""

from __future__ import annotations

import copy

import pytest
import torch

from moss_offload import dit
from moss_offload.memory import place_model
from moss_offload.trainable_offload import TrainableBlockStreamer

from gpu_util import requires_gpu

pytestmark = requires_gpu


class _FusedSGD:
    """Plain SGD applied inside backward by post-accumulate-grad hooks."""

    def __init__(self, parameters, lr: float) -> None:
        self.parameters = [p for p in parameters if p.requires_grad]
        self.lr = lr
        self.step_enabled = True
        self.stash: dict[int, torch.Tensor] = {}
        self.streamer = None
        self.skip: set[int] = set()

    def install_hooks(self, streamer=None) -> "_FusedSGD":
        self.streamer = streamer
        for p in self.parameters:
            p.register_post_accumulate_grad_hook(self._hook)
        return self

    def set_step_enabled(self, enabled: bool) -> None:
        self.step_enabled = enabled
        if self.streamer is not None:
            self.streamer.set_step_enabled(enabled)

    def _hook(self, p: torch.Tensor) -> None:
        grad = p.grad
        p.grad = None
        if not self.step_enabled:
            host = grad.detach().to("cpu")
            previous = self.stash.get(id(p))
            self.stash[id(p)] = host if previous is None else previous + host
            return
        previous = self.stash.pop(id(p), None)
        if previous is not None:
            grad = grad + previous.to(grad.device)
        if id(p) in self.skip:
            return
        with torch.no_grad():
            p.add_(grad.to(p.dtype), alpha=-self.lr)
        if self.streamer is not None:
            self.streamer.mark_updated(p)


def _tiny():
    torch.manual_seed(41)
    model = dit.MOSSImageTransformer(
        dim=32, ffn_dim=64, num_heads=4, num_layers=4, text_dim=16, freq_dim=8, latent_channels=4,
        gradient_checkpointing=True,
    )
    dit.init_weights(model, std=0.05)
    return model.train()


def _batch(device, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(1, 4, 3, 5, generator=g).to(device), torch.tensor([300.0 + seed], device=device),
            torch.randn(1, 4, 16, generator=g).to(device))


def _backward(model, batch):
    latent, t, context = batch
    model(latent, t, context).float().square().mean().backward()


def _params(model):
    return {n: p.detach().to("cpu").clone() for n, p in model.named_parameters()}


def _close(a, b, atol=2e-5, rtol=2e-3):
    assert a.keys() == b.keys()
    for name in a:
        torch.testing.assert_close(a[name], b[name], atol=atol, rtol=rtol, msg=lambda m: f"{name}: {m}")


def test_full_ring_matches_resident_and_updates_every_parameter() -> None:
    device = torch.device("cuda", 0)
    resident, streamed = _tiny(), None
    streamed = copy.deepcopy(resident)
    initial = _params(resident)
    place_model(resident, device, 0)
    place_model(streamed, device, 4, block_swap_mode="async_full")
    manager = streamed.block_swap_manager
    assert isinstance(manager, TrainableBlockStreamer)
    for layer in streamed.layers:
        assert all(p.device.type == "cpu" and p.is_pinned() for p in layer.parameters())
    opt_r = _FusedSGD(resident.parameters(), 5e-2).install_hooks()
    opt_s = _FusedSGD(streamed.parameters(), 5e-2).install_hooks(manager)
    for step in range(3):
        batch = _batch(device, step)
        _backward(resident, batch)
        _backward(streamed, batch)
        manager.finish_backward()
        assert manager.resident_block_indices == ()
    final = _params(streamed)
    _close(final, _params(resident))
    assert all(not torch.equal(final[n], initial[n]) for n in final if n.startswith("layers."))
    assert manager.d2h_copy_count > 0 and manager.h2d_copy_count > manager.d2h_copy_count
    stats = manager.stats()
    assert stats["writebacks"] == manager.d2h_copy_count and stats["fills"] == manager.h2d_copy_count
    assert stats["copy_failures"] == 0
    assert 1 <= manager.peak_resident_blocks <= 2


def test_accumulation_backward_stays_clean_until_enabled_boundary() -> None:
    device = torch.device("cuda", 0)
    resident = _tiny()
    streamed = copy.deepcopy(resident)
    place_model(resident, device, 0)
    place_model(streamed, device, 4, block_swap_mode="async_full")
    manager = streamed.block_swap_manager
    opt_r = _FusedSGD(resident.parameters(), 5e-2).install_hooks()
    opt_s = _FusedSGD(streamed.parameters(), 5e-2).install_hooks(manager)
    before = _params(streamed)
    for opt in (opt_r, opt_s):
        opt.set_step_enabled(False)
    _backward(resident, _batch(device, 7))
    _backward(streamed, _batch(device, 7))
    manager.finish_backward()
    assert manager.d2h_copy_count == 0
    assert all(torch.equal(v, before[n]) for n, v in _params(streamed).items())
    for opt in (opt_r, opt_s):
        opt.set_step_enabled(True)
    _backward(resident, _batch(device, 8))
    _backward(streamed, _batch(device, 8))
    manager.finish_backward()
    assert manager.d2h_copy_count > 0
    _close(_params(streamed), _params(resident))


def test_dirty_eviction_rejects_missing_streamed_parameter_updates() -> None:
    device = torch.device("cuda", 0)
    model = _tiny()
    place_model(model, device, 4, block_swap_mode="async_full")
    manager = model.block_swap_manager
    opt = _FusedSGD(model.parameters(), 5e-2).install_hooks(manager)
    opt.skip.add(id(model.layers[3].proj["q"].weight))
    with pytest.raises(RuntimeError, match="before all parameter updates"):
        _backward(model, _batch(device, 9))
    assert manager.requires_reload
    with pytest.raises(RuntimeError, match="requires checkpoint reload"):
        manager.set_step_enabled(True)


def test_commit_parks_masters_and_cpu_placement_closes_the_ring() -> None:
    device = torch.device("cuda", 0)
    model = _tiny()
    place_model(model, device, 2, block_swap_mode="async_full")
    manager = model.block_swap_manager
    opt = _FusedSGD(model.parameters(), 5e-2).install_hooks(manager)
    for layer in model.layers[:2]:
        assert all(p.device.type == "cuda" for p in layer.parameters())
    _backward(model, _batch(device, 10))
    manager.commit()
    assert manager.resident_block_indices == ()
    for layer in model.layers[2:]:
        assert all(p.device.type == "cpu" and p.is_pinned() for p in layer.parameters())
    masters = {n: p.detach().clone() for n, p in model.layers[2:].named_parameters()}
    place_model(model, torch.device("cpu"), 0)
    assert manager.closed and model.block_swap_manager is None
    assert all(p.device.type == "cpu" for p in model.parameters())
    for n, p in model.layers[2:].named_parameters():
        assert torch.equal(p, masters[n])
